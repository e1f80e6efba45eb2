/*
 * bytes_amd C ABI: the MI355X (gfx950) decode-attention hot path of the
 * saifmb0/bytes KV-cache study.
 *
 * Conventions (every entry point):
 *  - Tensor arguments are device pointers; shapes are ints; strides are int64
 *    ELEMENT strides; the innermost (head-dim / packed) axis has unit stride
 *    and every row starts on a 16-byte boundary.
 *  - `stream` is a hipStream_t (0 = legacy default stream).  Launches are
 *    asynchronous; nothing here synchronises, allocates or copies to host, so
 *    every call can be captured in a hipGraph.
 *  - `workspace` is caller-owned device memory of at least the size returned
 *    by the matching *_workspace_size query.  It must be zero-filled once
 *    before first use; the kernels leave their counters at zero on exit.
 *    One workspace may serve the split-K decode entry points together
 *    (dense, KIVI, gather); bytes_topk needs a workspace of its own.  Calls
 *    that share a workspace must be ordered on one stream.
 *  - Return value: 0 on success, otherwise a hipError_t value
 *    (bytes_error_string() gives its text).  No C++ exception crosses the ABI.
 */
#ifndef BYTES_AMD_H_
#define BYTES_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version of this ABI (bumped on incompatible changes). */
int bytes_abi_version(void);

/* Text of a status code returned by any entry point. */
const char* bytes_error_string(int code);

/* Kernel timing hook (no counterpart in the reference; for benchmarks): while
 * set, every entry point of kernel family `family` records the hipEvent_t
 * `start` on its stream right before launching its main kernel and `stop`
 * right after it (top-k: around its whole launch sequence).  Families:
 * 1 dense/fp8 decode, 2 KIVI decode, 3 PQ decode, 4 gather attention,
 * 5 score pass, 6 Quest page bounds, 7 top-k.  family 0 clears the hook.
 * Process-wide; not for concurrent use from several threads. */
int bytes_set_kernel_events(int family, void* start, void* stop);

/* ---------------------------------------------------------------------------
 * Dense bf16 GQA decode attention.
 * Replaces src/attention_kernels.py:65-92 (`decode_attn_bf16`, kernel :8-63).
 *   q   [B, Hq, D] bf16 (strides q_sb, q_sh)
 *   k,v [B, Hk, S, D] bf16 (strides *_sb, *_sh, *_ss)
 *   out [B, Hq, D] bf16 (strides o_sb, o_sh)
 *   out[b,h] = softmax(scale * q[b,h] . k[b,h/G]^T) v[b,h/G],  G = Hq/Hk
 * D in {64, 128}.  chunk = split-K chunk in tokens (0 = automatic).
 * The reference applies no scale; pass scale = 1.0 for identical semantics.
 * ------------------------------------------------------------------------- */
int bytes_decode_attn_bf16_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk,
                                          size_t* bytes);
int bytes_decode_attn_bf16(const void* q, const void* k, const void* v, void* out,
                           int B, int Hq, int Hk, int S, int D,
                           int64_t q_sb, int64_t q_sh,
                           int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           int64_t v_sb, int64_t v_sh, int64_t v_ss,
                           int64_t o_sb, int64_t o_sh,
                           float scale, int chunk, void* workspace, size_t workspace_bytes,
                           void* stream);

/* No-allocation variant of bytes_decode_attn_bf16.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * allocation).  Same arguments and results as bytes_decode_attn_bf16 without
 * the workspace: the split-K partials go to a device-resident scratch array of
 * BYTES_NOALLOC_SCRATCH_BYTES per device, held until the process ends.
 * Returns hipErrorOutOfMemory when the call's partials
 * (bytes_decode_attn_bf16_workspace_size) exceed that size.  Calls that
 * overlap on one device share the scratch and race; order them on one stream. */
#define BYTES_NOALLOC_SCRATCH_BYTES (16u << 20)
int bytes_decode_attn_bf16_noalloc(const void* q, const void* k, const void* v, void* out,
                                   int B, int Hq, int Hk, int S, int D,
                                   int64_t q_sb, int64_t q_sh,
                                   int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                   int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                   int64_t o_sb, int64_t o_sh,
                                   float scale, int chunk, void* stream);

/* FP8 dense decode: replaces src/attention_kernels.py:156-182 (`decode_attn_fp8`,
 * kernel :98-154).  Same arguments as bytes_decode_attn_bf16 with k, v OCP
 * float8_e4m3fn (strides in elements = bytes), widened to bf16 exactly; out bf16
 * (q's dtype).  Workspace size: bytes_decode_attn_bf16_workspace_size. */
int bytes_decode_attn_fp8(const void* q, const void* k, const void* v, void* out,
                          int B, int Hq, int Hk, int S, int D,
                          int64_t q_sb, int64_t q_sh,
                          int64_t k_sb, int64_t k_sh, int64_t k_ss,
                          int64_t v_sb, int64_t v_sh, int64_t v_ss,
                          int64_t o_sb, int64_t o_sh,
                          float scale, int chunk, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---------------------------------------------------------------------------
 * KIVI asymmetric min/max quantize + pack along the last axis.
 * Replaces the external KIVI `triton_quantize_and_pack_along_last_dim(x, 32, bits)`
 * called at benchmarks/kivi_latency.py:123,127 (arithmetic of
 * src/quantization.py:432-442; bit layout = inverse of kivi_latency.py:26-35).
 *   x     [rows, T], dtype x_dtype (0 bf16, 1 f16, 2 f32), row stride x_row_stride
 *   code  [rows, T*bits/32] int32: element i of word w = logical index w*(32/bits)+i,
 *         at bits [i*bits, (i+1)*bits)
 *   scale, mn [rows, T/group_size] f16:
 *         scale = max(hi-lo, 1e-8)/(2^bits-1), code = clamp(rint((x-lo)/scale)),
 *         both computed in fp32, scale/mn rounded to f16 afterwards.
 * bits in {2, 4}; T % group_size == 0; group_size % (32/bits) == 0.
 * ------------------------------------------------------------------------- */
int bytes_kivi_quantize_pack(const void* x, int x_dtype, int64_t rows, int T, int64_t x_row_stride,
                             int group_size, int bits, void* code, void* scale, void* mn, void* stream);

/* KIVI unpack + dequant along the last axis (kivi_latency.py:26-57):
 * out[r, t] = code * scale + mn, in f16 arithmetic when fp16_math != 0 (the
 * reference's unpacked-fp16 * fp16-scale + fp16-mn), else in fp32.
 * out [rows, T] contiguous, dtype out_dtype (0 bf16, 1 f16, 2 f32). */
int bytes_kivi_dequant(const void* code, const void* scale, const void* mn, int64_t rows, int T,
                       int group_size, int bits, int fp16_math, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Fused KIVI 2/4-bit decode attention.
 * Replaces benchmarks/kivi_latency.py:59-90 (`kivi_decode_attn`; semantics
 * `kivi_decode_attn_ref` :92-100): softmax([q.Kdq^T, q.Kres^T] * scale) [Vdq; Vres]
 * with GQA head map h -> h / (Hq/Hk).
 *   q        [B, Hq, D] bf16 (strides q_sb, q_sh)
 *   kq       [B, Hk, D, Sq*bits/32] int32  (keys packed per channel along tokens)
 *   k_scale, k_mn [B, Hk, D, Sq/32] f16
 *   k_res    [B, Hk, R, D] bf16 (strides kr_*)
 *   vq       [B, Hk, Sq, D*bits/32] int32  (values packed per token along channels)
 *   v_scale, v_mn [B, Hk, Sq, D/32] f16
 *   v_res    [B, Hk, R, D] bf16 (strides vr_*)
 *   out      [B, Hq, D] bf16 (strides o_sb, o_sh)
 * Packed tensors and their metadata are contiguous.  Sq % 32 == 0 (0 allowed;
 * other Sq return hipErrorInvalidValue), group size 32, D in {64, 128}.
 * scale: the reference uses 1/sqrt(D).
 * chunk: 0 = automatic kernel and split plan; > 0 = split length (tokens) of
 * the two-half / streaming kernels; < 0 = the pipelined kernel (D = 128,
 * Sq % 64 == 0, Sq >= 1024; otherwise as 0) with splits of -chunk
 * 256-token granules.  bytes_kivi_decode_workspace_size takes the same chunk.
 * ------------------------------------------------------------------------- */
int bytes_kivi_decode_workspace_size(int B, int Hq, int Hk, int Sq, int R, int D, int bits, int chunk,
                                     size_t* bytes);
int bytes_kivi_decode_attn(const void* q, const void* kq, const void* k_scale, const void* k_mn,
                           const void* k_res, const void* vq, const void* v_scale, const void* v_mn,
                           const void* v_res, void* out, int B, int Hq, int Hk, int Sq, int R, int D,
                           int bits, int64_t q_sb, int64_t q_sh, int64_t kr_sb, int64_t kr_sh,
                           int64_t kr_ss, int64_t vr_sb, int64_t vr_sh, int64_t vr_ss, int64_t o_sb,
                           int64_t o_sh, float scale, int chunk, void* workspace, size_t workspace_bytes,
                           void* stream);

/* ---------------------------------------------------------------------------
 * Token scoring.
 * Replaces src/attention_kernels.py:1113-1133 (`sparse_score_scalar`, kernel
 * :1077-1110) and :1199-1222 (`sparse_score_packed`, kernel :1136-1196).
 * k_mode selects the key format:
 *   0  bf16 keys [B, Hk, S, D] (score_bits = 16)
 *   1  OCP float8_e4m3fn keys [B, Hk, S, D] (score_bits = 8; widened to bf16 exactly)
 *   2  4-bit codes uint8 [B, Hk, S, D/2], two per byte, element c at bits 4*(c%2)
 *   3  2-bit codes uint8 [B, Hk, S, D/4], four per byte, element c at bits 2*(c%4)
 *   modes 2/3: k_scale, k_min bf16 [B, Hk, S, D/32] (strides m_*; one pair per
 *   32 dims, key = code * scale + min; the layout of bytes_score_keys_pack).
 * Scores:
 *   group_sum = 0: out [B, Hq, S] fp32, out[b,h,t] = (q[b,h] . k[b,h/G,t]) * scaling
 *   group_sum = 1: out [B, Hk, S] fp32, out[b,hk,t] = sum_{g<G} (q[b,hk*G+g] . k[b,hk,t]) * scaling
 *                  (the per-KV-head selection score of the token top-k path; G <= 16)
 *   q [B, Hq, D] bf16 (strides q_sb, q_sh); k strides k_* in storage elements
 *   (bytes for modes 1-3); out strides o_sb, o_sh (unit stride along S).
 *   D in {64, 128}.
 * hist (group_sum = 1 only, may be NULL): [B*Hk][2048] uint32, zero on entry,
 *   receives the count of each score's top 11 order-key bits; pass the first
 *   bytes of a bytes_topk workspace (its histogram region, B*Hk <= 1024) and
 *   call bytes_topk with hist_ready = 1 to skip its histogram pass.
 * ------------------------------------------------------------------------- */
int bytes_sparse_score(const void* q, const void* k, int k_mode, const void* k_scale, const void* k_min, void* out,
                       int B, int Hq, int Hk, int S, int D, int group_sum, int64_t q_sb, int64_t q_sh, int64_t k_sb,
                       int64_t k_sh, int64_t k_ss, int64_t m_sb, int64_t m_sh, int64_t m_ss, int64_t o_sb,
                       int64_t o_sh, float scaling, void* hist, void* stream);

/* ---------------------------------------------------------------------------
 * Quantize and pack score keys along head_dim.
 * Replaces src/attention_kernels.py:1225-1249 (`quantize_and_pack_score_keys`,
 * group_size = 32, the size every caller uses: benchmarks/test_correctness.py:706,
 * bench_sparse_crossover.py:188,201).  Per row and group of 32 dims, in fp32:
 * scale = max(max - min, 1e-8) / (2^bits - 1), code = clamp(rint((x - min) / scale)).
 *   x [rows, D] (x_dtype 0 bf16, 1 fp16, 2 fp32; row stride x_row_stride)
 *   packed uint8 [rows, D*bits/8]; scale, mn [rows, D/32] in x's dtype
 *   (rounded after the codes are chosen).  bits in {4, 2}, D % 32 == 0.
 * ------------------------------------------------------------------------- */
int bytes_score_keys_pack(const void* x, int x_dtype, int64_t rows, int D, int64_t x_row_stride, int bits,
                          void* packed, void* scale, void* mn, void* stream);

/* ---------------------------------------------------------------------------
 * Deterministic top-k per row.
 * Replaces `scores.topk(kb, dim=-1).indices` (src/attention_kernels.py:1262,
 * benchmarks/sparse_attention.py:307,358; selection semantics of
 * `select_topk` :226-325) with one total order: score descending, lowest index
 * first among equal scores, +0 == -0, NaN above +inf.
 *   scores [rows, n] fp32 (row stride row_stride, unit stride along n)
 *   out    [rows, k] int32 (row stride out_stride): ordered by that order when
 *          sorted != 0, else the same set by ascending index.
 * 1 <= k <= n, sorted or not.  k > 8192 takes a larger workspace (the
 * selection's sort values, rows * k * 8 bytes rounded up to 8192 entries).
 * hist_ready = 1: the workspace's histogram region already holds the rows'
 *   digit histograms (bytes_sparse_score with hist); rows <= 1024.
 * ------------------------------------------------------------------------- */
int bytes_topk_workspace_size(int64_t rows, int n, int k, size_t* bytes);
int bytes_topk(const void* scores, int64_t rows, int n, int64_t row_stride, int k, int sorted, int hist_ready,
               void* out, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Gather attention over selected rows.
 * Replaces src/attention_kernels.py:1037-1059 (`sparse_gather_attn`, kernel
 * :987-1034) with the masking of benchmarks/sparse_attention.py:367-387:
 *   out[b,h] = softmax_j(scaling * q[b,h] . k[b,h/G,idx_j]) v[b,h/G,idx_j]
 * over the kb entries idx_j in [0, S); other entries are ignored.
 *   per_head = 1: idx [B, Hq, kb] int32 (one list per query head, the reference layout)
 *   per_head = 0: idx [B, Hk, kb] int32 (one list per KV head, shared by its G query heads)
 *   idx strides i_sb, i_sh (unit stride along kb); k, v [B, Hk, S, D] bf16, or OCP
 *   float8_e4m3fn when kv_fp8 = 1 (widened to bf16 exactly); out [B, Hq, D] bf16.
 *   D in {64, 128}.
 * page = 0: idx entries are rows.  page > 0: idx holds kb/page page ids per list,
 *   page id p standing for rows min(p*page + o, S-1), o < page (the Quest
 *   expansion, benchmarks/sparse_attention.py:358-363).
 * limit: rows >= limit are masked (the causal bound pos+1; S at decode).
 * ------------------------------------------------------------------------- */
int bytes_gather_attn_workspace_size(int B, int Hq, int Hk, int kb, int D, int per_head, int chunk,
                                     size_t* bytes);
int bytes_gather_attn(const void* q, const void* k, const void* v, int kv_fp8, const void* idx, void* out,
                      int B, int Hq, int Hk, int S, int D, int kb, int per_head, int page, int limit,
                      int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                      int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t i_sb, int64_t i_sh,
                      int64_t o_sb, int64_t o_sh, float scaling, int chunk, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Quest page metadata and bounds.
 * Replaces the page part of benchmarks/sparse_attention.py:328-364 (`_quest_select`;
 * dense form benchmarks/eval_ppl.py:54-79).
 * bytes_quest_page_minmax: kmin/kmax [B, Hk, np, D] bf16 contiguous, np = ceil(S/page):
 *   elementwise min/max of the keys of each page, the last partial page padded
 *   with the last key (:336-341).  k [B, Hk, S, D] bf16 (strides k_*).
 * bytes_quest_page_scores: bound [B, Hq, np] fp32 (strides o_sb, o_sh):
 *   scale * sum_d max(q_d*kmin_d, q_d*kmax_d), d summed in ascending order in fp32
 *   (bit-identical to a sequential evaluation); -inf for pages starting after
 *   `pos`; +inf for pages overlapping (pos - local_w, pos] when local_w > 0.
 *   q [B, Hq, D] bf16; any G = Hq/Hk (head blocks of 16); D in {64, 128}.
 * ------------------------------------------------------------------------- */
int bytes_quest_page_minmax(const void* k, void* kmin, void* kmax, int B, int Hk, int S, int D, int page,
                            int64_t k_sb, int64_t k_sh, int64_t k_ss, void* stream);
int bytes_quest_page_scores(const void* q, const void* kmin, const void* kmax, void* bound, int B, int Hq,
                            int Hk, int np, int D, int page, int pos, int local_w, int64_t q_sb, int64_t q_sh,
                            int64_t o_sb, int64_t o_sh, float scale, void* stream);

/* Quest decode after the page bounds, in one kernel (plus the split merge):
 * replaces the page top-k and the attention of benchmarks/sparse_attention.py
 * :356-387 (`_quest_select`'s topk over page bounds, then `attend_topk`).
 * For every query head, the top npick pages of bound[b, hq, 0..np) (the
 * exact top-k of bytes_topk: bound descending, lowest page first on equal
 * bounds) are selected inside the gather kernel and attended over in
 * ascending page order, rows min(p*page + o, S-1), rows >= limit masked; the
 * result equals bytes_topk (unsorted) followed by bytes_gather_attn
 * (per_head = 1) bit for bit.  bound strides b_sb, b_sh (unit stride along
 * pages); np <= 4096 (hipErrorNotSupported above); other arguments as
 * bytes_gather_attn, whose workspace size (per_head = 1, kb = npick * page)
 * this call needs.
 */
int bytes_quest_gather_attn(const void* q, const void* k, const void* v, int kv_fp8, const void* bound, int64_t b_sb,
                            int64_t b_sh, int np, int npick, void* out, int B, int Hq, int Hk, int S, int D, int page,
                            int limit, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                            int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scaling,
                            int chunk, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Row steps of the selection functions for query chunks of Qc >= 1 rows
 * (benchmarks/sparse_attention.py:226-387: select_topk, _quest_select,
 * attend_topk).  Row r of a [.., Qc, n] array belongs to query row r % Qc,
 * whose position is pos[r % Qc] (int64 device array of Qc entries).
 * bytes_select_mask: in place over fp32 scores [rows, n] (row stride
 *   row_stride): candidate t stands for position t*unit (unit 1: tokens,
 *   :297-300; unit = page size: pages, :346-355); -inf where t*unit > pos,
 *   then +inf where local_w > 0 and max(pos-local_w+1, 0)/unit <= t <= pos/unit.
 * bytes_select_fill: out[r, j] = in[r, j] if j < k_in and 0 <= in[r, j] < S
 *   and in[r, j] <= pos, else S (the sentinel of :288-293 and the masking rule
 *   of :376).  in_dtype / out_dtype: 0 int32, 1 int64.
 * bytes_select_pages: out[r, j] = min(page_ids[r, j / page] * page + j % page,
 *   S - 1) int64 [rows, npick*page] from int32 page ids [rows, npick] (:358-363).
 * bytes_select_mask_at: bytes_select_mask over a chunk of candidates whose
 *   first one is candidate key0 (candidate j stands for position
 *   (key0 + j) * unit): the per-tile mask of the streaming loop (:294-300).
 * bytes_select_merge: one merge of the streaming top-k (:301-309).  Row r's
 *   candidates are cand[r][off .. off + nrun + n) fp32 (row stride cand_rs):
 *   its running list of nrun entries, whose key indices are ridx[r][0 .. nrun)
 *   int32, then the scores of keys kc0, kc0 + 1, ...; sel[r][0 .. ksel) int32
 *   are the positions the top-k picked there.  Writes the next running list:
 *   out_vals[r][out_off + i] (if out_vals is not NULL) and out_idx[r][i] =
 *   (score, key index) of candidate sel[r][i] for i < ksel, (-inf, S) for
 *   ksel <= i < kout.
 * bytes_select_recent: the "recent" selector (:261-265): out[r, j] =
 *   max(pos[r % Qc] - j, 0) int64 [rows, kb].
 * ------------------------------------------------------------------------- */
int bytes_select_mask(void* scores, int64_t rows, int n, int64_t row_stride, const void* pos, int Qc, int unit,
                      int local_w, void* stream);
int bytes_select_mask_at(void* scores, int64_t rows, int n, int64_t row_stride, int64_t key0, const void* pos,
                         int Qc, int unit, int local_w, void* stream);
int bytes_select_merge(const void* cand, int64_t cand_rs, int off, int nrun, const void* ridx, int64_t ridx_rs,
                       const void* sel, int64_t sel_rs, int ksel, int kc0, int S, int64_t rows, void* out_vals,
                       int64_t out_vals_rs, int out_off, void* out_idx, int64_t out_idx_rs, int kout,
                       void* stream);
int bytes_select_recent(const void* pos, int Qc, int64_t rows, int kb, void* out, void* stream);
int bytes_select_fill(const void* in, int in_dtype, int64_t in_rs, int k_in, void* out, int out_dtype,
                      int64_t out_rs, int k_out, int64_t rows, const void* pos, int Qc, int64_t S, void* stream);
int bytes_select_pages(const void* page_ids, int64_t rows, int npick, int page, int64_t S, void* out,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Study-harness microkernels.
 * bytes_gather_reduce: replaces `_gather_reduce_kernel` of
 *   benchmarks/bench_access_pattern.py:25-52: out[h, d] = sum_k v[h, idx[h, k], d]
 *   fp32 [H, D] for v fp16 [H, S, D] (strides v_sh, v_ss; D in {8, 16, 32, 64,
 *   128, 256}) and idx int32 [H, K] (row stride i_sh); entries outside [0, S)
 *   read the clamped row.  Sums in a fixed order (deterministic).
 * bytes_packed_stage: replaces `_packed_stage_kernel` of
 *   benchmarks/bench_unpack_ablation.py:19-53: out[b, hq, t] fp32 (strides o_sb,
 *   o_sh) over packed keys kp uint8 [B, Hk, S, D*bits/8] (strides k_*) with bf16
 *   scale/zero [B, Hk, S, D/32] (strides m_*) and q bf16 [B, Hq, D]:
 *   stage 0 sum of the packed byte of every column, 1 sum of the codes,
 *   2 sum of code*scale+zero, 3 sum of (code*scale+zero)*q.  D in {64, 128},
 *   bits in {4, 2}.
 * ------------------------------------------------------------------------- */
int bytes_gather_reduce(const void* v, int64_t v_sh, int64_t v_ss, const void* idx, int64_t i_sh, void* out, int H,
                        int S, int K, int D, void* stream);
int bytes_packed_stage(const void* q, int64_t q_sb, int64_t q_sh, const void* kp, int64_t k_sb, int64_t k_sh,
                       int64_t k_ss, const void* scale, const void* zero, int64_t m_sb, int64_t m_sh, int64_t m_ss,
                       void* out, int64_t o_sb, int64_t o_sh, int B, int Hq, int Hk, int S, int D, int bits,
                       int stage, void* stream);

/* Floor probes: the fixed cost of a launch, the first HBM round trip and the
 * streaming-read ceiling the decode kernels are measured against (no
 * counterpart in the reference; they bound what its decode paths can reach
 * on MI355X).  bytes_stream_read: `wgs` workgroups of 256 threads each read
 * bytes / wgs contiguous bytes of src in 16-byte loads (bytes a multiple of
 * 16 * wgs, src 16-byte aligned), out [wgs * 256] fp32 (a fold of the words
 * read); nontemporal != 0 issues the loads with the non-temporal hint (as
 * the decode kernels read K/V rows).  bytes_empty_launch: `wgs` workgroups
 * that do nothing. */
int bytes_stream_read(const void* src, int64_t bytes, int wgs, int nontemporal, void* out, void* stream);
int bytes_empty_launch(int wgs, void* stream);

/* ---------------------------------------------------------------------------
 * Product-quantized decode with paged caches, outlier channels and fp8 values.
 * Replaces src/attention_kernels.py:
 *   paged_attn_pq_lut_kv    :588-622 (kernel :505-586)   vidx + vcb, block_table
 *   decode_attn_pq_lut_asym :713-753 (kernel :625-711)   v dense, k_out/q_out
 *   paged_attn_pq_lut_asym  :858-906 (kernel :756-856)   the same, block_table
 * Scores: sum_j lut[b,h,j,kidx[row,j]] + sum_{c<C} q_out[b,h,c] * k_out[row,c]
 *   (fp32; C <= 16, C = 0: no outliers); softmax without a scale inside
 *   (`scale` multiplies the scores: pass 1.0).
 * Values: exactly one of  vidx (+ vcb, fp16 [M,K,8], per KV head when vcb_sh
 *   != 0: reconstructed rows)  or  v (bf16, or float8_e4m3fn when v_fp8 = 1).
 * Caches: block_table == NULL: contiguous [B, Hk, S, .] (strides *_sb, *_sh,
 *   *_ss).  Otherwise paged [num_blocks, Hk, block_size, .] with *_sb the block
 *   stride: token t of sequence b is row t % block_size of block
 *   block_table[b * bt_sb + t / block_size]; sequence b has context_lens[b]
 *   tokens (int32, device memory); S = max_blocks * block_size bounds every
 *   length.  Block ids are clamped into [0, num_blocks).
 * k_out / q_out dtypes: 0 bf16, 1 fp16, 2 fp32 (unit stride along C).
 * out [B, Hq, D] of out_dtype; workspace from bytes_pq_decode_workspace_size
 * (same S), in the split-K workspace family.
 * ------------------------------------------------------------------------- */
int bytes_pq_lut_decode_attn(const void* lut, int64_t l_sb, int64_t l_sh, const void* kidx, int64_t ki_sb,
                             int64_t ki_sh, int64_t ki_ss, const void* vidx, int64_t vi_sb, int64_t vi_sh,
                             int64_t vi_ss, const void* vcb, int64_t vcb_sh, const void* v, int v_fp8, int64_t v_sb,
                             int64_t v_sh, int64_t v_ss, const void* kout, int ko_dtype, int64_t ko_sb,
                             int64_t ko_sh, int64_t ko_ss, const void* qout, int qo_dtype, int64_t qo_sb,
                             int64_t qo_sh, int C, const int* block_table, int64_t bt_sb, const int* context_lens,
                             int block_size, int num_blocks, void* out, int out_dtype, int64_t o_sb, int64_t o_sh,
                             int B, int Hq, int Hk, int S, int D, int K, float scale, int chunk, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Per-key LUT + outlier scores.
 * Replaces src/attention_kernels.py:960-984 (`sparse_score_pq_lut_asym`,
 * kernel :909-958): out[b,h,t] = sum_j lut[b,h,j,kidx[b,h/G,t,j]]
 *   + sum_{c<C} q_out[b,h,c] * k_out[b,h/G,t,c], fp32 [B, Hq, S] (strides
 *   o_sb, o_sh; unit stride along S).  Layouts as bytes_pq_lut_decode_attn
 *   (contiguous caches).
 * ------------------------------------------------------------------------- */
int bytes_pq_lut_scores(const void* lut, int64_t l_sb, int64_t l_sh, const void* kidx, int64_t ki_sb, int64_t ki_sh,
                        int64_t ki_ss, const void* kout, int ko_dtype, int64_t ko_sb, int64_t ko_sh, int64_t ko_ss,
                        const void* qout, int qo_dtype, int64_t qo_sb, int64_t qo_sh, int C, void* out, int64_t o_sb,
                        int64_t o_sh, int B, int Hq, int Hk, int S, int D, int K, void* stream);

/* ---------------------------------------------------------------------------
 * Product-quantized decode attention (d_sub = 8, M = D/8 subspaces, K <= 256
 * codewords, K % 4 == 0; codebooks fp16 [M, K, 8], per KV head when the head
 * stride *_sh is non-zero; codes uint8 [B, Hk, S, M] with unit stride in M and
 * token stride M).
 *   mode 0  decode_attn_pq_lut_kv  src/attention_kernels.py:471-500 (kernel :397-469):
 *           score_t = sum_j lut[b,h,j,kidx[t,j]]; values = concat_j vcb[j, vidx[t,j]]
 *   mode 1  decode_attn_pq_lut     :365-392 (kernel :301-363): LUT scores, dense bf16 v
 *   mode 2  decode_attn_dequant    :267-296 (kernel :187-265): scores q . k_hat with
 *           k_hat = concat_j kcb[j, kidx[t,j]] (no scale), dense bf16 v
 *   mode 3  mode 0 with the LUT precompute fused (benchmarks/test_correctness.py:272-273
 *           followed by :471-500), no LUT in HBM: for G <= 8 the scores are
 *           scale * (q . k_hat) on MFMA from the codebook rows the codes select
 *           (exact products, fp32 sums; within the attention tolerance of
 *           bytes_pq_build_lut + mode 0); for G > 8 each workgroup builds
 *           lut = scale * (q . kcb) in LDS entry for entry as bytes_pq_build_lut
 *           (bit-identical to the two calls); q, kcb, vidx, vcb required, lut unused
 *   lut [B, Hq, M, K] fp32 (one head contiguous); q [B, Hq, D] bf16;
 *   out [B, Hq, D] of out_dtype (0 bf16, 1 f16, 2 f32).  `scale` multiplies the
 *   scores in modes 0-2 (the reference has none: pass 1.0) and the LUT entries in
 *   mode 3.
 * ------------------------------------------------------------------------- */
int bytes_pq_decode_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk, size_t* bytes);
int bytes_pq_decode_attn(int mode, const void* lut, const void* q, const void* kcb, const void* kidx,
                         const void* vidx, const void* vcb, const void* v, void* out, int out_dtype, int B,
                         int Hq, int Hk, int S, int D, int K, int64_t l_sb, int64_t l_sh, int64_t q_sb,
                         int64_t q_sh, int64_t kcb_sh, int64_t ki_sb, int64_t ki_sh, int64_t ki_ss,
                         int64_t vi_sb, int64_t vi_sh, int64_t vi_ss, int64_t vcb_sh, int64_t v_sb,
                         int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scale, int chunk,
                         void* workspace, size_t workspace_bytes, void* stream);

/* PQ setup path.
 * bytes_pq_build_lut: lut[b,h,j,c] = scale * sum_e q[b,h,8j+e] * cb[h/G][j][c][e] (fp32),
 *   the LUT precompute of benchmarks/test_correctness.py:272-273.
 * bytes_pq_encode: idx[r, j] = argmin_c sum_e (x[r, 8j+e] - cb[j][c][e])^2 in fp32
 *   (e ascending, no fused multiply-add), first index on ties: the CPU rule of
 *   src/quantization.py:203-211.  x [heads * rows_per_head, D] (dtype 0 bf16,
 *   1 f16, 2 f32, row stride x_row_stride); codebook fp16 (cb_f32 = 0) or fp32.
 * bytes_pq_decode_vectors: out[r, 8j+e] = cb[j][idx[r, j]][e] fp32
 *   (src/quantization.py:213-226).
 * bytes_pq_kmeans_update: one k-means centroid update (src/quantization.py:120-130)
 *   for x [heads, n, D] fp32 with labels [heads, n, M] uint8: cb = mean of the
 *   points of each cluster, summed in index order; an empty cluster takes the
 *   point reseed[head, j, c] (int64).  Writes cb_f16 and cb_f32 [heads, M, K, 8].
 * ------------------------------------------------------------------------- */
int bytes_pq_build_lut(const void* q, const void* cb, void* lut, int B, int Hq, int Hk, int D, int K,
                       int64_t q_sb, int64_t q_sh, int64_t cb_sh, float scale, void* stream);
int bytes_pq_encode(const void* x, int x_dtype, int heads, int64_t rows_per_head, int64_t x_row_stride, int D,
                    const void* cb, int cb_f32, int64_t cb_sh, int K, void* idx, void* stream);
int bytes_pq_decode_vectors(const void* idx, int heads, int64_t rows_per_head, int D, const void* cb,
                            int cb_f32, int64_t cb_sh, int K, void* out, void* stream);
int bytes_pq_kmeans_update(const void* x, int heads, int64_t n, int D, int K, const void* labels,
                           const void* reseed, void* cb_f16, void* cb_f32, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* BYTES_AMD_H_ */
