// Gather attention over selected key/value rows.
//
// Replaces src/attention_kernels.py:987-1059 (`sparse_gather_attn`): exact
// fp32 online-softmax attention of each query head over the K/V rows named by
// an index list, with the masking rule of benchmarks/sparse_attention.py:376
// (`attend_topk`: entries outside [0, S) take no part).  Two index layouts:
//  * per query head  idx [B, Hq, kb]  (the reference's layout): a unit is one
//    query head;
//  * per KV head     idx [B, Hk, kb]  (one selection shared by the GQA group,
//    the token top-k pipeline): a unit is up to 16 query heads of one group,
//    which share every gathered row, so one MFMA tile serves all of them.
// In page mode the list holds page ids, each standing for `page` consecutive
// rows p*page + o clamped to S-1 (benchmarks/sparse_attention.py:358-363, the
// Quest expansion), expanded while the list is staged.  Rows at or past
// `limit` (the causal bound, S at decode) are masked.
// K and V may be fp8 (OCP e4m3fn; the output is then bf16, :1044): rows are
// widened to bf16 exactly while staged in LDS.
// The index list of a unit is cut into split-K chunks; each workgroup stages
// its chunk's row numbers in LDS, then its waves run the dense bf16 tile loop
// with rows fetched through that list (prefetching the next tile's rows while
// the current tile is computed).
// Quest selection in the prologue (bytes_quest_gather_attn): instead of a
// page list, each workgroup receives its query head's row of page bounds and
// selects the top npick pages itself (exact: bound descending, lowest
// page first among equal bounds, the order of bytes_topk; the workgroup radix
// select of wave_select.h over bounds held in registers), listing them in
// ascending page order as the unfused top-k does; the page top-k launch of
// benchmarks/sparse_attention.py:356-358 then disappears from the step.
#include "dense_tile.h"
#include "wave_select.h"

namespace bytes_amd {

struct GatherArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const void* k;             // bf16 or fp8 e4m3fn rows
  int64_t k_sb, k_sh, k_ss;
  const void* v;
  int64_t v_sb, v_sh, v_ss;
  const int32_t* idx;        // [B, Hq or Hk, kb], unit stride along kb
  int64_t i_sb, i_sh;
  int Hk, G, HB, S, kb, chunk, per_head;
  int page;                  // 0: idx holds rows; > 0: idx holds page ids of `page` rows each
  int limit;                 // rows >= limit take no part
  const float* bound;        // Quest selection: page bounds [B, Hq, np] (row strides b_sb, b_sh)
  int64_t b_sb, b_sh;
  int np;
  int b_vec;                 // every bound row starts 16-byte aligned and np % 4 == 0
  float scale_log2;
  FastDiv dG;                // division by G
  SplitKOut o;
};

constexpr int kGatherWaves = 4;
constexpr int kGatherChunkMax = 1024;   // index-list entries per workgroup

constexpr int kGatherSelMax = 4096;     // pages per bound row selected in the prologue

template <int D>
struct GatherCfg {
  static constexpr int kRows = kGatherChunkMax * 4;
  static constexpr int kSelWs = block_select_words<kGatherWaves * 64>();
  static constexpr int kSel = kSelWs * 4 + kGatherSelMax * 4;   // selection words, page list
  static_assert(kSel <= DenseCfg<D>::kSmem, "the selection fits in the tile buffers");
  static constexpr int kSmem = DenseCfg<D>::kSmem + kRows;
};

// Loads of one 32-row tile whose rows are rows[j0 .. j0+31] (entries past n or
// negative read row 0: same instructions every tile, no divergence).
template <int D>
__device__ __forceinline__ void gather_issue(const uint16_t* kbase, const uint16_t* vbase, int64_t k_ss,
                                             int64_t v_ss, const int32_t* rows, int j0, int n, int lane,
                                             DenseRegs<D>& r) {
  using C = DenseCfg<D>;
#pragma unroll
  for (int i = 0; i < C::CPL; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / C::CPR, pos = p - rr * C::CPR;
    const int j = j0 + rr;
    int row = j < n ? rows[j] : 0;
    row = row < 0 ? 0 : row;
    r.k[i] = ld16_nt(kbase + (int64_t)row * k_ss + pos * 8);
    r.v[i] = ld16_nt(vbase + (int64_t)row * v_ss + pos * 8);
  }
}

template <int D>
__device__ __forceinline__ void gather_issue_fp8(const uint8_t* kbase, const uint8_t* vbase, int64_t k_ss,
                                                 int64_t v_ss, const int32_t* rows, int j0, int n, int lane,
                                                 DenseRegs8<D>& r) {
  using R = DenseRegs8<D>;
#pragma unroll
  for (int i = 0; i < R::CPL8; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / R::CPR8, pos = p - rr * R::CPR8;
    const int j = j0 + rr;
    int row = j < n ? rows[j] : 0;
    row = row < 0 ? 0 : row;
    r.k[i] = ld16_nt(kbase + (int64_t)row * k_ss + pos * 16);
    r.v[i] = ld16_nt(vbase + (int64_t)row * v_ss + pos * 16);
  }
}

// SEL > 0: Quest selection in the prologue, SEL bounds per thread.
template <int D, bool FP8, int SEL>
__global__ __launch_bounds__(kGatherWaves * 64, 2) void gather_decode_kernel(GatherArgs a) {
  using C = DenseCfg<D>;
  __shared__ __attribute__((aligned(16))) char smem_raw[GatherCfg<D>::kSmem];
  int32_t* rows = reinterpret_cast<int32_t*>(smem_raw + C::kSmem);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // per-head units are (b, query head): the split grid's "kv heads" are the
  // query heads (o.Hk = Hq, o.HB = 1) and the kv head is hq / G
  const UnitLoc loc = splitk_locate(a.o);
  const int unit = loc.unit, split = loc.split;

  int b = loc.b, hk, hq0, nh;
  const int32_t* irow;
  if (a.per_head) {
    const int hq = loc.hk;
    hk = fast_div(hq, a.dG);
    hq0 = hq;
    nh = 1;
    irow = a.idx + (int64_t)b * a.i_sb + (int64_t)hq * a.i_sh;
  } else {
    hk = loc.hk;
    const int hb = loc.hb;
    hq0 = hk * a.G + hb * 16;
    nh = min(16, a.G - hb * 16);
    irow = a.idx + (int64_t)b * a.i_sb + (int64_t)hk * a.i_sh;
  }

  // Q first: its load is then in flight with the index loads below
  bf16x8 qb[C::KK];
  load_q_bf16<D>(a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh, a.q_sh, nh, lane, qb);

  // Quest selection: thread t loads bounds SEL*t .. +SEL of the head's row
  // straight into registers, the workgroup selects the top kb / page pages
  // (block_select) and lists them, ascending, in LDS
  int32_t* pids = reinterpret_cast<int32_t*>(smem_raw + GatherCfg<D>::kSelWs * 4);
  if constexpr (SEL > 0) {
    constexpr int NT = kGatherWaves * 64;
    const float* bsrc = a.bound + (int64_t)b * a.b_sb + (int64_t)hq0 * a.b_sh;
    uint32_t key[SEL];
    // all of a thread's loads in flight together (indices clamped to the
    // row; elements past np are not selected): 16-byte chunks where the row
    // allows, else single floats
    if (a.b_vec) {
      u32x4 bv[SEL / 4];
#pragma unroll
      for (int u = 0; u < SEL / 4; ++u) bv[u] = ld16(bsrc + 4 * min((SEL / 4) * (int)threadIdx.x + u, a.np / 4 - 1));
#pragma unroll
      for (int u = 0; u < SEL / 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) key[4 * u + e] = score_order_key(__uint_as_float(bv[u][e]));
    } else {
      float bv[SEL];
#pragma unroll
      for (int u = 0; u < SEL; ++u) bv[u] = bsrc[min(SEL * (int)threadIdx.x + u, a.np - 1)];
#pragma unroll
      for (int u = 0; u < SEL; ++u) key[u] = score_order_key(bv[u]);
    }
    uint32_t* ws = reinterpret_cast<uint32_t*>(smem_raw);
    const BlockSel sel = block_select<NT, SEL>(key, a.np, a.kb / a.page, ws);
    block_select_emit<NT, SEL>(key, a.np, sel, ws, [&](uint32_t pos, int idx, uint32_t) { pids[pos] = idx; });
    __syncthreads();
  }

  const int p_begin = split * a.chunk;
  const int n = min(a.chunk, a.kb - p_begin);
  for (int i = threadIdx.x; i < n; i += kGatherWaves * 64) {
    const int j = p_begin + i;
    int64_t r;
    bool ok;
    if (a.page > 0) {
      const int pid = SEL > 0 ? pids[j / a.page] : irow[j / a.page];
      r = (int64_t)pid * a.page + j % a.page;
      r = r < a.S - 1 ? r : a.S - 1;
      ok = pid >= 0;
    } else {
      r = irow[j];
      ok = r >= 0;
    }
    rows[i] = (ok && r < a.limit) ? (int)r : -1;
  }
  __syncthreads();

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  char* kst = smem_raw + w * C::WAVE;
  char* vst = kst + C::VT;
  constexpr int STEP = kGatherWaves * kTile;
  int j = w * kTile;
  if (j < n) {
    using Regs = typename std::conditional<FP8, DenseRegs8<D>, DenseRegs<D>>::type;
    using Elem = typename std::conditional<FP8, uint8_t, uint16_t>::type;
    const Elem* kbase = static_cast<const Elem*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
    const Elem* vbase = static_cast<const Elem*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
    Regs r;
    auto issue = [&](int j0) {
      if constexpr (FP8) gather_issue_fp8<D>(kbase, vbase, a.k_ss, a.v_ss, rows, j0, n, lane, r);
      else gather_issue<D>(kbase, vbase, a.k_ss, a.v_ss, rows, j0, n, lane, r);
    };
    issue(j);
    for (; j < n; j += STEP) {
      // rows of this tile that take part: inside the chunk and a valid index
      const int jj = j + (lane & 31);
      const bool ok = jj < n && rows[jj < n ? jj : 0] >= 0;
      const uint32_t vmask = (uint32_t)__ballot(ok);
      wave_lds_sync();
      if constexpr (FP8) dense_stage_fp8<D>(lane, r, kst, vst);
      else dense_stage<D>(lane, r, kst, vst);
      issue(j + STEP);
      wave_lds_sync();
      dense_compute<D>(vmask, a.scale_log2, lane, qb, kst, vst, m_run, l_run, acc);
    }
  }
  splitk_epilogue<D, kGatherWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b, hq0,
                                   nh, kDmapDense);
}

static void gather_plan(int kb, long units, int chunk_req, int* chunk, int* ns) {
  const int step = kGatherWaves * kTile;
  int c;
  if (chunk_req > 0) {
    c = chunk_req;
  } else {
    // about one workgroup per CU: each wave then pipelines at least two tiles
    const long target = device_cu_count();
    c = (int)(((long)kb * units + target - 1) / target);
  }
  c = (c + step - 1) / step * step;
  if (c < step) c = step;
  if (c > kGatherChunkMax) c = kGatherChunkMax;
  *chunk = c;
  *ns = (kb + c - 1) / c;
}

static void gather_launch(const GatherArgs& a, int D, int kv_fp8, dim3 grid, dim3 block, hipStream_t st) {
#define GL(DD, F8, SL) BYTES_LAUNCH(kProfGather, (gather_decode_kernel<DD, F8, SL>), grid, block, 0, st, a)
#define GL_SEL(DD, F8)                  \
  if (!a.bound) GL(DD, F8, 0);          \
  else if (a.np <= 1024) GL(DD, F8, 4); \
  else if (a.np <= 2048) GL(DD, F8, 8); \
  else GL(DD, F8, 16);
  if (D == 128) {
    if (kv_fp8) { GL_SEL(128, true) } else { GL_SEL(128, false) }
  } else {
    if (kv_fp8) { GL_SEL(64, true) } else { GL_SEL(64, false) }
  }
#undef GL_SEL
#undef GL
}

static long gather_units(int B, int Hq, int Hk, int per_head) {
  const int G = Hq / Hk, HB = (G + 15) / 16;
  return per_head ? (long)B * Hq : (long)B * Hk * HB;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_gather_attn_workspace_size(int B, int Hq, int Hk, int kb, int D, int per_head, int chunk_req,
                                     size_t* bytes) {
  if (!bytes || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || kb <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  const long units = gather_units(B, Hq, Hk, per_head);
  int chunk, ns;
  gather_plan(kb, units, chunk_req, &chunk, &ns);
  *bytes = splitk_workspace_bytes(units, ns, D);
  return 0;
}

int bytes_gather_attn(const void* q, const void* k, const void* v, int kv_fp8, const void* idx, void* out, int B,
                      int Hq, int Hk, int S, int D, int kb, int per_head, int page, int limit, int64_t q_sb, int64_t q_sh,
                      int64_t k_sb, int64_t k_sh, int64_t k_ss, int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t i_sb, int64_t i_sh,
                      int64_t o_sb, int64_t o_sh, float scaling, int chunk_req, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !idx || !out || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || S <= 0 || kb <= 0)
    return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  if (page < 0 || (page > 0 && kb % page != 0) || limit < 0 || limit > S) return (int)hipErrorInvalidValue;
  const long units = gather_units(B, Hq, Hk, per_head);
  if (units > kMaxUnits) return (int)hipErrorInvalidConfiguration;
  GatherArgs a;
  a.page = page;
  a.limit = limit;
  a.bound = nullptr;
  a.b_sb = a.b_sh = 0;
  a.np = 0;
  a.b_vec = 0;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v = v;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.idx = static_cast<const int32_t*>(idx);
  a.i_sb = i_sb; a.i_sh = i_sh;
  a.Hk = Hk; a.G = Hq / Hk; a.HB = (a.G + 15) / 16; a.S = S; a.kb = kb;
  a.per_head = per_head ? 1 : 0;
  a.dG = make_fastdiv((uint32_t)a.G);
  a.scale_log2 = scaling * kLog2e;
  int ns;
  gather_plan(kb, units, chunk_req, &a.chunk, &ns);
  if (ns > 1024) return (int)hipErrorInvalidConfiguration;
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  a.o.out = out;
  a.o.out_dtype = kOutBF16;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  // the merge kernel maps unit -> (b, first query head) through (Hk, HB, G)
  if (per_head) {
    a.o.Hk = Hq; a.o.HB = 1; a.o.G = 1;
  } else {
    a.o.Hk = Hk; a.o.HB = a.HB; a.o.G = a.G;
  }
  splitk_carve(workspace, units, ns, a.o);
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)(ns * units)), block(kGatherWaves * 64);
  gather_launch(a, D, kv_fp8, grid, block, st);
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

// Quest decode after the page bounds: per query head, the top npick pages of
// bound[b, hq, :np] (exact; bound descending, lowest page first on equal
// bounds) are selected inside the gather kernel and attended over, rows
// p*page + o clamped to S-1, rows >= limit masked.  Same workspace as
// bytes_gather_attn with per_head = 1 and kb = npick * page.
int bytes_quest_gather_attn(const void* q, const void* k, const void* v, int kv_fp8, const void* bound, int64_t b_sb,
                            int64_t b_sh, int np, int npick, void* out, int B, int Hq, int Hk, int S, int D, int page,
                            int limit, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                            int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scaling,
                            int chunk_req, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !bound || !out || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || S <= 0)
    return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  if (page <= 0 || np <= 0 || npick <= 0 || npick > np || limit < 0 || limit > S) return (int)hipErrorInvalidValue;
  if (np > kGatherSelMax) return (int)hipErrorNotSupported;
  const long units = gather_units(B, Hq, Hk, 1);
  if (units > kMaxUnits) return (int)hipErrorInvalidConfiguration;
  const int kb = npick * page;
  GatherArgs a;
  a.page = page;
  a.limit = limit;
  a.bound = static_cast<const float*>(bound);
  a.b_sb = b_sb; a.b_sh = b_sh;
  a.np = np;
  a.b_vec = (reinterpret_cast<uintptr_t>(bound) % 16 == 0 && b_sb % 4 == 0 && b_sh % 4 == 0 && np % 4 == 0) ? 1 : 0;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v = v;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.idx = nullptr;
  a.i_sb = a.i_sh = 0;
  a.Hk = Hk; a.G = Hq / Hk; a.HB = (a.G + 15) / 16; a.S = S; a.kb = kb;
  a.per_head = 1;
  a.dG = make_fastdiv((uint32_t)a.G);
  a.scale_log2 = scaling * kLog2e;
  int ns;
  gather_plan(kb, units, chunk_req, &a.chunk, &ns);
  if (ns > 1024) return (int)hipErrorInvalidConfiguration;
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  a.o.out = out;
  a.o.out_dtype = kOutBF16;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  a.o.Hk = Hq; a.o.HB = 1; a.o.G = 1;
  splitk_carve(workspace, units, ns, a.o);
  hipStream_t st = static_cast<hipStream_t>(stream);
  gather_launch(a, D, kv_fp8, dim3((unsigned)(ns * units)), dim3(kGatherWaves * 64), st);
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

}  // extern "C"
