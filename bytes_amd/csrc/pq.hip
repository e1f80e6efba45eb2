// Product-quantized KV decode attention, LUT build, PQ encode and k-means update.
//
// Replaces src/attention_kernels.py:
//   decode_attn_pq_lut_kv  :397-500  LUT-scored keys, codebook-reconstructed values
//   decode_attn_pq_lut     :301-392  LUT-scored keys, dense V
//   decode_attn_dequant    :187-296  codebook-reconstructed keys, dense V
//   paged_attn_pq_lut_kv   :505-622  the LUT-KV decode over a paged cache
//   decode_attn_pq_lut_asym :625-753 LUT scores + exact outlier channels, bf16/fp8 V
//   paged_attn_pq_lut_asym :756-906  the same over a paged cache
//   sparse_score_pq_lut_asym :909-984 per-key LUT + outlier scores (no softmax)
// and, on the setup side, the LUT precompute of benchmarks/test_correctness.py
// :272-273, ProductQuantizer.quantize/.dequantize (src/quantization.py:160-226)
// and the k-means of src/quantization.py:102-132.
//
// Layouts (d_sub = 8, M = D/8 subspaces, K <= 256 codewords):
//   lut   [B, Hq, M, K] fp32, one head contiguous
//   codes [B, Hk, S, M] uint8 (unit stride along M)
//   codebooks fp16 [Hk or 1, M, K, 8] contiguous (per-KV-head or shared)
//
// Decode, general kernel (pq_decode_kernel: every mode, paged caches,
// outliers, any G): a unit is (b, kv head, group of up to 4 query heads); its
// token axis is cut into split-K chunks.  A workgroup stages the group's LUTs
// in LDS (for the q + codebook modes it builds them there on MFMA, entry for
// entry as pq_lut_kernel) and, for quantized values, the head's value
// codebook.  Per 32-token tile a wave sums M LUT entries per (token, head) into
// the score-MFMA layout, runs the fp32 online softmax and accumulates
// O^T += V^T P^T on MFMA, as the dense kernel does.  Quantized V is never
// materialised: the transposed PV reads address the codebook row of each
// lane's token directly; dense (bf16 / fp8) V rows are staged per tile.
// Modes 0 and 3 with G <= 8 and no outliers (contiguous or paged caches) run
// the grouped kernel (pq_group_kernel, below) instead; its mode 3 scores
// q . k_hat on MFMA from the staged key codebook rows rather than from LUT
// entries (within the attention tolerance, not bit-identical to the LUT path).
//
// Paged caches (block_table [B, max_blocks] int32, context_lens [B] int32):
// token t of sequence b is row t % bs of block block_table[b][t / bs]; the
// block index takes the place of the batch index in every cache stride.  The
// grid covers max_blocks * bs tokens and each workgroup stops at its
// sequence's length.  Outlier channels add sum_c q_out[b,h,c] * k_out[row,c]
// (fp32) to each LUT score; fp8 values are widened to bf16 while staged.
#include <string.h>

#include "dense_tile.h"

namespace bytes_amd {

constexpr int kPqWaves = 8;    // two waves per SIMD at one workgroup per CU
constexpr int kPqHeads = 4;     // query heads per unit (one 16-byte LUT entry holds all of them)
constexpr int kPqKMax = 256;    // codewords per subspace
constexpr int kPqOutMax = 16;   // outlier channels

struct PqArgs {
  const float* lut;          // mode LUT: [B, Hq, M, K]
  int64_t l_sb, l_sh;
  const uint16_t* q;         // mode dequant: q [B, Hq, D] bf16
  int64_t q_sb, q_sh;
  const _Float16* kcb;       // mode dequant: key codebook
  int64_t kcb_sh;            // elements between heads (0: shared)
  const uint8_t* kidx;
  int64_t ki_sb, ki_sh, ki_ss;
  const uint8_t* vidx;       // quantized V
  int64_t vi_sb, vi_sh, vi_ss;
  const _Float16* vcb;
  int64_t vcb_sh;
  const void* v;             // dense V [B, Hk, S, D] bf16 or fp8 e4m3fn
  int64_t v_sb, v_sh, v_ss;
  const void* kout;          // outlier keys [B, Hk, S, C] (bf16 / fp16 / fp32: ko_dt 0 / 1 / 2)
  int64_t ko_sb, ko_sh, ko_ss;
  const void* qout;          // outlier queries [B, Hq, C]
  int64_t qo_sb, qo_sh;
  int ko_dt, qo_dt, C;
  const int* btab;           // paged: block table [B, *] (row stride bt_sb), null: contiguous cache
  const int* clens;          // paged: sequence lengths [B]
  int64_t bt_sb;
  int bs, nblk;              // paged: rows per block, blocks in the cache
  int Hk, G, HG, S, K, chunk;   // S: tokens (paged: max_blocks * bs)
  float scale_log2;
  float lut_scale;           // LUTs built in the kernel: entries are lut_scale * (q . codeword)
  SplitKOut o;
};

__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  return dt == 0 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i])
                 : (dt == 1 ? (float)static_cast<const _Float16*>(p)[i] : static_cast<const float*>(p)[i]);
}

// Cache block and row of token t of sequence b.
__device__ __forceinline__ void pq_locate(const PqArgs& a, int b, int t, int& blk, int& row) {
  if (a.btab) {
    const int q = t / a.bs;
    blk = min(max(a.btab[(int64_t)b * a.bt_sb + q], 0), a.nblk - 1);
    row = t - q * a.bs;
  } else {
    blk = b;
    row = t;
  }
}

// Tokens of sequence b.
__device__ __forceinline__ int pq_len(const PqArgs& a, int b) {
  return a.btab ? max(0, min(a.clens[b], a.S)) : a.S;
}

// ---- LUT entries on MFMA ----
// Every kernel that builds LUT entries (pq_lut_kernel and the decodes that
// build their own) computes
//   lut[h][j][c] = (lut_scale * 2^k_h) * dot(q_h[8j .. 8j+7] * 2^-k_h, cb[j][c])
// where k_h = max(0, e_h - 15) for the head's largest |q| = 1.x * 2^e_h (the
// scaled row then fits fp16), and dot comes from v_mfma_f32_32x32x16_f16 on
// a block-diagonal pair of subspaces (j even, j + 1): rows 0-7 are up to 8
// heads against subspace j in k-slots 0-7, rows 16-23 the same heads against
// subspace j + 1 in slots 8-15 (other rows zero), and columns are 32
// consecutive codewords, so each lane reads one whole 16-byte codeword.  The
// A operand is hi = fp16(q'); a second MFMA accumulates lo = fp16(q' - hi)
// where any lane of the wave has a nonzero lo part (it adds exact zeros
// otherwise, so skipping it changes nothing).  Every product is exact
// (fp16 x fp16), q' = hi + lo exactly for |q'| >= 2^-17, and an entry depends
// only on its own head's q row and the slots its subspace takes: any grouping
// of heads gives the same bits.
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int lut_shift(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127;
  return (e >= 16 && e < 128) ? e - 15 : 0;
}

// Row and slot block of lane l's A operand: row m = l % 32 (head m % 16 of
// subspace j + m / 16 when m % 16 < 8), slots 8 * (l / 32) .. +7.  The lane
// holds values only where its row block matches its slot block.
__device__ __forceinline__ bool lut_a_live(int lane, int* head, int* sub) {
  const int m = lane & 31;
  *head = m & 15;
  *sub = m >> 4;
  return (m & 15) < 8 && (m >> 4) == (lane >> 5);
}

// hi and lo parts of eight scaled q values (zero where !live).
__device__ __forceinline__ void lut_a_operands(const float* x, bool live, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float v = live ? x[i] : 0.f;
    const _Float16 h = (_Float16)v;
    hi[i] = h;
    lo[i] = (_Float16)(v - (float)h);
  }
}

// B operand of codewords c0 .. c0+31 for subspace pair (j, j + 1): lane l
// holds codeword c0 + l % 32 of subspace j + l / 32 (codewords past K repeat
// codeword K - 1).
__device__ __forceinline__ f16x8 lut_b_operand(const _Float16* cb, int K, int j, int c0, int lane) {
  const int c = min(c0 + (lane & 31), K - 1);
  return __builtin_bit_cast(f16x8, ld16(cb + ((int64_t)(j + (lane >> 5)) * K + c) * 8));
}

// Entries of one subspace pair and 32 codewords: lane l receives heads
// 4 * (l / 32) + i of codeword c0 + l % 32 in e[i] (subspace j) and e[8 + i]
// (subspace j + 1), i = 0..3.
__device__ __forceinline__ f32x16 lut_mfma(f16x8 hi, f16x8 lo, bool use_lo, f16x8 b) {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  f32x16 e = __builtin_amdgcn_mfma_f32_32x32x16_f16(hi, b, z, 0, 0, 0);
  if (use_lo) e = __builtin_amdgcn_mfma_f32_32x32x16_f16(lo, b, e, 0, 0, 0);
  return e;
}

// True where any lane of the wave holds a nonzero lo part (wave-uniform).
__device__ __forceinline__ bool lut_need_lo(const f16x8& lo) {
  bool nz = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) nz = nz || (float)lo[i] != 0.f;
  return __ballot(nz) != 0;
}

// Scaled rows q' = q * 2^-k_h (fp32, qs[h][D]) and entry multipliers
// lut_scale * 2^k_h (mul[h]) of a workgroup's heads, in LDS: wave w takes
// row h = w.  The row is loaded first (lut_load_q, issued before any other
// request so that it heads the queue) and stored later (lut_store_q); rows at
// or past nh are zero with multiplier zero.  q0 points at head 0's row.
template <int D>
struct LutQ {
  uint32_t x[D / 64];      // raw bf16 bits, one value per word (rows past nh are zeroed where they are stored)
};

template <int D>
__device__ __forceinline__ LutQ<D> lut_load_q(const uint16_t* q0, int64_t q_sh, int h, int nh) {
  constexpr int PL = D / 64;
  const int lane = threadIdx.x & 63;
  const uint16_t* row = q0 + (int64_t)min(h, nh - 1) * q_sh + lane * PL;
  LutQ<D> r;
#pragma unroll
  for (int p = 0; p < PL; ++p) r.x[p] = row[p];
  return r;
}

template <int D>
__device__ __forceinline__ void lut_store_q(const LutQ<D>& r, int h, int nh, float lut_scale, float* qs,
                                            float* mul) {
  constexpr int PL = D / 64;
  const int lane = threadIdx.x & 63;
  float x[PL];
#pragma unroll
  for (int p = 0; p < PL; ++p) x[p] = h < nh ? __uint_as_float(r.x[p] << 16) : 0.f;
  float amax = 0.f;
#pragma unroll
  for (int p = 0; p < PL; ++p) amax = fmaxf(amax, fabsf(x[p]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, shfl_xor_f(amax, o));
  const int k = lut_shift(amax);
#pragma unroll
  for (int p = 0; p < PL; ++p) qs[h * D + lane * PL + p] = ldexpf(x[p], -k);
  if (lane == 0) mul[h] = h < nh ? ldexpf(lut_scale, k) : 0.f;
}

template <int D, bool QV>
struct PqCfg {
  static constexpr int M = D / 8;
  static constexpr int LUT = kPqHeads * M * kPqKMax * 4;          // fp32 LUTs of the unit's heads
  static constexpr int VCB = QV ? M * kPqKMax * 8 * 2 : 0;         // fp16 value codebook
  static constexpr int SCORES = kPqHeads * kTile * 4;              // one wave's tile scores
  // per wave: the tile scores, and (dense V) the V tile in the same buffer
  static constexpr int TILE = QV ? SCORES : kTile * D * 2;
  static constexpr int QOUT = QV ? 0 : kPqHeads * kPqOutMax * 4;    // fp32 outlier queries (dense-V modes)
  static constexpr int kSmem0 = LUT + VCB + kPqWaves * TILE + QOUT;
  static constexpr int kEpi = splitk_smem_floats<D, kPqWaves>() * 4;
  static constexpr int kSmem = kSmem0 > kEpi ? kSmem0 : kEpi;
};

// Codes and rows of one 32-token tile, in registers:
//  kc: the M key codes of tile row lane % 32 (every lane scores whole rows)
//  vc[i]: value code of row p / M, subspace p % M, for staging chunk p = lane + 64*i
//  vd[i]: dense V chunk p = lane + 64*i (row p / chunks-per-row), bf16 or fp8
//  ko: the outlier keys of tile row lane % 32
template <int D, bool QV, bool VF8, bool OUT>
struct PqRegs {
  static constexpr int CPR = VF8 ? D / 16 : D / 8;   // 16-byte V chunks per row
  static constexpr int CPL = kTile * CPR / 64;
  u32x4 kc;
  u32x4 vr[QV ? 2 : 1];   // quantized V: value codes of PV rows hf*16 + lg*4 + (l16 >> 2), hf = 0, 1
  u32x4 vd[QV ? 1 : CPL];
  float ko[OUT ? kPqOutMax : 1];
};

// Issue the tile at t0 (rows clamped to len - 1).  Each lane locates its own
// row lane % 32; rows of the V chunks come from the owning lane by shuffle.
template <int D, bool QV, bool VF8, bool OUT>
__device__ __forceinline__ void pq_issue(const PqArgs& a, int b, const uint8_t* kih, const uint8_t* vih,
                                         const char* vh, const char* koh, int len, int t0, int lane,
                                         PqRegs<D, QV, VF8, OUT>& r) {
  using R = PqRegs<D, QV, VF8, OUT>;
  constexpr int M = D / 8;
  int blk, row;
  pq_locate(a, b, min(t0 + (lane & 31), len - 1), blk, row);
  {
    const uint8_t* p = kih + (int64_t)blk * a.ki_sb + (int64_t)row * a.ki_ss;
    if constexpr (M == 16) {
      r.kc = ld16(p);
    } else {
      const u32x2 h = *reinterpret_cast<const u32x2*>(p);
      r.kc = u32x4{h[0], h[1], 0u, 0u};
    }
  }
  if constexpr (OUT) {
    // channels past C read channel C - 1; their query weights are zero
    const int64_t o = (int64_t)blk * a.ko_sb + (int64_t)row * a.ko_ss;
#pragma unroll
    for (int c = 0; c < kPqOutMax; ++c) r.ko[c] = load_any(koh, a.ko_dt, o + min(c, a.C - 1));
  }
  if constexpr (QV) {
    const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int rr = hf * 16 + lg * 4 + (l16 >> 2);
      const int bq = __shfl(blk, rr, 64), rq = __shfl(row, rr, 64);
      const uint8_t* p = vih + (int64_t)bq * a.vi_sb + (int64_t)rq * a.vi_ss;
      if constexpr (M == 16) {
        r.vr[hf] = ld16(p);
      } else {
        const u32x2 h = *reinterpret_cast<const u32x2*>(p);
        r.vr[hf] = u32x4{h[0], h[1], 0u, 0u};
      }
    }
  } else {
    constexpr int ES = VF8 ? 1 : 2;
#pragma unroll
    for (int i = 0; i < R::CPL; ++i) {
      const int p = lane + 64 * i;
      const int rr = p / R::CPR, pos = p - rr * R::CPR;
      const int bq = __shfl(blk, rr, 64), rq = __shfl(row, rr, 64);
      r.vd[i] = ld16(vh + ((int64_t)bq * a.v_sb + (int64_t)rq * a.v_ss) * ES + pos * 16);
    }
  }
}

// V elements (row, col .. col+3) of a quantized-V tile, read straight from
// the value codebook in LDS: subspace j = col / 8, codeword = the row's code
// j (the lane holds the codes of its two PV rows, hf = row / 16).
template <int D>
struct CodebookV {
  const char* vcb;
  const u32x4* vr;
  __device__ __forceinline__ const char* operator()(int hf, int row, int col) const {
    const int j = col >> 3;
    const uint32_t code = (vr[hf][j >> 2] >> ((j & 3) * 8)) & 0xFFu;
    return vcb + (((j * kPqKMax + (int)code) * 8) + (col & 7)) * 2;
  }
};

template <int D, bool QV, bool VF8, bool OUT>
__device__ __forceinline__ void pq_stage_dense_v(int lane, const PqRegs<D, QV, VF8, OUT>& r, char* vst) {
  using R = PqRegs<D, QV, VF8, OUT>;
#pragma unroll
  for (int i = 0; i < R::CPL; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / R::CPR, pos = p - rr * R::CPR;
    if constexpr (VF8) {
      u32x4 v0, v1;
      fp8x16_to_bf16(r.vd[i], v0, v1);
      *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, 2 * pos) * 16) = v0;
      *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, 2 * pos + 1) * 16) = v1;
    } else {
      *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, pos) * 16) = r.vd[i];
    }
  }
}

// One 32-row tile.  Scores: lane l sums the LUT entries of row l % 32 over
// half l/32 of the subspaces for the four heads at once (LUTs are kept
// [subspace][code][head], one 16-byte read per subspace), the halves are
// added, the wave passes the scores through its tile buffer into the
// score-MFMA layout (head l%16, rows blk*16 + lg*4 + i) and the softmax/PV
// step runs: quantized V straight from the codebook in LDS, dense V staged in
// the same buffer first.
template <int D, bool QV, bool VF8, bool OUT>
__device__ __forceinline__ void pq_tile(const PqArgs& a, const PqRegs<D, QV, VF8, OUT>& r, uint32_t vmask, int lane,
                                        int nh, const float* lut, const char* vcb, const float* qo, char* vst,
                                        float& m_run, float& l_run, f32x4 (&acc)[D / 16]) {
  constexpr int M = D / 8;
  const int l16 = lane & 15, lg = lane >> 4;
  float* sc_lds = reinterpret_cast<float*>(vst);   // [kPqHeads][32]
  // lane half hf sums subspaces hf*M/2 .. of its row for all four heads at
  // once (the LUT keeps a (subspace, code)'s heads adjacent); the halves are
  // added as (first + second) on both sides
  constexpr int MH = M / 2;
  const int hf = lane >> 5;
  f32x4 ps = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jj = 0; jj < MH; ++jj) {
    const uint32_t w = hf ? r.kc[MH / 4 + (jj >> 2)] : r.kc[jj >> 2];
    const uint32_t code = (w >> ((jj & 3) * 8)) & 0xFFu;
    ps += *reinterpret_cast<const f32x4*>(lut + ((hf * MH + jj) * kPqKMax + code) * kPqHeads);
  }
  f32x4 sc4;
#pragma unroll
  for (int h = 0; h < kPqHeads; ++h) {
    const float o = shfl_xor_f(ps[h], 32);
    sc4[h] = hf ? o + ps[h] : ps[h] + o;
    if constexpr (OUT) {
      float so = 0.f;
#pragma unroll
      for (int c = 0; c < kPqOutMax; ++c) so += qo[h * kPqOutMax + c] * r.ko[c];   // zero past C
      sc4[h] += so;
    }
  }
#pragma unroll
  for (int rep = 0; rep < 2; ++rep) {
    const int h = hf * 2 + rep;
    if (h < nh) sc_lds[h * kTile + (lane & 31)] = hf ? sc4[2 + rep] : sc4[rep];
  }
  wave_lds_sync();
  f32x4 s[2];
  const int hh = l16 < nh ? l16 : 0;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[blk][i] = sc_lds[hh * kTile + blk * 16 + lg * 4 + i];
  if constexpr (QV) {
    // V gathered from the codebook by the PV reads themselves
    tile_softmax_pv_at<D, true>(s, l16 < nh ? vmask : 0u, a.scale_log2, lane, CodebookV<D>{vcb, r.vr}, m_run, l_run,
                                acc);
  } else {
    // V tile into the same buffer
    wave_lds_sync();
    pq_stage_dense_v<D>(lane, r, vst);
    wave_lds_sync();
    tile_softmax_pv<D, false>(s, l16 < nh ? vmask : 0u, a.scale_log2, lane, vst, m_run, l_run, acc);
  }
}

// Copy n >= 1 16-byte chunks global -> LDS with the workgroup, 8 loads in
// flight per thread.  Chunks past n repeat chunk n - 1 (same value, same
// place): no load or store sits under a lane mask.
template <typename SRC, typename DST>
__device__ __forceinline__ void stage_chunks(int n, SRC src, DST dst) {
  constexpr int NT = kPqWaves * 64, BATCH = 8;
  for (int e0 = threadIdx.x; e0 < n; e0 += NT * BATCH) {
    u32x4 v[BATCH];
#pragma unroll
    for (int bb = 0; bb < BATCH; ++bb) v[bb] = ld16(src(min(e0 + bb * NT, n - 1)));
#pragma unroll
    for (int bb = 0; bb < BATCH; ++bb) *reinterpret_cast<u32x4*>(dst(min(e0 + bb * NT, n - 1))) = v[bb];
  }
}

template <int D, bool BUILD_LUT, bool QV, bool VF8, bool OUT>
__global__ __launch_bounds__(kPqWaves * 64, 1) void pq_decode_kernel(PqArgs a) {
  using C = PqCfg<D, QV>;
  using Regs = PqRegs<D, QV, VF8, OUT>;
  constexpr int M = D / 8;
  __shared__ __attribute__((aligned(16))) char smem_raw[C::kSmem];
  float* lut = reinterpret_cast<float*>(smem_raw);
  char* vcb = smem_raw + C::LUT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const UnitLoc loc = splitk_locate(a.o);     // head blocks of kPqHeads: o.HB = HG
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk, hg = loc.hb;
  const int hq0 = hk * a.G + hg * kPqHeads;
  const int nh = min(kPqHeads, a.G - hg * kPqHeads);

  const int len = pq_len(a, b);
  const int t_begin = split * a.chunk;
  const int t_end = min(t_begin + a.chunk, len);
  // per-head bases; the row offsets (batch or block, row) are added per token
  const uint8_t* kih = a.kidx + (int64_t)hk * a.ki_sh;
  const uint8_t* vih = QV ? a.vidx + (int64_t)hk * a.vi_sh : nullptr;
  const char* vh = QV ? nullptr : static_cast<const char*>(a.v) + (int64_t)hk * a.v_sh * (VF8 ? 1 : 2);
  const char* koh = OUT ? static_cast<const char*>(a.kout) + (int64_t)hk * a.ko_sh * (a.ko_dt == 2 ? 4 : 2)
                        : nullptr;
  char* vst = smem_raw + C::LUT + C::VCB + w * C::TILE;
  constexpr int STEP = kPqWaves * kTile;
  int t = t_begin + w * kTile;
  const bool any = t < t_end;          // wave-uniform; tiles past the end are issued clamped (len >= 1 then)

  // The first tile's codes are requested before the LUTs are staged, so they
  // arrive meanwhile.  Every later request is unconditional (rows clamped to
  // len - 1 past the end), so each wait counts the same requests.
  LutQ<D> qrow;
  if (BUILD_LUT && w < kPqHeads) qrow = lut_load_q<D>(a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh, a.q_sh, w, nh);
  Regs r;
  if (any) pq_issue<D, QV, VF8, OUT>(a, b, kih, vih, vh, koh, len, t, lane, r);

  // The value codebook (quantized V) is requested now, with the first tile's
  // codes, so it arrives while the LUTs are built or staged; it is stored to
  // LDS after them (chunks past M*K repeat the last one).
  const int K = a.K;
  constexpr int VPT = (M * kPqKMax + kPqWaves * 64 - 1) / (kPqWaves * 64);   // codebook chunks per thread
  u32x4 vraw[QV ? VPT : 1];
  const _Float16* vcbh = QV ? a.vcb + (int64_t)hk * a.vcb_sh : nullptr;
  if constexpr (QV) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) vraw[i] = ld16(vcbh + (int64_t)min((int)threadIdx.x + kPqWaves * 64 * i, M * K - 1) * 8);
  }

  // ---- stage the group's LUTs ----
  if (BUILD_LUT) {
    // the unit's LUT entries on MFMA (see lut_a_live): wave w builds
    // subspace pair 2w, 2w + 1 (waves past M/2 idle); its codeword operands
    // are requested before the scaled q rows are staged (in the tile buffers,
    // unused until the tile loop)
    static_assert(kPqWaves * C::TILE >= kPqHeads * D * 4 + kPqHeads * 4, "q rows fit in the tile buffers");
    const _Float16* cb = a.kcb + (int64_t)hk * a.kcb_sh;
    const int jp = min(2 * w, M - 2);
    f16x8 bop[kPqKMax / 32];
#pragma unroll
    for (int c32 = 0; c32 < kPqKMax / 32; ++c32) bop[c32] = lut_b_operand(cb, K, jp, c32 * 32, lane);
    float* qs = reinterpret_cast<float*>(smem_raw + C::LUT + C::VCB);
    float* mul = qs + kPqHeads * D;
    if (w < kPqHeads) lut_store_q<D>(qrow, w, nh, a.lut_scale, qs, mul);
    __syncthreads();
    if (2 * w < M) {
      int hm, sub;
      const bool live = lut_a_live(lane, &hm, &sub) && hm < kPqHeads;
      f16x8 hi, lo;
      lut_a_operands(qs + min(hm, kPqHeads - 1) * D + 8 * (jp + sub), live, hi, lo);
      const bool use_lo = lut_need_lo(lo);
      const float mul4[4] = {mul[0], mul[1], mul[2], mul[3]};
      const int n = lane & 31;
#pragma unroll
      for (int c32 = 0; c32 < kPqKMax / 32; ++c32) {
        const f32x16 e = lut_mfma(hi, lo, use_lo, bop[c32]);
        // lanes 0..31 hold heads 0..3 of codeword c32 * 32 + n for subspaces jp, jp + 1
        if (lane < 32) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
            *reinterpret_cast<f32x4*>(lut + ((jp + s2) * kPqKMax + c32 * 32 + n) * kPqHeads) =
                f32x4{mul4[0] * e[8 * s2], mul4[1] * e[8 * s2 + 1], mul4[2] * e[8 * s2 + 2], mul4[3] * e[8 * s2 + 3]};
        }
      }
    }
  } else {
    // the caller's LUTs, transposed so the heads of one (subspace, code) are
    // adjacent; chunks past n repeat the last one (same values, same place)
    const int K4 = K / 4, n = nh * M * K4;
    constexpr int NT = kPqWaves * 64, BATCH = 8;
    for (int e0 = threadIdx.x; e0 < n; e0 += NT * BATCH) {
      u32x4 v[BATCH];
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int e = min(e0 + bb * NT, n - 1);
        const int h = e / (M * K4), r2 = e - h * (M * K4);
        const int j = r2 / K4, c4 = r2 - j * K4;
        v[bb] = ld16(a.lut + (int64_t)b * a.l_sb + (int64_t)(hq0 + h) * a.l_sh + j * K + c4 * 4);
      }
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int e = min(e0 + bb * NT, n - 1);
        const int h = e / (M * K4), r2 = e - h * (M * K4);
        const int j = r2 / K4, c4 = r2 - j * K4;
#pragma unroll
        for (int x = 0; x < 4; ++x) lut[(j * kPqKMax + c4 * 4 + x) * kPqHeads + h] = __uint_as_float(v[bb][x]);
      }
    }
  }
  if constexpr (QV) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = min((int)threadIdx.x + kPqWaves * 64 * i, M * K - 1);
      const int j = e / K, c = e - j * K;
      *reinterpret_cast<u32x4*>(vcb + ((j * kPqKMax + c) * 8) * 2) = vraw[i];
    }
  }
  float* qo = reinterpret_cast<float*>(smem_raw + C::LUT + C::VCB + kPqWaves * C::TILE);
  if constexpr (OUT) {
    for (int e = threadIdx.x; e < kPqHeads * kPqOutMax; e += kPqWaves * 64) {
      const int h = e / kPqOutMax, c = e - h * kPqOutMax;
      qo[e] = (h < nh && c < a.C) ? load_any(a.qout, a.qo_dt, (int64_t)b * a.qo_sb + (int64_t)(hq0 + h) * a.qo_sh + c)
                                  : 0.f;
    }
  }

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  __syncthreads();
  if (any) {
    // tile t runs on the registers that arrived during the last tile, which
    // are copied out first and refilled with tile t+STEP (clamped past the end)
    for (; t < t_end; t += STEP) {
      const Regs cur = r;
      pq_issue<D, QV, VF8, OUT>(a, b, kih, vih, vh, koh, len, t + STEP, lane, r);
      wave_lds_sync();
      pq_tile<D, QV, VF8, OUT>(a, cur, range_mask(t, t_end), lane, nh, lut, vcb, qo, vst, m_run, l_run, acc);
    }
  }
  splitk_epilogue<D, kPqWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b, hq0, nh,
                               kDmapDense);
}

// ============================================================================
// Grouped decode for quantized values (modes 0 and 3, G <= 8): a unit is
// (b, kv head) with all G of its query heads, so every token's codes are read
// once and its per-token work is shared by the whole group.  A workgroup takes
// a chunk of <= kPqgChunk tokens; phases A and B reuse one LDS region:
//   A. scores of every (token, head) of the chunk, by one of two routes:
//      SRC 0 (the caller's LUT): the unit's LUTs (fp32, [head quad][subspace]
//      [code][4 heads]: a code's entries for four heads are one 16-byte read,
//      and a wave's reads of random codes spread over all 16 16-byte bank
//      slots) are resident; thread i scores token i for every head, summing
//      the M entries in subspace order;
//      SRC 2 (q and the key codebook): the key codebook is resident and the
//      scores are q . k_hat on v_mfma_f32_16x16x32_f16, whose A operand (a
//      token's 8 channels of one subspace) is exactly the codeword its code
//      selects: each lane reads that 16-byte codebook row, no LUT is formed;
//      q enters as the B operand in the LUT's scaled hi/lo form, so every
//      product is exact and the sums run in fp32;
//      the scores and the tokens' value codes are stored;
//   B. the value codebook replaces the LUTs.  The chunk's per-head maximum is
//      known, so each wave turns its 32-token tiles straight into fp16
//      probabilities (no running rescale), stored in MFMA operand order; then
//      each wave accumulates two 16-column blocks of the output over a group
//      of tiles (O^T += V^T P^T, the V operand read from the codebook by
//      transposed LDS reads), the tile groups are added in group order, and
//      each column block is written to the split's partial (or the output).
// ============================================================================
constexpr int kPqgThreads = kPqWaves * 64;
constexpr int kPqgChunk = kPqgThreads;    // tokens per workgroup: one per thread in phase A

template <int D, int HP>
struct PqgCfg {
  static constexpr int M = D / 8;
  static constexpr int NT = kPqgChunk / kTile;                 // tiles per chunk
  static constexpr int LUT = M * kPqKMax * HP * 4;             // A: fp32 LUTs [HP/4][M][256][4]
  static constexpr int VCB = M * kPqKMax * 8 * 2;              // B: fp16 value codebook
  static constexpr int PS = NT * 64 * 16;                      // B: fp16 probabilities, [tile][lane] x 8
  static constexpr int A2 = (kPqWaves - D / 32) * 2 * 64 * 16;  // B: accumulators of tile groups past 0
  static constexpr int X = LUT > VCB + PS + A2 ? LUT : VCB + PS + A2;
  static constexpr int KCB = M * kPqKMax * 8 * 2;              // A (SRC 2): fp16 key codebook
  static_assert(KCB <= LUT, "the key codebook fits the LUT area");
  static_assert(kPqgChunk * 16 + HP * D * 4 <= PS, "SRC 2 staging: key codes and q rows fit the probability area");
  static constexpr int SC = HP * kPqgChunk * 4;                // scores [HP][chunk]
  static constexpr int VC = kPqgChunk * M;                     // value codes [chunk][M]
  static constexpr int HS = 16 * 4;                            // per-head multipliers, then maxima
  static constexpr int LS = kPqWaves * 16 * 4;                 // per-wave probability sums
  static constexpr int kSmem = X + SC + VC + HS + LS;
  static_assert(HP * D * 4 <= SC, "q rows fit in the score area");
};

// M code bytes of one row (16 or 8 bytes, aligned), streamed non-temporally
// (consecutive threads read consecutive rows).
template <int M>
__device__ __forceinline__ u32x4 ld_codes(const uint8_t* p) {
  if constexpr (M == 16) {
    return ld16_nt(p);
  } else {
    const u32x2 h = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return u32x4{h[0], h[1], 0u, 0u};
  }
}

template <int D, int SRC, int HP, bool PAGED>
__global__ __launch_bounds__(kPqgThreads, 1) void pq_group_kernel(PqArgs a) {
  static_assert(SRC == 0 || SRC == 2, "scores from the caller's LUT or from q and the key codebook");
  using C = PqgCfg<D, HP>;
  constexpr int M = D / 8;
  __shared__ __attribute__((aligned(16))) char smem[C::kSmem];
  float* lut = reinterpret_cast<float*>(smem);
  char* vcb = smem;
  f16x8* ps = reinterpret_cast<f16x8*>(smem + C::VCB);
  float* sc = reinterpret_cast<float*>(smem + C::X);
  uint8_t* vc = reinterpret_cast<uint8_t*>(smem + C::X + C::SC);
  float* hsm = reinterpret_cast<float*>(smem + C::X + C::SC + C::VC);
  float* lsum = hsm + 16;
  f32x4* acc2 = reinterpret_cast<f32x4*>(smem + C::VCB + C::PS);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const UnitLoc loc = splitk_locate(a.o);     // o.HB = 1: unit = b * Hk + hk
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk;
  const int G = a.G, hq0 = hk * G, K = a.K;
  const int len = PAGED ? pq_len(a, b) : a.S;       // a contiguous cache needs no length load
  const int t_begin = split * a.chunk;
  const int n = max(0, min(a.chunk, len - t_begin));   // tokens of this chunk

  // wave w's q row heads the queue; then this thread's token (clamped into
  // the chunk), whose codes arrive while the LUTs are built or staged
  LutQ<D> qrow;
  if constexpr (SRC == 2) qrow = lut_load_q<D>(a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh, a.q_sh, min(w, HP - 1), G);
  u32x4 kc, vcd;
  {
    int blk, row;
    if constexpr (PAGED) {
      pq_locate(a, b, t_begin + min(tid, max(n - 1, 0)), blk, row);
    } else {
      blk = b;
      row = t_begin + min(tid, max(n - 1, 0));
    }
    kc = ld_codes<M>(a.kidx + (int64_t)hk * a.ki_sh + (int64_t)blk * a.ki_sb + (int64_t)row * a.ki_ss);
    vcd = ld_codes<M>(a.vidx + (int64_t)hk * a.vi_sh + (int64_t)blk * a.vi_sb + (int64_t)row * a.vi_ss);
  }

  // ---- phase A: the key codebook (SRC 2) or the LUTs (SRC 0) ----
  char* kcbl = smem;                                          // SRC 2: key codebook [M][256][8] fp16
  uint8_t* kcl = reinterpret_cast<uint8_t*>(smem + C::VCB);   // SRC 2: key codes [chunk][16]
  float* qs = reinterpret_cast<float*>(smem + C::VCB + kPqgChunk * 16);   // SRC 2: scaled q rows [HP][D]
  if constexpr (SRC == 2) {
    // codebook slot s = (j, c) of 256 per subspace (codewords past K repeat
    // codeword K - 1; no code reads them), all loads in flight at once
    constexpr int KPT = M * kPqKMax / kPqgThreads;
    const _Float16* cb = a.kcb + (int64_t)hk * a.kcb_sh;
    u32x4 kraw[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int sl = tid + kPqgThreads * i;
      kraw[i] = ld16(cb + (int64_t)((sl >> 8) * K + min(sl & 255, K - 1)) * 8);
    }
    if (w < HP) lut_store_q<D>(qrow, w, G, a.lut_scale, qs, hsm);
#pragma unroll
    for (int i = 0; i < KPT; ++i) *reinterpret_cast<u32x4*>(kcbl + (tid + kPqgThreads * i) * 16) = kraw[i];
    *reinterpret_cast<u32x4*>(kcl + tid * 16) = kc;
  } else {
    // the caller's LUTs [B, Hq, M, K]: slot s = (j, c) of 256 per subspace,
    // consecutive codes across lanes (each load instruction reads 256
    // contiguous bytes of one head's row), all HP x M*256/threads loads in
    // flight; codes past K repeat code K - 1, heads past G repeat head G - 1
    constexpr int SPT = M * kPqKMax / kPqgThreads;
    const float* lb = a.lut + (int64_t)b * a.l_sb + (int64_t)hq0 * a.l_sh;
    float v[SPT][HP];
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int sl = tid + kPqgThreads * i;
      const int off = (sl >> 8) * K + min(sl & 255, K - 1);
#pragma unroll
      for (int h = 0; h < HP; ++h) v[i][h] = lb[(int64_t)min(h, G - 1) * a.l_sh + off];
    }
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int sl = tid + kPqgThreads * i;
#pragma unroll
      for (int h4 = 0; h4 < HP / 4; ++h4)
        *reinterpret_cast<f32x4*>(lut + ((h4 * M + (sl >> 8)) * kPqKMax + (sl & 255)) * 4) =
            f32x4{v[i][4 * h4], v[i][4 * h4 + 1], v[i][4 * h4 + 2], v[i][4 * h4 + 3]};
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // the value codebook, held in registers until phase B (requested after the
  // LUT operands so it arrives during phase A): slot s = (j, c) of 256 per
  // subspace (codewords past K repeat codeword K - 1; no code reads them)
  constexpr int VPT = M * kPqKMax / kPqgThreads;
  static_assert(VPT * kPqgThreads == M * kPqKMax, "codebook slots per thread");
  const _Float16* vcbh = a.vcb + (int64_t)hk * a.vcb_sh;
  u32x4 vraw[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int sl = tid + kPqgThreads * i;
    vraw[i] = ld16(vcbh + (int64_t)((sl >> 8) * K + min(sl & 255, K - 1)) * 8);
  }
  __syncthreads();

  // ---- phase A: scores ----
  if constexpr (SRC == 2) {
    // wave w scores 16-token blocks w, w + 8, ..: lane (l16, lg) supplies the
    // codeword of subspace 4*kk + lg of token 16*blk + l16 (A) and q of head
    // l16 at channels 32*kk + 8*lg .. +7 (B); the MFMA leaves head l16's
    // scores of tokens 16*blk + 4*lg + i in lane (l16, lg).  Every LDS read
    // of the wave's blocks is issued before the first MFMA.
    const int l16 = lane & 15, lg = lane >> 4;
    constexpr int KS = M / 4;                                   // MFMA k-steps
    constexpr int NB = kPqgChunk / 16 / kPqWaves;               // blocks per wave
    const bool hlive = l16 < HP;
    const float* qrow = qs + min(l16, HP - 1) * D + lg * 8;
    f16x8 qhi[KS], qlo[KS];
    bool nzl = false;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(qrow + kk * 32);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(qrow + kk * 32 + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = hlive ? (i < 4 ? x0[i] : x1[i - 4]) : 0.f;
        const _Float16 hv = (_Float16)v;
        qhi[kk][i] = hv;
        qlo[kk][i] = (_Float16)(v - (float)hv);
        nzl = nzl || (float)qlo[kk][i] != 0.f;
      }
    }
    const bool nz = __ballot(nzl) != 0;
    const float mul = hsm[min(l16, HP - 1)];
    u32x4 cw[NB];
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
      cw[bi] = *reinterpret_cast<const u32x4*>(kcl + ((w + kPqWaves * bi) * 16 + l16) * 16);   // the token's codes
    f16x8 cwd[NB][KS];
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const uint32_t code = (cw[bi][kk] >> (8 * lg)) & 0xFFu;       // subspace 4*kk + lg
        cwd[bi][kk] = *reinterpret_cast<const f16x8*>(kcbl + ((4 * kk + lg) * kPqKMax + (int)code) * 16);
      }
    f32x4 acc[NB];
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) acc[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nz) {
#pragma unroll
      for (int bi = 0; bi < NB; ++bi)
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          acc[bi] = mfma_f16(cwd[bi][kk], qhi[kk], acc[bi]);
          acc[bi] = mfma_f16(cwd[bi][kk], qlo[kk], acc[bi]);
        }
    } else {
#pragma unroll
      for (int bi = 0; bi < NB; ++bi)
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) acc[bi] = mfma_f16(cwd[bi][kk], qhi[kk], acc[bi]);
    }
    if (hlive) {
#pragma unroll
      for (int bi = 0; bi < NB; ++bi) {
        const int t0 = (w + kPqWaves * bi) * 16 + lg * 4;
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = t0 + i < n ? mul * acc[bi][i] : kNegInf;
        *reinterpret_cast<f32x4*>(sc + l16 * kPqgChunk + t0) = o;
      }
    }
    if constexpr (M == 16) {
      *reinterpret_cast<u32x4*>(vc + tid * M) = vcd;
    } else {
      *reinterpret_cast<u32x2*>(vc + tid * M) = u32x2{vcd[0], vcd[1]};
    }
  } else {
    float s[HP];
#pragma unroll
    for (int h = 0; h < HP; ++h) s[h] = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const uint32_t code = (kc[j >> 2] >> ((j & 3) * 8)) & 0xFFu;
#pragma unroll
      for (int h4 = 0; h4 < HP / 4; ++h4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(lut + ((h4 * M + j) * kPqKMax + (int)code) * 4);
#pragma unroll
        for (int x = 0; x < 4; ++x) s[4 * h4 + x] += v[x];
      }
    }
    const bool live = tid < n;
#pragma unroll
    for (int h = 0; h < HP; ++h) sc[h * kPqgChunk + tid] = live ? s[h] : kNegInf;
    if constexpr (M == 16) {
      *reinterpret_cast<u32x4*>(vc + tid * M) = vcd;
    } else {
      *reinterpret_cast<u32x2*>(vc + tid * M) = u32x2{vcd[0], vcd[1]};
    }
  }
  __syncthreads();

  // ---- phase B: the value codebook over the LUTs; per-head chunk maxima ----
#pragma unroll
  for (int i = 0; i < VPT; ++i) *reinterpret_cast<u32x4*>(vcb + (tid + kPqgThreads * i) * 16) = vraw[i];
  if (w < HP) {
    float m = kNegInf;
#pragma unroll
    for (int i = 0; i < kPqgChunk / 64; ++i) m = fmaxf(m, sc[w * kPqgChunk + lane + 64 * i] * a.scale_log2);
    m = wave_max_f32(m);
    if (lane == 0) hsm[w] = m;
  }
  __syncthreads();

  // B0: fp16 probabilities of tiles w, w + 8 in P^T operand order (head l16,
  // tokens t0 + blk*16 + lg*4 + i at position blk*4 + i); tokens past n have
  // score -inf and so probability zero
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = l16 < HP ? l16 : 0;
  const bool col = l16 < G;
  const float m_run = hsm[hh];
  const float m_use = m_run == kNegInf ? 0.f : m_run;
  constexpr int NT = C::NT;
  {
    float l_part = 0.f;
#pragma unroll
    for (int tile = w; tile < NT; tile += kPqWaves) {
      f16x8 ph;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc + hh * kPqgChunk + tile * kTile + blk * 16 + lg * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = col ? fast_exp2(s4[i] * a.scale_log2 - m_use) : 0.f;
          l_part += p;
          ph[blk * 4 + i] = (_Float16)p;
        }
      }
      ps[tile * 64 + lane] = ph;
    }
    l_part = col_sum4(l_part);
    if (lg == 0) lsum[w * 16 + l16] = l_part;
  }
  __syncthreads();

  // B1: wave w accumulates output column blocks db = 2*dp, 2*dp + 1
  // (dp = w % DP) over tiles tq, tq + TS, .. (tq = w / DP); for block db
  // the lane supplies V rows of codeword subspace 2*db + (l16 & 3) / 2 to the
  // transposed reads (columns db*16 + (l16 & 3)*4 .. +3); both subspaces'
  // codes sit in byte 2*e + (l16 & 3) / 2 of value-code word dp
  constexpr int DP = D / 32, TS = kPqWaves / DP;
  const int dp = w % DP, tq = w / DP;
  const int sub = (l16 & 3) >> 1;
  const char* vb0 = vcb + ((4 * dp + sub) * kPqKMax * 8 + (l16 & 1) * 4) * 2;
  const char* vb1 = vb0 + 2 * kPqKMax * 8 * 2;
  const uint8_t* vcw = vc + dp * 4;
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // every tile's code words and probabilities are read, then every codeword
  // row, then the MFMAs run: two LDS round trips for the wave's tiles
  // instead of two per tile
  constexpr int KT = NT / TS;
  uint32_t word[KT][2];
  f16x8 ph[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int tile = tq + k * TS;
    ph[k] = ps[tile * 64 + lane];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
      word[k][hf] = *reinterpret_cast<const uint32_t*>(vcw + (tile * kTile + hf * 16 + lg * 4 + (l16 >> 2)) * M);
  }
  u32x2 hv[KT][2][2];
#pragma unroll
  for (int k = 0; k < KT; ++k)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      hv[k][0][hf] = tr16(vb0 + ((word[k][hf] >> (8 * sub)) & 0xFFu) * 16);
      hv[k][1][hf] = tr16(vb1 + ((word[k][hf] >> (8 * (2 + sub))) & 0xFFu) * 16);
    }
#pragma unroll
  for (int k = 0; k < KT; ++k)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const u32x4 raw = {hv[k][e][0][0], hv[k][e][0][1], hv[k][e][1][0], hv[k][e][1][1]};
      acc[e] = mfma_f16(__builtin_bit_cast(f16x8, raw), ph[k], acc[e]);
    }
  // the tile groups' sums join group 0's, in group order
  if (tq > 0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) acc2[(((tq - 1) * DP + dp) * 2 + e) * 64 + lane] = acc[e];
  }
  __syncthreads();

  // B2: acc[e][i] = O^T[d = (2*dp + e)*16 + lg*4 + i][head l16]; the head's
  // sum over the waves' probability sums, in wave order
  if (tq == 0 && col) {
#pragma unroll
    for (int t2 = 1; t2 < TS; ++t2)
#pragma unroll
      for (int e = 0; e < 2; ++e) acc[e] += acc2[(((t2 - 1) * DP + dp) * 2 + e) * 64 + lane];
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < kPqWaves; ++ww) L += lsum[ww * 16 + l16];
    const SplitKOut& o = a.o;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int d0 = (2 * dp + e) * 16 + lg * 4;
      if (o.nsplit <= 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) store_out(o, b, hq0 + l16, d0 + i, acc[e][i] / L);
      } else {
        const size_t r = ((size_t)unit * 16 + l16) * o.nsplit + split;
        *reinterpret_cast<f32x4*>(o.part_acc + r * D + d0) = acc[e];
        if (dp == 0 && e == 0 && lg == 0) {
          o.part_ml[r * 2 + 0] = m_run;
          o.part_ml[r * 2 + 1] = L;
        }
      }
    }
  }
}

// ============================================================================
// Per-wave grouped decode (mode 3 on contiguous caches, G <= 8; the C3 step):
// a unit is (b, kv head) with all G query heads, a workgroup a chunk of
// <= kPqgChunk tokens and wave w the chunk's tokens [64w, 64w + 64).  Both
// codebooks (64 KB each at D = 128) go HBM/L2 -> LDS by LDS-DMA, the wave's
// key and value codes into registers; once the key codebook is published
// every wave runs on its own (a second barrier publishes the value codebook,
// which streams in under the scores): scores q . k_hat on MFMA exactly as pq_group_kernel's
// SRC 2 (the same scaled hi/lo q and MFMA order, so the same fp32 scores),
// the softmax of its 64 tokens in registers (the probabilities never leave
// them: the score MFMA's output layout is the P^T operand layout of the PV
// MFMA), and PV over all D columns from transposed reads of the value
// codebook.  The waves' states then merge in the split-K epilogue.  Against
// pq_group_kernel this drops the LDS round trips of scores, probabilities
// and per-head maxima and three of its five workgroup barriers.
// ============================================================================
template <int D>
struct PqwCfg {
  static constexpr int M = D / 8;
  static constexpr int CB = M * kPqKMax * 16;                  // one fp16 codebook [M][256][8]
  static constexpr int CPT = M * kPqKMax / kPqgThreads;        // codebook rows per thread
  static constexpr int kEpi = splitk_smem_floats<D, kPqWaves>() * 4;
  static constexpr int kSmem = 2 * CB > kEpi ? 2 * CB : kEpi;
  static_assert(kPqgChunk == kPqWaves * 64, "64 tokens per wave");
  static_assert(CPT * kPqgThreads == M * kPqKMax, "whole codebook rows per thread");
};

template <int D>
__global__ __launch_bounds__(kPqgThreads, 1) void pq_wave_kernel(PqArgs a) {
  using C = PqwCfg<D>;
  constexpr int M = D / 8;
  constexpr int KS = M / 4;                 // score MFMA k-steps (4 subspaces each)
  constexpr int DB = D / 16;                // output column blocks
  __shared__ __attribute__((aligned(16))) char smem[C::kSmem];
  char* kcbl = smem;
  char* vcbl = smem + C::CB;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const UnitLoc loc = splitk_locate(a.o);     // o.HB = 1: unit = b * Hk + hk
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk;
  const int G = a.G, hq0 = hk * G, K = a.K;
  const int t_begin = split * a.chunk;
  const int n = max(0, min(a.chunk, a.S - t_begin));
  const int tw = 64 * w;

  // Requests, oldest first: the key codebook (LDS-DMA), the q rows and codes
  // (VGPRs), the value codebook (LDS-DMA into its own region).  The scores
  // need all but the value codebook, which arrives while they are computed
  // (into LDS: returns into VGPRs measured to slow the tiles they overlap);
  // the compiler, which does not see the LDS-DMA requests, counts the later
  // requests short and so waits at most longer than needed.  Codebook row
  // s = (j, c) of 256 per subspace sits at s * 16 in LDS (codewords past K
  // repeat codeword K - 1; no code reads them).
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(a.kcb + (int64_t)hk * a.kcb_sh, (uint32_t)(M * K * 16));
  auto cb_off = [&](int i) {
    const int sl = tid + kPqgThreads * i;
    return (uint32_t)(((sl >> 8) * K + min(sl & 255, K - 1)) * 16);
  };
#pragma unroll
  for (int i = 0; i < C::CPT; ++i) lds_dma16<false>(rk, kcbl + (kPqgThreads * i + 64 * w) * 16, cb_off(i));
  // q of head l16 (columns past G take head 0 and are zeroed below), lane
  // (l16, lg) holding channels 32 kk + 8 lg .. +7: the score B operand
  u32x4 qraw[KS];
  {
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hq0 + (l16 < G ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qraw[kk] = ld16(qp + kk * 32);
  }
  // codes, clamped into the chunk: key codes of tokens tw + 16 bi + l16 (score
  // A operands) and value codes of tokens tw + 32 k + 16 hf + 4 lg + l16 / 4
  // (PV transposed reads)
  const uint8_t* kb = a.kidx + (int64_t)b * a.ki_sb + (int64_t)hk * a.ki_sh;
  const uint8_t* vb = a.vidx + (int64_t)b * a.vi_sb + (int64_t)hk * a.vi_sh;
  auto crow = [&](int t) { return (int64_t)(t_begin + min(t, max(n - 1, 0))); };
  u32x4 kc[4], vcw[2][2];
#pragma unroll
  for (int bi = 0; bi < 4; ++bi) kc[bi] = ld_codes<M>(kb + crow(tw + 16 * bi + l16) * a.ki_ss);
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
      vcw[k][hf] = ld_codes<M>(vb + crow(tw + 32 * k + 16 * hf + 4 * lg + (l16 >> 2)) * a.vi_ss);
  __builtin_amdgcn_sched_barrier(0);
  {
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc_uniform(a.vcb + (int64_t)hk * a.vcb_sh, (uint32_t)(M * K * 16));
#pragma unroll
    for (int i = 0; i < C::CPT; ++i) lds_dma16<false>(rv, vcbl + (kPqgThreads * i + 64 * w) * 16, cb_off(i));
  }
  __builtin_amdgcn_sched_barrier(0);

  // q scaled by 2^-k_h so the row fits fp16 (k_h from the row's largest |q|,
  // the four lanes of head l16 holding the row), split into hi + lo fp16
  // parts: the LUT contract's operands (lut_store_q, pq_group_kernel SRC 2)
  const bool hlive = l16 < G;
  float amax = 0.f;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(bf16_bits_to_f32((uint16_t)(qraw[kk][i >> 1] >> (16 * (i & 1))))));
  amax = col_max4(amax);
  const int kh = lut_shift(amax);
  const float mul = hlive ? ldexpf(a.lut_scale, kh) : 0.f;
  f16x8 qhi[KS], qlo[KS];
  bool nzl = false;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = hlive ? ldexpf(bf16_bits_to_f32((uint16_t)(qraw[kk][i >> 1] >> (16 * (i & 1)))), -kh) : 0.f;
      const _Float16 hv = (_Float16)v;
      qhi[kk][i] = hv;
      qlo[kk][i] = (_Float16)(v - (float)hv);
      nzl = nzl || (float)qlo[kk][i] != 0.f;
    }
  const bool nz = __ballot(nzl) != 0;

  // every request but the value codebook's has returned (in order): the key
  // codebook is in LDS, and the barrier publishes it
  static_assert(C::CPT <= 15, "the value codebook's requests fit the wait count");
  __builtin_amdgcn_s_waitcnt(0x0F70 | C::CPT);      // vmcnt(CPT)
  lds_barrier();

  // ---- scores of the wave's 4 blocks of 16 tokens: head l16's scores of
  // tokens tw + 16 bi + 4 lg + i in s[bi][i] ----
  f16x8 cwd[4][KS];
#pragma unroll
  for (int bi = 0; bi < 4; ++bi)
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const uint32_t code = (kc[bi][kk] >> (8 * lg)) & 0xFFu;       // subspace 4 kk + lg
      cwd[bi][kk] = *reinterpret_cast<const f16x8*>(kcbl + ((4 * kk + lg) * kPqKMax + (int)code) * 16);
    }
  f32x4 s[4];
#pragma unroll
  for (int bi = 0; bi < 4; ++bi) s[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (nz) {
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        s[bi] = mfma_f16(cwd[bi][kk], qhi[kk], s[bi]);
        s[bi] = mfma_f16(cwd[bi][kk], qlo[kk], s[bi]);
      }
  } else {
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) s[bi] = mfma_f16(cwd[bi][kk], qhi[kk], s[bi]);
  }

  // ---- softmax of the wave's tokens (log2 domain; tokens past n: -inf) ----
  float mx = kNegInf;
#pragma unroll
  for (int bi = 0; bi < 4; ++bi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = tw + 16 * bi + 4 * lg + i < n ? (mul * s[bi][i]) * a.scale_log2 : kNegInf;
      s[bi][i] = x;
      mx = fmaxf(mx, x);
    }
  const float m_run = col_max4(mx);
  const float m_use = m_run == kNegInf ? 0.f : m_run;
  float l_run = 0.f;
  f16x8 ph[2];
#pragma unroll
  for (int bi = 0; bi < 4; ++bi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = hlive ? fast_exp2(s[bi][i] - m_use) : 0.f;
      l_run += p;
      ph[bi >> 1][(bi & 1) * 4 + i] = (_Float16)p;
    }

  // ---- the value codebook in LDS (its requests done); publish it ----
  __builtin_amdgcn_s_waitcnt(0x0F70);               // vmcnt(0)
  lds_barrier();

  // ---- PV: O^T[d][h] += V^T[d][t] P^T[t][h] over the wave's two 32-token
  // tiles; block db's rows come from codeword subspaces 2 db + sub ----
  f32x4 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int sub = (l16 & 3) >> 1;
  const char* vrow = vcbl + (sub * kPqKMax) * 16 + (l16 & 1) * 8;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    u32x2 hv[DB][2];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int j = 2 * db + sub;                                  // subspace
        const uint32_t code = (vcw[k][hf][j >> 2] >> (8 * (j & 3))) & 0xFFu;
        hv[db][hf] = tr16(vrow + (2 * db * kPqKMax + (int)code) * 16);
      }
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const u32x4 raw = {hv[db][0][0], hv[db][0][1], hv[db][1][0], hv[db][1][1]};
      acc[db] = mfma_f16(__builtin_bit_cast(f16x8, raw), ph[k], acc[db]);
    }
  }
  splitk_epilogue<D, kPqWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem), a.o, unit, split, b, hq0, G,
                               kDmapDense);
}

// ============================================================================
// Per-key LUT scores: out[b, h, t] = sum_j lut[b, h, j, k_idx[t, j]] (j in
// order) + sum_c q_out[b, h, c] * k_out[t, c] (C > 0), fp32.  A workgroup
// stages the LUTs of one (b, kv head, group of <= 4 query heads) in LDS and
// scores a run of tokens, one token per thread.
// ============================================================================
constexpr int kPqScoreThreads = 256;

template <int M, bool OUT>
__global__ __launch_bounds__(kPqScoreThreads, 2) void pq_score_kernel(PqArgs a, float* out, int64_t o_sb,
                                                                      int64_t o_sh, int parts) {
  __shared__ __attribute__((aligned(16))) float lut[kPqHeads * M * kPqKMax];
  __shared__ float qo[kPqHeads * kPqOutMax];
  const int unit = blockIdx.x / parts, part = blockIdx.x - unit * parts;
  const int b = unit / (a.Hk * a.HG);
  const int rem = unit - b * a.Hk * a.HG;
  const int hk = rem / a.HG, hg = rem - (rem / a.HG) * a.HG;
  const int hq0 = hk * a.G + hg * kPqHeads;
  const int nh = min(kPqHeads, a.G - hg * kPqHeads);
  const int K = a.K, K4 = K / 4;
  for (int e = threadIdx.x; e < nh * M * K4; e += kPqScoreThreads) {
    const int h = e / (M * K4), r2 = e - h * (M * K4);
    const int j = r2 / K4, c4 = r2 - j * K4;
    *reinterpret_cast<u32x4*>(lut + (h * M + j) * kPqKMax + c4 * 4) =
        ld16(a.lut + (int64_t)b * a.l_sb + (int64_t)(hq0 + h) * a.l_sh + j * K + c4 * 4);
  }
  if constexpr (OUT) {
    for (int e = threadIdx.x; e < kPqHeads * kPqOutMax; e += kPqScoreThreads) {
      const int h = e / kPqOutMax, c = e - h * kPqOutMax;
      qo[e] = (h < nh && c < a.C) ? load_any(a.qout, a.qo_dt, (int64_t)b * a.qo_sb + (int64_t)(hq0 + h) * a.qo_sh + c)
                                  : 0.f;
    }
  }
  __syncthreads();
  const int per = a.chunk;
  const int t_end = min((part + 1) * per, a.S);
  const uint8_t* kib = a.kidx + (int64_t)b * a.ki_sb + (int64_t)hk * a.ki_sh;
  const char* kob = OUT ? static_cast<const char*>(a.kout) +
                              ((int64_t)b * a.ko_sb + (int64_t)hk * a.ko_sh) * (a.ko_dt == 2 ? 4 : 2)
                        : nullptr;
  for (int t = part * per + threadIdx.x; t < t_end; t += kPqScoreThreads) {
    u32x4 kc;
    if constexpr (M == 16) {
      kc = ld16(kib + (int64_t)t * a.ki_ss);
    } else {
      const u32x2 hh = *reinterpret_cast<const u32x2*>(kib + (int64_t)t * a.ki_ss);
      kc = u32x4{hh[0], hh[1], 0u, 0u};
    }
    float ko[OUT ? kPqOutMax : 1];
    if constexpr (OUT) {
#pragma unroll
      for (int c = 0; c < kPqOutMax; ++c) ko[c] = c < a.C ? load_any(kob, a.ko_dt, (int64_t)t * a.ko_ss + c) : 0.f;
    }
    for (int h = 0; h < nh; ++h) {
      const float* lh = lut + h * (M * kPqKMax);
      float sc = 0.f;
#pragma unroll
      for (int j = 0; j < M; ++j) sc += lh[j * kPqKMax + ((kc[j >> 2] >> ((j & 3) * 8)) & 0xFFu)];
      if constexpr (OUT) {
        float so = 0.f;
#pragma unroll
        for (int c = 0; c < kPqOutMax; ++c) so += qo[h * kPqOutMax + c] * ko[c];
        sc += so;
      }
      out[(int64_t)b * o_sb + (int64_t)(hq0 + h) * o_sh + t] = sc;
    }
  }
}

static void pq_plan(int S, long units, int chunk_req, int* chunk, int* ns) {
  const int step = kPqWaves * kTile;
  int c;
  if (chunk_req > 0) {
    c = chunk_req;
  } else {
    const long target = device_cu_count();   // one workgroup per CU (LDS-bound)
    c = (int)(((long)S * units + target - 1) / target);
  }
  c = (c + step - 1) / step * step;
  if (c < step) c = step;
  *chunk = c;
  *ns = (S + c - 1) / c;
}

// Plan of the grouped kernel (units = B * Hk): chunks of <= kPqgChunk tokens,
// a multiple of the 32-token tile, sized to fill the CUs once; false where it
// does not apply (G > 8, a requested chunk above kPqgChunk, too many splits).
static bool pq_group_plan(int G, int S, long units, int chunk_req, int* chunk, int* ns) {
  if (G > 8) return false;
  long c;
  if (chunk_req > 0) {
    if (chunk_req > kPqgChunk) return false;
    c = chunk_req;
  } else {
    const long target = device_cu_count();
    c = ((long)S * units + target - 1) / target;
  }
  c = (c + kTile - 1) / kTile * kTile;
  if (c > kPqgChunk) c = kPqgChunk;
  *chunk = (int)c;
  *ns = (int)((S + c - 1) / c);
  return *ns <= 1024;
}

// ============================================================================
// LUT build: lut[b, h, j, c] = scale * q[b, h, 8j..8j+7] . cb[h/G][j][c], the
// entries of the MFMA contract above.  One wave per (b, kv head, block of 8
// query heads of its group, subspace pair): lane l finds the largest |q| of
// head l % 8 over an eighth of its row, then one MFMA (two where a lo part is
// nonzero) per 32 codewords.
// ============================================================================
__global__ __launch_bounds__(64) void pq_lut_kernel(const uint16_t* q, int64_t q_sb, int64_t q_sh, const _Float16* cb,
                                                    int64_t cb_sh, int Hk, int G, int HB, int M, int K, float scale,
                                                    float* lut) {
  const int lane = threadIdx.x;
  const int MP = (M + 1) / 2;
  int r = blockIdx.x;
  const int jp = 2 * (r % MP);
  r /= MP;
  const int hb = r % HB;
  r /= HB;
  const int hk = r % Hk, b = r / Hk;
  const int h0 = hb * 8, nh = min(8, G - h0);
  const uint16_t* qb = q + (int64_t)b * q_sb + (int64_t)(hk * G + h0) * q_sh;
  // head l % 8 (clamped to the block): the largest |q| over dims (l / 8) * M .. +M
  const int ha = min(lane & 7, nh - 1);
  float amax = 0.f;
  for (int d = (lane >> 3) * M; d < ((lane >> 3) + 1) * M; ++d)
    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(qb[(int64_t)ha * q_sh + d])));
  amax = fmaxf(amax, shfl_xor_f(amax, 8));
  amax = fmaxf(amax, shfl_xor_f(amax, 16));
  amax = fmaxf(amax, shfl_xor_f(amax, 32));
  const int k_own = lut_shift(amax);                     // of head l % 8
  const float mul_own = (lane & 7) < nh ? ldexpf(scale, k_own) : 0.f;
  int hm, sub;
  const bool live = lut_a_live(lane, &hm, &sub) && hm < nh && jp + sub < M;
  const int k_m = __shfl(k_own, hm & 7, 64);
  float x[8];
  const uint16_t* qr = qb + (int64_t)min(hm, nh - 1) * q_sh + 8 * min(jp + sub, M - 1);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = ldexpf(bf16_bits_to_f32(qr[i]), -k_m);
  f16x8 hi, lo;
  lut_a_operands(x, live, hi, lo);
  const bool use_lo = lut_need_lo(lo);
  const int quad = lane >> 5, n = lane & 31;
  float mg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) mg[i] = __shfl(mul_own, 4 * quad + i, 64);
  // subspace jp + 1 past M (odd M) reads subspace M - 1; its entries are not stored
  const _Float16* cbh = cb + (int64_t)hk * cb_sh - (jp + 1 < M ? 0 : (int64_t)K * 8 * (lane >> 5));
  const int64_t Hq = (int64_t)Hk * G;
  float* lb = lut + ((int64_t)b * Hq + hk * G + h0) * M * K;
  const int ncb = (K + 31) / 32;
  for (int c32 = 0; c32 < ncb; ++c32) {
    const f32x16 e = lut_mfma(hi, lo, use_lo, lut_b_operand(cbh, K, jp, c32 * 32, lane));
    const int c = c32 * 32 + n;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * quad + i, j = jp + s2;
        if (h < nh && j < M && c < K) lb[((int64_t)h * M + j) * K + c] = mg[i] * e[8 * s2 + i];
      }
  }
}

// ============================================================================
// Encode: idx[n, j] = argmin_c sum_e (x[n, 8j+e] - cb[j][c][e])^2, the sum in
// fp32 in e order with separate multiply and add, first index on ties.
// One thread per (vector, subspace); the head's codebook is staged in LDS.
// ============================================================================
constexpr int kEncThreads = 256;

__global__ __launch_bounds__(kEncThreads) void pq_encode_kernel(const void* x, int x_dtype, int64_t rows_per_head,
                                                                int64_t x_rs, const void* cb, int cb_f32,
                                                                int64_t cb_sh, int M, int K, uint8_t* idx) {
  __shared__ float cbs[16 * kPqKMax * 8];   // 128 KB: M <= 16 subspaces, K <= 256
  const int head = blockIdx.y;
  for (int e = threadIdx.x; e < M * K * 8; e += kEncThreads) {
    const int64_t o = (int64_t)head * cb_sh + e;
    cbs[e] = cb_f32 ? static_cast<const float*>(cb)[o] : (float)static_cast<const _Float16*>(cb)[o];
  }
  __syncthreads();
  const int64_t gid = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
  if (gid >= rows_per_head * M) return;
  const int64_t n = gid / M;
  const int j = (int)(gid - n * M);
  const int64_t row = (int64_t)head * rows_per_head + n;
  float xv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t o = row * x_rs + j * 8 + e;
    xv[e] = x_dtype == 0 ? bf16_bits_to_f32(static_cast<const uint16_t*>(x)[o])
                         : (x_dtype == 1 ? (float)static_cast<const _Float16*>(x)[o] : static_cast<const float*>(x)[o]);
  }
  float best = __builtin_inff();
  int bi = 0;
  const float* cj = cbs + j * K * 8;
  for (int c = 0; c < K; ++c) {
    float dist = 0.f;
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = xv[e] - cj[c * 8 + e];
        dist = dist + d * d;
      }
    }
    if (dist < best) {
      best = dist;
      bi = c;
    }
  }
  idx[row * M + j] = (uint8_t)bi;
}

// out[row, 8j + e] = cb[j][idx[row, j]][e] (ProductQuantizer.dequantize, src/quantization.py:213-226).
__global__ void pq_decode_vectors_kernel(const uint8_t* idx, int64_t rows_per_head, const void* cb, int cb_f32,
                                         int64_t cb_sh, int M, int K, float* out) {
  const int head = blockIdx.y;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows_per_head * M * 8) return;
  const int64_t row = (int64_t)head * rows_per_head + gid / (M * 8);
  const int r = (int)(gid % (M * 8));
  const int j = r / 8, e = r % 8;
  const int c = idx[row * M + j];
  const int64_t o = (int64_t)head * cb_sh + ((int64_t)j * K + c) * 8 + e;
  out[row * (M * 8) + r] = cb_f32 ? static_cast<const float*>(cb)[o] : (float)static_cast<const _Float16*>(cb)[o];
}

// ============================================================================
// k-means centroid update, one workgroup per (head, subspace j), one thread
// per cluster c: thread c walks the points in index order and sums the ones
// labelled c, so every centroid is a sequential (deterministic) fp32 mean.
// Empty clusters take the point reseed[head, j, c] drawn by the caller, as
// src/quantization.py:128-130 re-initialises them.
// ============================================================================
constexpr int kKmThreads = 256;

__global__ __launch_bounds__(kKmThreads) void pq_kmeans_update_kernel(const float* x, int64_t n, int M, int K,
                                                                      const uint8_t* labels, const int64_t* reseed,
                                                                      _Float16* cb_out, float* cb32) {
  const int j = blockIdx.x % M;
  const int head = blockIdx.x / M;
  const int c = threadIdx.x;
  const float* xh = x + (int64_t)head * n * (M * 8);
  const uint8_t* lh = labels + (int64_t)head * n * M + j;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t cnt = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (lh[i * M] == c) {
      const float* p = xh + i * (M * 8) + j * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] += p[e];
      ++cnt;
    }
  }
  if (c >= K) return;
  const int64_t o = (((int64_t)head * M + j) * K + c) * 8;
  const float* src = cnt ? nullptr : xh + reseed[((int64_t)head * M + j) * K + c] * (M * 8) + j * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = cnt ? s[e] / (float)cnt : src[e];
    cb32[o + e] = v;
    cb_out[o + e] = (_Float16)v;
  }
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_pq_decode_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk_req, size_t* bytes) {
  if (!bytes || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HG = (G + kPqHeads - 1) / kPqHeads;
  const long units = (long)B * Hk * HG;
  int chunk, ns;
  pq_plan(S, units, chunk_req, &chunk, &ns);
  *bytes = splitk_workspace_bytes(units, ns, D);
  // the grouped kernel's plan (quantized-value modes) may need more
  if (pq_group_plan(G, S, (long)B * Hk, chunk_req, &chunk, &ns)) {
    const size_t g = splitk_workspace_bytes((long)B * Hk, ns, D);
    if (g > *bytes) *bytes = g;
  }
  return 0;
}

// Launch the decode on a filled PqArgs (strides, pointers, modes set).
// mode 0: LUT + PQ values, 1: LUT + dense V, 2: q + key codebook + dense V,
// 3: q + key codebook + PQ values.
static int pq_launch(PqArgs& a, int mode, bool vf8, int B, int Hq, int Hk, int S, int D, int K, void* out,
                     int out_dtype, int64_t o_sb, int64_t o_sh, float scale, int chunk_req, void* workspace,
                     size_t workspace_bytes, void* stream) {
  a.Hk = Hk; a.G = Hq / Hk; a.HG = (a.G + kPqHeads - 1) / kPqHeads; a.S = S; a.K = K;
  a.scale_log2 = scale * kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  a.o.out = out;
  a.o.out_dtype = out_dtype;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  {
    // quantized values and G <= 8: one unit per (b, kv head)
    const long gunits = (long)B * Hk;
    int gns;
    if ((mode == 0 || mode == 3) && a.C == 0 && gunits <= kMaxUnits &&
        pq_group_plan(a.G, S, gunits, chunk_req, &a.chunk, &gns)) {
      if (!workspace || workspace_bytes < splitk_workspace_bytes(gunits, gns, D)) return (int)hipErrorInvalidValue;
      a.o.Hk = Hk; a.o.HB = 1; a.o.G = a.G; a.o.hbs = a.G;
      splitk_carve(workspace, gunits, gns, a.o);
      const dim3 grid((unsigned)(gns * gunits)), block(kPqgThreads);
      if (mode == 3 && !a.btab) {
        if (D == 128) BYTES_LAUNCH(kProfPq, (pq_wave_kernel<128>), grid, block, 0, st, a);
        else BYTES_LAUNCH(kProfPq, (pq_wave_kernel<64>), grid, block, 0, st, a);
        const int rc = (int)hipGetLastError();
        if (rc) return rc;
        return splitk_combine(a.o, gunits, D, st);
      }
#define PQG_LAUNCH(DD, BL, HP)                                                                   \
  if (a.btab) BYTES_LAUNCH(kProfPq, (pq_group_kernel<DD, BL, HP, true>), grid, block, 0, st, a);  \
  else BYTES_LAUNCH(kProfPq, (pq_group_kernel<DD, BL, HP, false>), grid, block, 0, st, a);
#define PQG_HP(DD, BL)            \
  if (a.G <= 4) { PQG_LAUNCH(DD, BL, 4) } \
  else { PQG_LAUNCH(DD, BL, 8) }
      if (D == 128) {
        if (mode == 3) { PQG_HP(128, 2) } else { PQG_HP(128, 0) }
      } else {
        if (mode == 3) { PQG_HP(64, 2) } else { PQG_HP(64, 0) }
      }
#undef PQG_HP
#undef PQG_LAUNCH
      const int rc = (int)hipGetLastError();
      if (rc) return rc;
      return splitk_combine(a.o, gunits, D, st);
    }
  }
  const long units = (long)B * Hk * a.HG;
  if (units > kMaxUnits) return (int)hipErrorInvalidConfiguration;
  int ns;
  pq_plan(S, units, chunk_req, &a.chunk, &ns);
  if (ns > 1024) return (int)hipErrorInvalidConfiguration;
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  // the merge kernel maps unit -> (b, hk, head group of kPqHeads)
  a.o.Hk = Hk; a.o.HB = a.HG; a.o.G = a.G; a.o.hbs = kPqHeads;
  splitk_carve(workspace, units, ns, a.o);
  dim3 grid((unsigned)(ns * units)), block(kPqWaves * 64);
  const bool outl = a.C > 0;
#define PQ_LAUNCH(DD, BL, QQ, F8, OU) BYTES_LAUNCH(kProfPq, (pq_decode_kernel<DD, BL, QQ, F8, OU>), grid, block, 0, st, a)
#define PQ_MODES(DD)                                          \
  if (mode == 0) PQ_LAUNCH(DD, false, true, false, false);    \
  else if (mode == 2) PQ_LAUNCH(DD, true, false, false, false); \
  else if (mode == 3) PQ_LAUNCH(DD, true, true, false, false); \
  else if (!vf8 && !outl) PQ_LAUNCH(DD, false, false, false, false); \
  else if (!vf8) PQ_LAUNCH(DD, false, false, false, true);   \
  else if (!outl) PQ_LAUNCH(DD, false, false, true, false);  \
  else PQ_LAUNCH(DD, false, false, true, true);
  if (D == 128) {
    PQ_MODES(128)
  } else {
    PQ_MODES(64)
  }
#undef PQ_MODES
#undef PQ_LAUNCH
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

static PqArgs pq_args_zero() {
  PqArgs a;
  memset(&a, 0, sizeof(a));
  return a;
}

// mode 0: LUT scores + PQ values (decode_attn_pq_lut_kv)
// mode 1: LUT scores + dense bf16 values (decode_attn_pq_lut)
// mode 2: scores from q and the key codebook + dense bf16 values (decode_attn_dequant)
// mode 3: mode 0 with no LUT in HBM.  G <= 8 without outliers (the grouped
//         kernel): scores scale * (q . k_hat) on MFMA straight from the key
//         codebook rows the codes select (exact products, fp32 sums), within
//         the attention tolerance of bytes_pq_build_lut + mode 0.  G > 8: each
//         workgroup builds the LUT in LDS, entries scale * (q . codeword)
//         exactly as bytes_pq_build_lut writes them (bit-identical to the two
//         calls).  The softmax takes the scores unscaled.
int bytes_pq_decode_attn(int mode, const void* lut, const void* q, const void* kcb, const void* kidx,
                         const void* vidx, const void* vcb, const void* v, void* out, int out_dtype, int B, int Hq,
                         int Hk, int S, int D, int K, int64_t l_sb, int64_t l_sh, int64_t q_sb, int64_t q_sh,
                         int64_t kcb_sh, int64_t ki_sb, int64_t ki_sh, int64_t ki_ss, int64_t vi_sb, int64_t vi_sh,
                         int64_t vi_ss, int64_t vcb_sh, int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb,
                         int64_t o_sh, float scale, int chunk_req, void* workspace, size_t workspace_bytes,
                         void* stream) {
  if (mode < 0 || mode > 3 || !kidx || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0)
    return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || K <= 0 || K > kPqKMax || K % 4 != 0) return (int)hipErrorInvalidValue;
  if (mode == 0 && (!lut || !vidx || !vcb)) return (int)hipErrorInvalidValue;
  if (mode == 1 && (!lut || !v)) return (int)hipErrorInvalidValue;
  if (mode == 2 && (!q || !kcb || !v)) return (int)hipErrorInvalidValue;
  if (mode == 3 && (!q || !kcb || !vidx || !vcb)) return (int)hipErrorInvalidValue;
  if (out_dtype < 0 || out_dtype > 2) return (int)hipErrorInvalidValue;
  PqArgs a = pq_args_zero();
  a.lut_scale = mode == 3 ? scale : 1.f;
  if (mode == 3) scale = 1.f;
  a.lut = static_cast<const float*>(lut);
  a.l_sb = l_sb; a.l_sh = l_sh;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.kcb = static_cast<const _Float16*>(kcb);
  a.kcb_sh = kcb_sh;
  a.kidx = static_cast<const uint8_t*>(kidx);
  a.ki_sb = ki_sb; a.ki_sh = ki_sh; a.ki_ss = ki_ss;
  a.vidx = static_cast<const uint8_t*>(vidx);
  a.vi_sb = vi_sb; a.vi_sh = vi_sh; a.vi_ss = vi_ss;
  a.vcb = static_cast<const _Float16*>(vcb);
  a.vcb_sh = vcb_sh;
  a.v = v;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  return pq_launch(a, mode, false, B, Hq, Hk, S, D, K, out, out_dtype, o_sb, o_sh, scale, chunk_req, workspace,
                   workspace_bytes, stream);
}

int bytes_pq_lut_decode_attn(const void* lut, int64_t l_sb, int64_t l_sh, const void* kidx, int64_t ki_sb,
                             int64_t ki_sh, int64_t ki_ss, const void* vidx, int64_t vi_sb, int64_t vi_sh,
                             int64_t vi_ss, const void* vcb, int64_t vcb_sh, const void* v, int v_fp8, int64_t v_sb,
                             int64_t v_sh, int64_t v_ss, const void* kout, int ko_dtype, int64_t ko_sb,
                             int64_t ko_sh, int64_t ko_ss, const void* qout, int qo_dtype, int64_t qo_sb,
                             int64_t qo_sh, int C, const int* block_table, int64_t bt_sb, const int* context_lens,
                             int block_size, int num_blocks, void* out, int out_dtype, int64_t o_sb, int64_t o_sh,
                             int B, int Hq, int Hk, int S, int D, int K, float scale, int chunk_req, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!lut || !kidx || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || K <= 0 || K > kPqKMax || K % 4 != 0) return (int)hipErrorInvalidValue;
  const bool qv = vidx != nullptr;
  if (qv == (v != nullptr) || (qv && (!vcb || v_fp8 || C > 0))) return (int)hipErrorInvalidValue;
  if (C < 0 || C > kPqOutMax || (C > 0 && (!kout || !qout))) return C > kPqOutMax ? (int)hipErrorNotSupported
                                                                                  : (int)hipErrorInvalidValue;
  if (ko_dtype < 0 || ko_dtype > 2 || qo_dtype < 0 || qo_dtype > 2) return (int)hipErrorInvalidValue;
  if (block_table && (!context_lens || block_size <= 0 || num_blocks <= 0 || S % block_size != 0))
    return (int)hipErrorInvalidValue;
  if (out_dtype < 0 || out_dtype > 2) return (int)hipErrorInvalidValue;
  PqArgs a = pq_args_zero();
  a.lut = static_cast<const float*>(lut);
  a.l_sb = l_sb; a.l_sh = l_sh;
  a.kidx = static_cast<const uint8_t*>(kidx);
  a.ki_sb = ki_sb; a.ki_sh = ki_sh; a.ki_ss = ki_ss;
  a.vidx = static_cast<const uint8_t*>(vidx);
  a.vi_sb = vi_sb; a.vi_sh = vi_sh; a.vi_ss = vi_ss;
  a.vcb = static_cast<const _Float16*>(vcb);
  a.vcb_sh = vcb_sh;
  a.v = v;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.kout = kout;
  a.ko_sb = ko_sb; a.ko_sh = ko_sh; a.ko_ss = ko_ss; a.ko_dt = ko_dtype;
  a.qout = qout;
  a.qo_sb = qo_sb; a.qo_sh = qo_sh; a.qo_dt = qo_dtype;
  a.C = C;
  a.btab = block_table;
  a.bt_sb = bt_sb;
  a.clens = context_lens;
  a.bs = block_size;
  a.nblk = num_blocks;
  return pq_launch(a, qv ? 0 : 1, v_fp8 != 0, B, Hq, Hk, S, D, K, out, out_dtype, o_sb, o_sh, scale, chunk_req,
                   workspace, workspace_bytes, stream);
}

int bytes_pq_lut_scores(const void* lut, int64_t l_sb, int64_t l_sh, const void* kidx, int64_t ki_sb, int64_t ki_sh,
                        int64_t ki_ss, const void* kout, int ko_dtype, int64_t ko_sb, int64_t ko_sh, int64_t ko_ss,
                        const void* qout, int qo_dtype, int64_t qo_sb, int64_t qo_sh, int C, void* out, int64_t o_sb,
                        int64_t o_sh, int B, int Hq, int Hk, int S, int D, int K, void* stream) {
  if (!lut || !kidx || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || K <= 0 || K > kPqKMax || K % 4 != 0) return (int)hipErrorInvalidValue;
  if (C < 0 || C > kPqOutMax || (C > 0 && (!kout || !qout))) return C > kPqOutMax ? (int)hipErrorNotSupported
                                                                                  : (int)hipErrorInvalidValue;
  if (ko_dtype < 0 || ko_dtype > 2 || qo_dtype < 0 || qo_dtype > 2) return (int)hipErrorInvalidValue;
  PqArgs a = pq_args_zero();
  a.lut = static_cast<const float*>(lut);
  a.l_sb = l_sb; a.l_sh = l_sh;
  a.kidx = static_cast<const uint8_t*>(kidx);
  a.ki_sb = ki_sb; a.ki_sh = ki_sh; a.ki_ss = ki_ss;
  a.kout = kout;
  a.ko_sb = ko_sb; a.ko_sh = ko_sh; a.ko_ss = ko_ss; a.ko_dt = ko_dtype;
  a.qout = qout;
  a.qo_sb = qo_sb; a.qo_sh = qo_sh; a.qo_dt = qo_dtype;
  a.C = C;
  a.Hk = Hk; a.G = Hq / Hk; a.HG = (a.G + kPqHeads - 1) / kPqHeads; a.S = S; a.K = K;
  const long units = (long)B * Hk * a.HG;
  // runs of >= 2048 tokens per workgroup (the LUT staging is paid per workgroup), ~2 per CU
  const long target = 2L * device_cu_count();
  long per = ((long)S * units + target - 1) / target;
  if (per < 2048) per = 2048;
  per = (per + kPqScoreThreads - 1) / kPqScoreThreads * kPqScoreThreads;
  if (per > S) per = (S + kPqScoreThreads - 1) / kPqScoreThreads * kPqScoreThreads;
  a.chunk = (int)per;
  const long parts = (S + per - 1) / per;
  const long grid = units * parts;
  if (grid > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* o = static_cast<float*>(out);
  if (D == 128) {
    if (C > 0) hipLaunchKernelGGL((pq_score_kernel<16, true>), dim3((unsigned)grid), dim3(kPqScoreThreads), 0, st, a, o, o_sb, o_sh, (int)parts);
    else hipLaunchKernelGGL((pq_score_kernel<16, false>), dim3((unsigned)grid), dim3(kPqScoreThreads), 0, st, a, o, o_sb, o_sh, (int)parts);
  } else {
    if (C > 0) hipLaunchKernelGGL((pq_score_kernel<8, true>), dim3((unsigned)grid), dim3(kPqScoreThreads), 0, st, a, o, o_sb, o_sh, (int)parts);
    else hipLaunchKernelGGL((pq_score_kernel<8, false>), dim3((unsigned)grid), dim3(kPqScoreThreads), 0, st, a, o, o_sb, o_sh, (int)parts);
  }
  return (int)hipGetLastError();
}

int bytes_pq_build_lut(const void* q, const void* cb, void* lut, int B, int Hq, int Hk, int D, int K, int64_t q_sb,
                       int64_t q_sh, int64_t cb_sh, float scale, void* stream) {
  if (!q || !cb || !lut || B <= 0 || Hk <= 0 || Hq % Hk != 0 || D % 8 != 0 || K <= 0 || K > kPqKMax)
    return (int)hipErrorInvalidValue;
  const int M = D / 8, G = Hq / Hk, HB = (G + 7) / 8;
  const int64_t waves = (int64_t)B * Hk * HB * ((M + 1) / 2);
  if (waves > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(pq_lut_kernel, dim3((unsigned)waves), dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(q), q_sb, q_sh, static_cast<const _Float16*>(cb), cb_sh, Hk, G, HB,
                     M, K, scale, static_cast<float*>(lut));
  return (int)hipGetLastError();
}

int bytes_pq_encode(const void* x, int x_dtype, int heads, int64_t rows_per_head, int64_t x_row_stride, int D,
                    const void* cb, int cb_f32, int64_t cb_sh, int K, void* idx, void* stream) {
  if (!x || !cb || !idx || heads <= 0 || rows_per_head < 0 || D % 8 != 0 || D / 8 > 16 || K <= 0 || K > kPqKMax)
    return (int)hipErrorInvalidValue;
  if (x_dtype < 0 || x_dtype > 2 || heads > 65535) return (int)hipErrorInvalidValue;
  if (rows_per_head == 0) return 0;
  const int M = D / 8;
  const int64_t blocks = (rows_per_head * M + kEncThreads - 1) / kEncThreads;
  if (blocks > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(pq_encode_kernel, dim3((unsigned)blocks, (unsigned)heads), dim3(kEncThreads), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, rows_per_head, x_row_stride, cb, cb_f32 ? 1 : 0,
                     cb_sh, M, K, static_cast<uint8_t*>(idx));
  return (int)hipGetLastError();
}

int bytes_pq_decode_vectors(const void* idx, int heads, int64_t rows_per_head, int D, const void* cb, int cb_f32,
                            int64_t cb_sh, int K, void* out, void* stream) {
  if (!idx || !cb || !out || heads <= 0 || rows_per_head < 0 || D % 8 != 0 || K <= 0 || K > kPqKMax)
    return (int)hipErrorInvalidValue;
  if (heads > 65535) return (int)hipErrorInvalidConfiguration;
  if (rows_per_head == 0) return 0;
  const int64_t per = rows_per_head * D;
  const int th = 256;
  hipLaunchKernelGGL(pq_decode_vectors_kernel, dim3((unsigned)((per + th - 1) / th), (unsigned)heads), dim3(th), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(idx), rows_per_head, cb,
                     cb_f32 ? 1 : 0, cb_sh, D / 8, K, static_cast<float*>(out));
  return (int)hipGetLastError();
}

int bytes_pq_kmeans_update(const void* x, int heads, int64_t n, int D, int K, const void* labels, const void* reseed,
                           void* cb_f16, void* cb_f32, void* stream) {
  if (!x || !labels || !reseed || !cb_f16 || !cb_f32 || heads <= 0 || n <= 0 || D % 8 != 0 || K <= 0 ||
      K > kKmThreads)
    return (int)hipErrorInvalidValue;
  const int M = D / 8;
  const int64_t blocks = (int64_t)heads * M;
  if (blocks > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(pq_kmeans_update_kernel, dim3((unsigned)blocks), dim3(kKmThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(x), n, M, K,
                     static_cast<const uint8_t*>(labels), static_cast<const int64_t*>(reseed),
                     static_cast<_Float16*>(cb_f16), static_cast<float*>(cb_f32));
  return (int)hipGetLastError();
}

}  // extern "C"
