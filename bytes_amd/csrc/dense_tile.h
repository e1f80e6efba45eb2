// Dense bf16 flash-decode tile machinery shared by the dense and KIVI kernels.
//
// Per wave, per 32-token tile:
//   S^T[t][h] = K[t][:] . Q[h][:]    two 16x16 MFMA blocks over D; A = K rows
//                                    read back from LDS, B = Q in VGPRs
//   fp32 online softmax per head     lane l owns head l%16
//   O^T[d][h] += V^T[d][t] P^T[t][h] MFMA; V read back transposed with
//                                    ds_read_b64_tr_b16
// K and V rows of the next tile are prefetched into VGPRs while the current
// tile is computed from wave-private LDS buffers (XOR-swizzled 16-byte chunks,
// so both the row reads and the transposed reads are bank-conflict free).
// LDS-DMA (global_load_lds) is deliberately not used here: the compiler
// places a vmcnt(0) wait before every LDS read that follows one, which would
// drain the prefetch on every tile.
#pragma once
#include "splitk.h"

namespace bytes_amd {

constexpr int kDenseWaves = 4;
constexpr int kTile = 32;

template <int D>
struct DenseCfg {
  static constexpr int KK = D / 32;                  // MFMA k-steps over D
  static constexpr int DB = D / 16;                  // 16-wide output blocks over D
  static constexpr int CPR = D / 8;                  // 16-byte chunks per K/V row
  static constexpr int CPL = kTile * CPR / 64;       // chunks per lane per tile (each of K, V)
  static constexpr int VT = kTile * D * 2;           // bytes of one K or V tile
  static constexpr int WAVE = 2 * VT;                // K + V buffers of one wave
  static constexpr int kRing = kDenseWaves * WAVE;
  static constexpr int kEpi = splitk_smem_floats<D, kDenseWaves>() * 4;
  static constexpr int kSmem = kRing > kEpi ? kRing : kEpi;
};

// One tile's worth of prefetched K and V rows (raw 16-byte chunks, chunk
// p = lane + 64*i is row p / CPR, column chunk p % CPR).
template <int D>
struct DenseRegs {
  u32x4 k[DenseCfg<D>::CPL];
  u32x4 v[DenseCfg<D>::CPL];
};

// LDS placement of 16-byte column chunk c of row r.
//  K: XOR by the row, so the 16 rows an MFMA A-operand read touches hit
//     distinct banks.
//  V: XOR so the 4 rows (and the neighbouring 4-row group) a transposed
//     ds_read_b64_tr_b16 touches hit distinct banks.
template <int D>
__device__ __forceinline__ int kswz(int r, int c) { return c ^ (r & (D / 8 - 1)); }
template <int D>
__device__ __forceinline__ int vswz(int r, int c) {
  return D >= 128 ? c ^ ((r & 3) << 1) ^ (((r >> 2) & 1) << 3) : c ^ ((r & 3) << 1);
}

typedef __fp16 fp16x4_vs __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_vs* tr16_ptr_t;
__device__ __forceinline__ u32x2 tr16(const char* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16((tr16_ptr_t)p));
}

// Issue the loads of one tile into registers.  A tile at or past t_end is
// issued as a dummy (every lane reads the same 16 bytes of row S-1), so every
// iteration issues the same vector-memory instructions and control flow stays
// uniform, which lets the compiler wait for exactly the registers it uses.
template <int D>
__device__ __forceinline__ void dense_issue(const uint16_t* kbase, const uint16_t* vbase, int64_t k_ss,
                                            int64_t v_ss, int S, int t0, int t_end, int lane, DenseRegs<D>& r) {
  using C = DenseCfg<D>;
  const bool live = t0 < t_end;
#pragma unroll
  for (int i = 0; i < C::CPL; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / C::CPR, pos = p - rr * C::CPR;
    const int row = live ? min(t0 + rr, S - 1) : S - 1;
    const int col = live ? pos * 8 : 0;
    r.k[i] = ld16_nt(kbase + (int64_t)row * k_ss + col);
    r.v[i] = ld16_nt(vbase + (int64_t)row * v_ss + col);
  }
}

template <int D>
__device__ __forceinline__ void dense_stage(int lane, const DenseRegs<D>& r, char* kst, char* vst) {
  using C = DenseCfg<D>;
#pragma unroll
  for (int i = 0; i < C::CPL; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / C::CPR, pos = p - rr * C::CPR;
    *reinterpret_cast<u32x4*>(kst + rr * (D * 2) + kswz<D>(rr, pos) * 16) = r.k[i];
    *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, pos) * 16) = r.v[i];
  }
}

// Bit j of the tile mask = tile row j (0..31) takes part in the softmax.
__device__ __forceinline__ uint32_t range_mask(int t0, int t_end) {
  const int n = t_end - t0;
  return n >= 32 ? 0xFFFFFFFFu : (n <= 0 ? 0u : ((1u << n) - 1u));
}

// Address of the 4 consecutive V elements (row, col .. col+3) of a tile staged
// in vst (vswz layout).
template <int D>
struct StagedV {
  const char* vst;
  __device__ __forceinline__ const char* operator()(int hf, int row, int col) const {
    return vst + row * (D * 2) + vswz<D>(row, col >> 3) * 16 + (col & 7) * 2;
  }
};

// Online softmax and PV for one 32-row tile whose raw scores are s[blk][i]
// (row blk*16 + lg*4 + i, head l%16; the layout of the score MFMA output);
// vaddr(hf, row, col) gives the LDS address of V elements (row, col .. col+3)
// of the tile (hf = row / 16).  Rows whose vmask bit is clear get probability
// zero.  F16: V and P in fp16 (f16 MFMA), else bf16.
template <int D, bool F16 = false, class VA>
__device__ __forceinline__ void tile_softmax_pv_at(const f32x4 (&s)[2], uint32_t vmask, float scale_log2, int lane,
                                                   const VA& vaddr, float& m_run, float& l_run,
                                                   f32x4 (&acc)[D / 16]) {
  using C = DenseCfg<D>;
  const int l16 = lane & 15, lg = lane >> 4;
  float x[8];
  float mx = kNegInf;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = blk * 16 + lg * 4 + i;
      const float xv = ((vmask >> j) & 1u) ? s[blk][i] * scale_log2 : kNegInf;
      x[blk * 4 + i] = xv;
      mx = __builtin_elementwise_maximum(mx, xv);
    }
  mx = col_max4(mx);
  const float m_new = fmaxf(m_run, mx);
  const float m_use = (m_new == kNegInf) ? 0.f : m_new;
  const float alpha = fast_exp2(m_run - m_use);
  float psum = 0.f;
  bf16x8 pb;
  f16x8 ph;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = fast_exp2(x[j] - m_use);
    psum += p;
    if (F16)
      ph[j] = (_Float16)p;
    else
      pb[j] = (__bf16)p;
  }
  l_run = l_run * alpha + psum;
  m_run = m_new;
  // PV: A = V^T[d = db*16 + l16][k], k = lg*8 + j <-> token (j<4 ? lg*4+j : 16+lg*4+j-4).
  // Two transposed reads per block: lane i of the 16-lane group supplies row
  // base + i/4, columns db*16 + (i%4)*4 .. +3; lane j receives column j.
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    acc[db] *= alpha;
    u32x2 h[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = hf * 16 + lg * 4 + (l16 >> 2);
      const int col = db * 16 + (l16 & 3) * 4;
      h[hf] = tr16(vaddr(hf, row, col));
    }
    const u32x4 raw = {h[0][0], h[0][1], h[1][0], h[1][1]};
    if (F16)
      acc[db] = mfma_f16(__builtin_bit_cast(f16x8, raw), ph, acc[db]);
    else
      acc[db] = mfma_bf16(__builtin_bit_cast(bf16x8, raw), pb, acc[db]);
  }
}

template <int D, bool F16 = false>
__device__ __forceinline__ void tile_softmax_pv(const f32x4 (&s)[2], uint32_t vmask, float scale_log2, int lane,
                                                const char* vst, float& m_run, float& l_run,
                                                f32x4 (&acc)[D / 16]) {
  tile_softmax_pv_at<D, F16>(s, vmask, scale_log2, lane, StagedV<D>{vst}, m_run, l_run, acc);
}

// Scores (K rows staged in kst, Q in VGPRs), online softmax and PV for the
// tile staged in kst/vst; rows whose vmask bit is clear get probability zero.
template <int D>
__device__ __forceinline__ void dense_compute(uint32_t vmask, float scale_log2, int lane,
                                              const bf16x8 (&qb)[D / 32], const char* kst, const char* vst,
                                              float& m_run, float& l_run, f32x4 (&acc)[D / 16]) {
  using C = DenseCfg<D>;
  const int l16 = lane & 15, lg = lane >> 4;
  f32x4 s[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    s[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int row = blk * 16 + l16;
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
      const bf16x8 ka = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(kst + row * (D * 2) + kswz<D>(row, kk * 4 + lg) * 16));
      s[blk] = mfma_bf16(ka, qb[kk], s[blk]);
    }
  }
  tile_softmax_pv<D, false>(s, vmask, scale_log2, lane, vst, m_run, l_run, acc);
}

// Runs the pipelined dense tile loop of one wave over tokens
// [t_begin + w*32, t_end) with stride kDenseWaves*32.  At the top of each
// tile the prefetched registers are written to the wave's LDS buffers and
// immediately refilled with the next tile, so one tile is always in flight.
template <int D>
__device__ __forceinline__ void dense_wave_loop(const uint16_t* kbase, const uint16_t* vbase, int64_t k_ss,
                                                int64_t v_ss, int S, int t_begin, int t_end, int w, int lane,
                                                float scale_log2, const bf16x8 (&qb)[D / 32], char* wbuf,
                                                float& m_run, float& l_run, f32x4 (&acc)[D / 16]) {
  constexpr int STEP = kDenseWaves * kTile;
  char* kst = wbuf;
  char* vst = wbuf + DenseCfg<D>::VT;
  DenseRegs<D> r;
  int t = t_begin + w * kTile;
  if (t >= t_end) return;
  dense_issue<D>(kbase, vbase, k_ss, v_ss, S, t, t_end, lane, r);
  for (; t < t_end; t += STEP) {
    wave_lds_sync();
    dense_stage<D>(lane, r, kst, vst);
    dense_issue<D>(kbase, vbase, k_ss, v_ss, S, t + STEP, t_end, lane, r);
    wave_lds_sync();
    dense_compute<D>(range_mask(t, t_end), scale_log2, lane, qb, kst, vst, m_run, l_run, acc);
  }
}

// ---- fp8 (OCP e4m3fn) K/V rows, widened to bf16 while they are staged ----
// 16 fp8 values -> 16 bf16 (two 16-byte LDS chunks).  v_cvt_pk_f32_fp8 decodes
// e4m3fn exactly (NaN included); every e4m3 value is a bf16 value, so the
// bf16 bits are the top half of the f32 bits.
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
  return (__float_as_uint(f[0]) >> 16) | (__float_as_uint(f[1]) & 0xFFFF0000u);
}
__device__ __forceinline__ void fp8x16_to_bf16(const u32x4& in, u32x4& lo, u32x4& hi) {
  lo = u32x4{fp8x2_to_bf16x2<false>(in[0]), fp8x2_to_bf16x2<true>(in[0]), fp8x2_to_bf16x2<false>(in[1]),
             fp8x2_to_bf16x2<true>(in[1])};
  hi = u32x4{fp8x2_to_bf16x2<false>(in[2]), fp8x2_to_bf16x2<true>(in[2]), fp8x2_to_bf16x2<false>(in[3]),
             fp8x2_to_bf16x2<true>(in[3])};
}

template <int D>
struct DenseRegs8 {
  static constexpr int CPR8 = D / 16;                 // 16-byte fp8 chunks per row
  static constexpr int CPL8 = kTile * CPR8 / 64;      // per lane per tile (each of K, V)
  u32x4 k[CPL8];
  u32x4 v[CPL8];
};

template <int D>
__device__ __forceinline__ void dense_issue_fp8(const uint8_t* kbase, const uint8_t* vbase, int64_t k_ss, int64_t v_ss,
                                                int S, int t0, int t_end, int lane, DenseRegs8<D>& r) {
  using R = DenseRegs8<D>;
  const bool live = t0 < t_end;
#pragma unroll
  for (int i = 0; i < R::CPL8; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / R::CPR8, pos = p - rr * R::CPR8;
    const int row = live ? min(t0 + rr, S - 1) : S - 1;
    const int col = live ? pos * 16 : 0;
    r.k[i] = ld16_nt(kbase + (int64_t)row * k_ss + col);
    r.v[i] = ld16_nt(vbase + (int64_t)row * v_ss + col);
  }
}

template <int D>
__device__ __forceinline__ void dense_stage_fp8(int lane, const DenseRegs8<D>& r, char* kst, char* vst) {
  using R = DenseRegs8<D>;
#pragma unroll
  for (int i = 0; i < R::CPL8; ++i) {
    const int p = lane + 64 * i;
    const int rr = p / R::CPR8, pos = p - rr * R::CPR8;
    u32x4 k0, k1, v0, v1;
    fp8x16_to_bf16(r.k[i], k0, k1);
    fp8x16_to_bf16(r.v[i], v0, v1);
    *reinterpret_cast<u32x4*>(kst + rr * (D * 2) + kswz<D>(rr, 2 * pos) * 16) = k0;
    *reinterpret_cast<u32x4*>(kst + rr * (D * 2) + kswz<D>(rr, 2 * pos + 1) * 16) = k1;
    *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, 2 * pos) * 16) = v0;
    *reinterpret_cast<u32x4*>(vst + rr * (D * 2) + vswz<D>(rr, 2 * pos + 1) * 16) = v1;
  }
}

// The dense tile loop over fp8 rows (same pipeline as dense_wave_loop).
template <int D>
__device__ __forceinline__ void dense_wave_loop_fp8(const uint8_t* kbase, const uint8_t* vbase, int64_t k_ss,
                                                    int64_t v_ss, int S, int t_begin, int t_end, int w, int lane,
                                                    float scale_log2, const bf16x8 (&qb)[D / 32], char* wbuf,
                                                    float& m_run, float& l_run, f32x4 (&acc)[D / 16]) {
  constexpr int STEP = kDenseWaves * kTile;
  char* kst = wbuf;
  char* vst = wbuf + DenseCfg<D>::VT;
  DenseRegs8<D> r;
  int t = t_begin + w * kTile;
  if (t >= t_end) return;
  dense_issue_fp8<D>(kbase, vbase, k_ss, v_ss, S, t, t_end, lane, r);
  for (; t < t_end; t += STEP) {
    wave_lds_sync();
    dense_stage_fp8<D>(lane, r, kst, vst);
    dense_issue_fp8<D>(kbase, vbase, k_ss, v_ss, S, t + STEP, t_end, lane, r);
    wave_lds_sync();
    dense_compute<D>(range_mask(t, t_end), scale_log2, lane, qb, kst, vst, m_run, l_run, acc);
  }
}

// Q rows as the MFMA B operand of the dense tile: lane holds Q[h = l16][d = kk*32 + lg*8 + j].
template <int D>
__device__ __forceinline__ void load_q_bf16(const uint16_t* qrow0, int64_t q_sh, int nh, int lane,
                                            bf16x8 (&qb)[D / 32]) {
  const int l16 = lane & 15, lg = lane >> 4;
  const bool live = l16 < nh;
  const uint16_t* qp = qrow0 + (int64_t)(live ? l16 : 0) * q_sh + lg * 8;
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) {
    u32x4 raw = ld16_live(qp + kk * 32, live);
    qb[kk] = __builtin_bit_cast(bf16x8, raw);
  }
}

}  // namespace bytes_amd
