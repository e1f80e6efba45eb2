// Dense bf16 GQA single-query decode attention (split-K flash-decode).
//
// Replaces src/attention_kernels.py:8-92 (`_decode_attn_bf16_kernel` /
// `decode_attn_bf16`).  The reference launches one program per (b, h_q) and
// so streams each KV head G times; here one workgroup serves all query heads
// of a GQA group for one chunk of the token axis, so K and V are read once.
//
// Per wave, per 32-token tile (waves of a workgroup take interleaved tiles):
//   S^T[t][h] = K[t][:] . Q[h][:]    two 16x16 MFMA blocks over D; A = K rows
//                                    loaded straight into VGPRs, B = Q in VGPRs
//   fp32 online softmax per head     lane l owns head l%16
//   O^T[d][h] += V^T[d][t] P^T[t][h] MFMA; V is streamed into a wave-private
//                                    LDS ring with global_load_lds_dwordx4
//                                    (XOR-swizzled 16-byte chunks, so the
//                                    transposed reads are bank-conflict free)
// The next tile's K and V loads are issued before the current tile is
// computed (two-stage software pipeline).
#include "splitk.h"

namespace bytes_amd {

struct DenseArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int Hk, G, S, HB, chunk;
  float scale_log2;
  SplitKOut o;
};

constexpr int kDenseWaves = 4;
constexpr int kTile = 32;

template <int D>
struct DenseCfg {
  static constexpr int KK = D / 32;                  // MFMA k-steps over D
  static constexpr int DB = D / 16;                  // 16-wide output blocks over D
  static constexpr int CPR = D / 8;                  // 16-byte chunks per K/V row
  static constexpr int CPL = kTile * CPR / 64;       // V chunks per lane per tile
  static constexpr int VT = kTile * D * 2;           // V tile bytes
  static constexpr int kRing = kDenseWaves * 2 * VT; // two stages per wave
  static constexpr int kEpi = splitk_smem_floats<D, kDenseWaves>() * 4;
  static constexpr int kSmem = kRing > kEpi ? kRing : kEpi;
};

// Chunk position of (row r, 16-byte column chunk c) inside an LDS V tile.
__device__ __forceinline__ int vswz(int r, int c) { return c ^ (((r >> 2) & 3) << 1); }

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt/lgkmcnt left at "don't wait").
#define BYTES_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Issue the loads of one tile.  A tile at or past t_end is issued as a dummy
// (every lane reads the same 16 bytes of row S-1), so that every loop
// iteration issues the same number of vector-memory instructions and the
// waits stay exact.
template <int D>
__device__ __forceinline__ void dense_issue(const uint16_t* kbase, const uint16_t* vbase, int64_t k_ss,
                                            int64_t v_ss, int S, int t0, int t_end, int lane,
                                            bf16x8 (&kr)[2][D / 32], char* vst) {
  using C = DenseCfg<D>;
  const int l16 = lane & 15, lg = lane >> 4;
  const bool live = t0 < t_end;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int row = live ? min(t0 + blk * 16 + l16, S - 1) : S - 1;
    const uint16_t* kp = kbase + (int64_t)row * k_ss + (live ? lg * 8 : 0);
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) kr[blk][kk] = __builtin_bit_cast(bf16x8, ld16(kp + (live ? kk * 32 : 0)));
  }
#pragma unroll
  for (int i = 0; i < C::CPL; ++i) {
    const int p = lane + 64 * i;
    const int r = p / C::CPR, pos = p - r * C::CPR;
    const int row = live ? min(t0 + r, S - 1) : S - 1;
    const uint16_t* src = vbase + (int64_t)row * v_ss + (live ? vswz(r, pos) * 8 : 0);
    __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)(vst + i * 1024), 16, 0, 0);
  }
}

template <int D>
__device__ __forceinline__ void dense_tile(int t0, int t_end, float scale_log2, int lane, const bf16x8 (&qb)[D / 32],
                                           const bf16x8 (&kr)[2][D / 32], const char* vst, float& m_run,
                                           float& l_run, f32x4 (&acc)[D / 16]) {
  using C = DenseCfg<D>;
  const int l16 = lane & 15, lg = lane >> 4;
  f32x4 s[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    s[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) s[blk] = mfma_bf16(kr[blk][kk], qb[kk], s[blk]);
  }
  float x[8];
  float mx = kNegInf;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + blk * 16 + lg * 4 + i;
      const float xv = t < t_end ? s[blk][i] * scale_log2 : kNegInf;
      x[blk * 4 + i] = xv;
      mx = fmaxf(mx, xv);
    }
  mx = fmaxf(mx, shfl_xor_f(mx, 16));
  mx = fmaxf(mx, shfl_xor_f(mx, 32));
  const float m_new = fmaxf(m_run, mx);
  const float m_use = (m_new == kNegInf) ? 0.f : m_new;
  const float alpha = exp2f(m_run - m_use);
  float psum = 0.f;
  bf16x8 pb;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = exp2f(x[j] - m_use);
    psum += p;
    pb[j] = (__bf16)p;
  }
  l_run = l_run * alpha + psum;
  m_run = m_new;
  // PV: A = V^T[d = db*16 + l16][k], k = lg*8 + j <-> token (j<4 ? lg*4+j : 16+lg*4+j-4);
  // every token row this lane reads has ((row >> 2) & 3) == lg.
  const uint16_t* vt = reinterpret_cast<const uint16_t*>(vst);
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    acc[db] *= alpha;
    const int pos = (2 * db + (l16 >> 3)) ^ (lg << 1);
    const int colw = pos * 8 + (l16 & 7);
    bf16x8 va;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int tok = (j < 4) ? (lg * 4 + j) : (16 + lg * 4 + j - 4);
      va[j] = __builtin_bit_cast(__bf16, vt[tok * D + colw]);
    }
    acc[db] = mfma_bf16(va, pb, acc[db]);
  }
}

template <int D>
__global__ __launch_bounds__(kDenseWaves * 64, 2) void dense_decode_kernel(DenseArgs a) {
  using C = DenseCfg<D>;
  constexpr int NLOAD = 2 * C::KK + C::CPL;  // vector-memory instructions per tile
  __shared__ __attribute__((aligned(16))) char smem_raw[C::kSmem];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, unit = blockIdx.y;
  const int b = unit / (a.Hk * a.HB);
  const int rem = unit - b * a.Hk * a.HB;
  const int hk = rem / a.HB, hb = rem - (rem / a.HB) * a.HB;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);

  // Q as the MFMA B operand: lane holds Q[h = l16][d = kk*32 + lg*8 + j].
  bf16x8 qb[C::KK];
  {
    const bool live = l16 < nh;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hq0 + (live ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
      u32x4 raw = live ? ld16(qp + kk * 32) : u32x4{0, 0, 0, 0};
      qb[kk] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  const int t_begin = split * a.chunk;
  const int t_end = min(t_begin + a.chunk, a.S);
  const uint16_t* kbase = a.k + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
  const uint16_t* vbase = a.v + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
  char* st0 = smem_raw + w * 2 * C::VT;
  char* st1 = st0 + C::VT;

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int STEP = kDenseWaves * kTile;
  bf16x8 kA[2][C::KK], kB[2][C::KK];
  int t = t_begin + w * kTile;
  const int ntiles = t < t_end ? (t_end - t + STEP - 1) / STEP : 0;
  if (ntiles > 0) {
    dense_issue<D>(kbase, vbase, a.k_ss, a.v_ss, a.S, t, t_end, lane, kA, st0);
    for (int it = 0;; it += 2) {
      dense_issue<D>(kbase, vbase, a.k_ss, a.v_ss, a.S, t + STEP, t_end, lane, kB, st1);
      BYTES_WAIT_VMCNT(NLOAD);
      __asm__ volatile("" ::: "memory");
      dense_tile<D>(t, t_end, a.scale_log2, lane, qb, kA, st0, m_run, l_run, acc);
      t += STEP;
      if (it + 1 >= ntiles) break;
      dense_issue<D>(kbase, vbase, a.k_ss, a.v_ss, a.S, t + STEP, t_end, lane, kA, st0);
      BYTES_WAIT_VMCNT(NLOAD);
      __asm__ volatile("" ::: "memory");
      dense_tile<D>(t, t_end, a.scale_log2, lane, qb, kB, st1, m_run, l_run, acc);
      t += STEP;
      if (it + 2 >= ntiles) break;
    }
    // the last prefetch (a dummy) may still be landing in LDS: drain it
    BYTES_WAIT_VMCNT(0);
    __asm__ volatile("" ::: "memory");
  }

  splitk_epilogue<D, kDenseWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b,
                                  hq0, nh);
}

// Host-side split choice: chunk is a multiple of (waves * tile) tokens; aim
// for two resident workgroups per CU.
static void dense_plan(int S, long units, int chunk_req, int* chunk, int* nsplit) {
  const int step = kDenseWaves * kTile;
  int c;
  if (chunk_req > 0) {
    c = (chunk_req + step - 1) / step * step;
  } else {
    const long target = 2L * device_cu_count();
    long per = ((long)S * units + target - 1) / target;
    c = (int)((per + step - 1) / step * step);
    if (c < step) c = step;
  }
  int ns = (S + c - 1) / c;
  if (ns > 256) {  // the merge keeps one weight per split in LDS
    c = ((S + 255) / 256 + step - 1) / step * step;
    ns = (S + c - 1) / c;
  }
  *chunk = c;
  *nsplit = ns;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_decode_attn_bf16_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk_req, size_t* bytes) {
  if (!bytes || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0 || (D != 64 && D != 128)) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  int chunk, ns;
  dense_plan(S, units, chunk_req, &chunk, &ns);
  *bytes = splitk_workspace_bytes(units, ns, D);
  return 0;
}

int bytes_decode_attn_bf16(const void* q, const void* k, const void* v, void* out, int B, int Hq, int Hk, int S,
                           int D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scale,
                           int chunk_req, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  if (units > 65535) return (int)hipErrorInvalidConfiguration;
  DenseArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.Hk = Hk; a.G = G; a.S = S; a.HB = HB;
  a.scale_log2 = scale * kLog2e;
  int ns;
  dense_plan(S, units, chunk_req, &a.chunk, &ns);
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  a.o.out = out;
  a.o.out_dtype = kOutBF16;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  a.o.Hk = Hk; a.o.HB = HB; a.o.G = G;
  splitk_carve(workspace, units, ns, a.o);
  dim3 grid(ns, (unsigned)units);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 64)
    hipLaunchKernelGGL(dense_decode_kernel<64>, grid, dim3(kDenseWaves * 64), 0, st, a);
  else
    hipLaunchKernelGGL(dense_decode_kernel<128>, grid, dim3(kDenseWaves * 64), 0, st, a);
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

}  // extern "C"
