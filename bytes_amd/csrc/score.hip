// Token scoring: fp32 q.k scores of every cached key.
//
// Replaces src/attention_kernels.py:1077-1133 (`sparse_score_scalar`,
// scores[b, h, t] = (q[b, h] . k[b, h // G, t]) * scaling for bf16 keys) and
// adds the group-summed score of the token top-k pipeline,
// s[b, hk, t] = sum_{g < G} scores[b, hk*G + g, t] (g ascending), the
// selection score of one KV head shared by its query group.
//
// The query heads of a GQA group are scored together: one
// v_mfma_f32_16x16x32_bf16 computes S[h][t] for 16 heads x 16 tokens with
// A = Q (heads as rows) and B = K^T (tokens as columns).  Both operands use
// the same permutation of the contraction index: at k-step kk, lane l holds
// dims (kk*4 + l/16)*8 .. +8 of its row, so a lane's four k-steps cover 64
// contiguous bytes of one key row and each key row is read by 16-byte loads
// straight from HBM into the MFMA operand registers (no LDS round trip).  The
// output tile lands with head (l/16)*4 + i and token l%16 in lane l, so the
// group sum of up to four heads is a sum inside one lane.
//
// fp8 (OCP e4m3fn) keys (`score_bits=8`, :1113) load 8 bytes per operand and
// are widened to bf16 exactly in registers.
#include "dense_tile.h"

namespace bytes_amd {

struct ScoreArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const void* k;             // bf16 or fp8 e4m3fn keys
  int64_t k_sb, k_sh, k_ss;
  float* out;                // [B, Hq, S] (per head) or [B, Hk, S] (group sum); unit stride along S
  int64_t o_sb, o_sh;
  uint32_t* hist;            // group sum only, optional: [B*Hk][2048] counts of the top 11 key bits
  int Hk, G, HB, S, tok_per_wg, parts, group_sum;
  float scaling;
};

constexpr int kScoreWaves = 4;
constexpr int kScoreIter = 64;   // tokens per wave iteration (4 MFMA column tiles)

template <int D, bool FP8>
struct ScoreRegs {
  typedef typename std::conditional<FP8, u32x2, u32x4>::type T;
  T k[4][D / 32];            // [column tile][k-step]
};

// K rows t .. t+63 of one iteration as B operands (rows clamped to S-1).
template <int D, bool FP8>
__device__ __forceinline__ void score_issue(const void* kbase, int64_t k_ss, int S, int t, int lane,
                                            ScoreRegs<D, FP8>& r) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int row = min(t + c * 16 + l16, S - 1);
    if constexpr (FP8) {
      const uint8_t* p = static_cast<const uint8_t*>(kbase) + (int64_t)row * k_ss + lg * 8;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) r.k[c][kk] = *reinterpret_cast<const u32x2*>(p + kk * 32);
    } else {
      const uint16_t* p = static_cast<const uint16_t*>(kbase) + (int64_t)row * k_ss + lg * 8;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) r.k[c][kk] = ld16(p + kk * 32);
    }
  }
}

template <bool FP8>
__device__ __forceinline__ bf16x8 score_operand(const u32x4& w) { return __builtin_bit_cast(bf16x8, w); }
template <bool FP8>
__device__ __forceinline__ bf16x8 score_operand(const u32x2& w) {
  const u32x4 b = {fp8x2_to_bf16x2<false>(w[0]), fp8x2_to_bf16x2<true>(w[0]), fp8x2_to_bf16x2<false>(w[1]),
                   fp8x2_to_bf16x2<true>(w[1])};
  return __builtin_bit_cast(bf16x8, b);
}

template <int D, bool FP8>
__device__ __forceinline__ void score_tile(const ScoreRegs<D, FP8>& r, const bf16x8 (&qa)[D / 32], int t, int lane,
                                           const ScoreArgs& a, int b, int hk, int hq0, int nh, uint32_t* hlds) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) s = mfma_bf16(qa[kk], score_operand<FP8>(r.k[c][kk]), s);
    const int tok = t + c * 16 + l16;
    if (a.group_sum) {
      // heads lg*4 + i; group sum in head order, lane groups added in order
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (lg * 4 + i < nh) part += s[i] * a.scaling;
      const float p1 = __shfl(part, l16 + 16, 64);
      const float p2 = __shfl(part, l16 + 32, 64);
      const float p3 = __shfl(part, l16 + 48, 64);
      float tot = part;
      if (nh > 4) tot += p1;
      if (nh > 8) tot += p2;
      if (nh > 12) tot += p3;
      if (lg == 0 && tok < a.S) {
        a.out[(int64_t)b * a.o_sb + (int64_t)hk * a.o_sh + tok] = tot;
        if (hlds) atomicAdd(&hlds[score_order_key(tot) >> 21], 1u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = lg * 4 + i;
        if (h < nh && tok < a.S) a.out[(int64_t)b * a.o_sb + (int64_t)(hq0 + h) * a.o_sh + tok] = s[i] * a.scaling;
      }
    }
  }
}

template <int D, bool FP8>
__global__ __launch_bounds__(kScoreWaves * 64, 2) void score_kernel(ScoreArgs a) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int unit = blockIdx.x / a.parts, part = blockIdx.x - unit * a.parts;
  const int b = unit / (a.Hk * a.HB);
  const int rem = unit - b * a.Hk * a.HB;
  const int hk = rem / a.HB, hb = rem - (rem / a.HB) * a.HB;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);

  // Q as the A operand: lane holds Q[h = l16][dims (kk*4 + lg)*8 .. +8]
  bf16x8 qa[D / 32];
  {
    const bool live = l16 < nh;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hq0 + (live ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) qa[kk] = __builtin_bit_cast(bf16x8, live ? ld16(qp + kk * 32) : u32x4{0, 0, 0, 0});
  }

  const void* kbase = FP8 ? (const void*)(static_cast<const uint8_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh)
                          : (const void*)(static_cast<const uint16_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh);
  const int t_begin = part * a.tok_per_wg;
  const int t_end = min(t_begin + a.tok_per_wg, a.S);
  constexpr int STEP = kScoreWaves * kScoreIter;
  __shared__ uint32_t hlds_mem[2048];
  uint32_t* hlds = nullptr;
  if (a.hist) {
    for (int i = threadIdx.x; i < 2048; i += kScoreWaves * 64) hlds_mem[i] = 0u;
    __syncthreads();
    hlds = hlds_mem;
  }
  int t = t_begin + w * kScoreIter;
  if (t < t_end) {
    // two register sets: the next iteration's rows are in flight while one is scored
    ScoreRegs<D, FP8> r0, r1;
    score_issue<D, FP8>(kbase, a.k_ss, a.S, t, lane, r0);
    while (true) {
      const bool more1 = t + STEP < t_end;
      score_issue<D, FP8>(kbase, a.k_ss, a.S, more1 ? t + STEP : t, lane, r1);
      score_tile<D, FP8>(r0, qa, t, lane, a, b, hk, hq0, nh, hlds);
      t += STEP;
      if (!more1) break;
      const bool more0 = t + STEP < t_end;
      score_issue<D, FP8>(kbase, a.k_ss, a.S, more0 ? t + STEP : t, lane, r0);
      score_tile<D, FP8>(r1, qa, t, lane, a, b, hk, hq0, nh, hlds);
      t += STEP;
      if (!more0) break;
    }
  }
  if (a.hist) {
    __syncthreads();
    uint32_t* hr = a.hist + ((int64_t)b * a.Hk + hk) * 2048;
    for (int i = threadIdx.x; i < 2048; i += kScoreWaves * 64)
      if (hlds_mem[i]) atomicAdd(hr + i, hlds_mem[i]);
  }
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_sparse_score(const void* q, const void* k, int k_fp8, void* out, int B, int Hq, int Hk, int S, int D,
                       int group_sum, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                       int64_t o_sb, int64_t o_sh, float scaling, void* hist, void* stream) {
  if (!q || !k || !out || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  ScoreArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.out = static_cast<float*>(out);
  a.o_sb = o_sb; a.o_sh = o_sh;
  a.hist = static_cast<uint32_t*>(hist);
  a.Hk = Hk; a.G = Hq / Hk; a.HB = (a.G + 15) / 16; a.S = S;
  a.group_sum = group_sum ? 1 : 0;
  if (a.group_sum && a.G > 16) return (int)hipErrorNotSupported;
  if (a.hist && !a.group_sum) return (int)hipErrorInvalidValue;
  a.scaling = scaling;
  const long units = (long)B * Hk * a.HB;
  // about 8 workgroups per CU in total, each a multiple of one iteration of all waves
  const long target = 8L * device_cu_count();
  const int step = kScoreWaves * kScoreIter;
  long per = ((long)S * units + target - 1) / target;
  per = (per + step - 1) / step * step;
  if (per < step) per = step;
  if (per > 8192) per = 8192;
  a.tok_per_wg = (int)per;
  a.parts = (int)((S + per - 1) / per);
  const long grid = units * a.parts;
  if (grid > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)grid), blk(kScoreWaves * 64);
  if (D == 128) {
    if (k_fp8) hipLaunchKernelGGL((score_kernel<128, true>), g, blk, 0, st, a);
    else hipLaunchKernelGGL((score_kernel<128, false>), g, blk, 0, st, a);
  } else {
    if (k_fp8) hipLaunchKernelGGL((score_kernel<64, true>), g, blk, 0, st, a);
    else hipLaunchKernelGGL((score_kernel<64, false>), g, blk, 0, st, a);
  }
  return (int)hipGetLastError();
}

}  // extern "C"
