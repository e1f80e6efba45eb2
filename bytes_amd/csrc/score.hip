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
//
// Packed 4/2-bit keys (`sparse_score_packed`, :1136-1222; layout of
// `quantize_and_pack_score_keys`, :1225-1249: codes along head_dim, two or
// four per byte, bf16 scale/min per 32-dim group) are scored group by group:
// k-step kk of the MFMA covers exactly group kk, so
//   score = sum_kk scale_kk * (q . code)_kk + min_kk * (sum of q over group kk)
// with the integer codes as exact bf16 operands and both terms in fp32.
#include "dense_tile.h"

namespace bytes_amd {

enum KeyMode : int { kKeyBf16 = 0, kKeyFp8 = 1, kKeyP4 = 2, kKeyP2 = 3 };

struct ScoreArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const void* k;             // bf16, fp8 e4m3fn or packed codes (strides in storage elements)
  int64_t k_sb, k_sh, k_ss;
  const uint16_t* ksc;       // packed modes: bf16 scale / min [B, Hk, S, D/32]
  const uint16_t* kmn;
  int64_t m_sb, m_sh, m_ss;
  float* out;                // [B, Hq, S] (per head) or [B, Hk, S] (group sum); unit stride along S
  int64_t o_sb, o_sh;
  uint32_t* hist;            // group sum only, optional: [B*Hk][2048] counts of the top 11 key bits
  int Hk, G, HB, S, tok_per_wg, parts, group_sum;
  float scaling;
};

constexpr int kScoreWaves = 4;
constexpr int kScoreIter = 64;   // tokens per wave iteration (4 MFMA column tiles)

template <int D, int KM>
struct ScoreRegs {
  typedef typename std::conditional<KM == kKeyBf16, u32x4,
                                    typename std::conditional<KM == kKeyFp8, u32x2, uint32_t>::type>::type T;
  T k[4][D / 32];            // [column tile][k-step]
  u32x2 sc[KM >= kKeyP4 ? 4 : 1], mn[KM >= kKeyP4 ? 4 : 1];   // packed: bf16 scale/min of the 4 groups
};

// K rows t .. t+63 of one iteration as B operands (rows clamped to S-1).
template <int D, int KM>
__device__ __forceinline__ void score_issue(const ScoreArgs& a, const void* kbase, const uint16_t* scb,
                                            const uint16_t* mnb, int t, int lane, ScoreRegs<D, KM>& r) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int row = min(t + c * 16 + l16, a.S - 1);
    if constexpr (KM == kKeyFp8) {
      const uint8_t* p = static_cast<const uint8_t*>(kbase) + (int64_t)row * a.k_ss + lg * 8;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) r.k[c][kk] = *reinterpret_cast<const u32x2*>(p + kk * 32);
    } else if constexpr (KM == kKeyBf16) {
      const uint16_t* p = static_cast<const uint16_t*>(kbase) + (int64_t)row * a.k_ss + lg * 8;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) r.k[c][kk] = ld16(p + kk * 32);
    } else {
      // group kk, dims kk*32 + lg*8 .. +8: 4 bytes (4-bit) or 2 bytes (2-bit)
      constexpr int GB = KM == kKeyP4 ? 16 : 8;          // bytes per group
      const uint8_t* p = static_cast<const uint8_t*>(kbase) + (int64_t)row * a.k_ss;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        if constexpr (KM == kKeyP4)
          r.k[c][kk] = *reinterpret_cast<const uint32_t*>(p + kk * GB + lg * 4);
        else
          r.k[c][kk] = *reinterpret_cast<const uint16_t*>(p + kk * GB + lg * 2);
      }
      // D/32 bf16 values per row: 8 bytes at D = 128, 4 bytes at D = 64
      if constexpr (D == 128) {
        r.sc[c] = *reinterpret_cast<const u32x2*>(scb + (int64_t)row * a.m_ss);
        r.mn[c] = *reinterpret_cast<const u32x2*>(mnb + (int64_t)row * a.m_ss);
      } else {
        r.sc[c] = u32x2{*reinterpret_cast<const uint32_t*>(scb + (int64_t)row * a.m_ss), 0u};
        r.mn[c] = u32x2{*reinterpret_cast<const uint32_t*>(mnb + (int64_t)row * a.m_ss), 0u};
      }
    }
  }
}

template <int KM>
__device__ __forceinline__ bf16x8 score_operand(const u32x4& w) { return __builtin_bit_cast(bf16x8, w); }
template <int KM>
__device__ __forceinline__ bf16x8 score_operand(const u32x2& w) {
  const u32x4 b = {fp8x2_to_bf16x2<false>(w[0]), fp8x2_to_bf16x2<true>(w[0]), fp8x2_to_bf16x2<false>(w[1]),
                   fp8x2_to_bf16x2<true>(w[1])};
  return __builtin_bit_cast(bf16x8, b);
}
// 8 packed codes (4 or 2 bits each, element j at bits j*bits) -> 8 exact bf16 integers
template <int KM>
__device__ __forceinline__ bf16x8 score_operand(const uint32_t& w) {
  constexpr int BITS = KM == kKeyP4 ? 4 : 2;
  u32x4 b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float c0 = (float)((w >> (2 * j * BITS)) & ((1u << BITS) - 1u));
    const float c1 = (float)((w >> ((2 * j + 1) * BITS)) & ((1u << BITS) - 1u));
    b[j] = (__float_as_uint(c0) >> 16) | (__float_as_uint(c1) & 0xFFFF0000u);
  }
  return __builtin_bit_cast(bf16x8, b);
}

__device__ __forceinline__ float bf16_at(const u32x2& v, int i) {
  const uint32_t w = v[i >> 1];
  return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

template <int D, int KM>
__device__ __forceinline__ void score_tile(const ScoreRegs<D, KM>& r, const bf16x8 (&qa)[D / 32],
                                           const f32x4 (&qsum)[D / 32], int t, int lane, const ScoreArgs& a, int b,
                                           int hk, int hq0, int nh, uint32_t* hlds) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KM >= kKeyP4) {
      // per group: scale * (q . code) + min * (sum of q), groups in order
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        const f32x4 g = mfma_bf16(qa[kk], score_operand<KM>(r.k[c][kk]), f32x4{0.f, 0.f, 0.f, 0.f});
        const float sc = bf16_at(r.sc[c], kk), mn = bf16_at(r.mn[c], kk);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] += sc * g[i] + mn * qsum[kk][i];
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) s = mfma_bf16(qa[kk], score_operand<KM>(r.k[c][kk]), s);
    }
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

template <int D, int KM>
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

  const void* kbase =
      KM == kKeyBf16 ? (const void*)(static_cast<const uint16_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh)
                     : (const void*)(static_cast<const uint8_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh);
  const uint16_t* scb = KM >= kKeyP4 ? a.ksc + (int64_t)b * a.m_sb + (int64_t)hk * a.m_sh : nullptr;
  const uint16_t* mnb = KM >= kKeyP4 ? a.kmn + (int64_t)b * a.m_sb + (int64_t)hk * a.m_sh : nullptr;
  // packed keys: sum of q over each 32-dim group, in the output layout (head lg*4+i)
  f32x4 qsum[D / 32];
  if constexpr (KM >= kKeyP4) {
    const u32x4 one = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0 x 8
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk)
      qsum[kk] = mfma_bf16(qa[kk], __builtin_bit_cast(bf16x8, one), f32x4{0.f, 0.f, 0.f, 0.f});
  }
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
    ScoreRegs<D, KM> r0, r1;
    score_issue<D, KM>(a, kbase, scb, mnb, t, lane, r0);
    while (true) {
      const bool more1 = t + STEP < t_end;
      score_issue<D, KM>(a, kbase, scb, mnb, more1 ? t + STEP : t, lane, r1);
      score_tile<D, KM>(r0, qa, qsum, t, lane, a, b, hk, hq0, nh, hlds);
      t += STEP;
      if (!more1) break;
      const bool more0 = t + STEP < t_end;
      score_issue<D, KM>(a, kbase, scb, mnb, more0 ? t + STEP : t, lane, r0);
      score_tile<D, KM>(r1, qa, qsum, t, lane, a, b, hk, hq0, nh, hlds);
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

int bytes_sparse_score(const void* q, const void* k, int k_mode, const void* k_scale, const void* k_min, void* out,
                       int B, int Hq, int Hk, int S, int D, int group_sum, int64_t q_sb, int64_t q_sh, int64_t k_sb,
                       int64_t k_sh, int64_t k_ss, int64_t m_sb, int64_t m_sh, int64_t m_ss, int64_t o_sb,
                       int64_t o_sh, float scaling, void* hist, void* stream) {
  if (!q || !k || !out || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  if (k_mode < kKeyBf16 || k_mode > kKeyP2) return (int)hipErrorInvalidValue;
  if (k_mode >= kKeyP4 && (!k_scale || !k_min)) return (int)hipErrorInvalidValue;
  ScoreArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.ksc = static_cast<const uint16_t*>(k_scale);
  a.kmn = static_cast<const uint16_t*>(k_min);
  a.m_sb = m_sb; a.m_sh = m_sh; a.m_ss = m_ss;
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
#define SCORE_LAUNCH(DD, KMV) hipLaunchKernelGGL((score_kernel<DD, KMV>), g, blk, 0, st, a)
  if (D == 128) {
    switch (k_mode) {
      case kKeyBf16: SCORE_LAUNCH(128, kKeyBf16); break;
      case kKeyFp8: SCORE_LAUNCH(128, kKeyFp8); break;
      case kKeyP4: SCORE_LAUNCH(128, kKeyP4); break;
      default: SCORE_LAUNCH(128, kKeyP2); break;
    }
  } else {
    switch (k_mode) {
      case kKeyBf16: SCORE_LAUNCH(64, kKeyBf16); break;
      case kKeyFp8: SCORE_LAUNCH(64, kKeyFp8); break;
      case kKeyP4: SCORE_LAUNCH(64, kKeyP4); break;
      default: SCORE_LAUNCH(64, kKeyP2); break;
    }
  }
#undef SCORE_LAUNCH
  return (int)hipGetLastError();
}

// Quantize and pack score keys along head_dim (src/attention_kernels.py:1225-1249):
// per row and group of 32, scale = max(hi - lo, 1e-8) / (2^bits - 1) and
// code = clamp(rint((x - lo) / scale)) in fp32; scale and lo stored in x's
// dtype (round to nearest even).
__device__ __forceinline__ void store_as(void* p, int64_t i, int dtype, float v) {
  if (dtype == 0)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else if (dtype == 1)
    static_cast<_Float16*>(p)[i] = (_Float16)v;
  else
    static_cast<float*>(p)[i] = v;
}

__global__ void score_pack_kernel(const void* x, int x_dtype, int64_t rows, int D, int64_t x_rs, int bits,
                                  uint8_t* packed, void* scale, void* mn) {
  const int ng = D / 32;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * ng) return;
  const int64_t row = gid / ng;
  const int g = (int)(gid - row * ng);
  const int64_t base = row * x_rs + g * 32;
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    v[i] = x_dtype == 0 ? bf16_bits_to_f32(static_cast<const uint16_t*>(x)[base + i])
                        : (x_dtype == 1 ? (float)static_cast<const _Float16*>(x)[base + i]
                                        : static_cast<const float*>(x)[base + i]);
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
  const int levels = 1 << bits;
  const float s = fmaxf(hi - lo, 1e-8f) / (float)(levels - 1);
  const int per = 8 / bits;
  uint8_t* out = packed + row * (int64_t)(D * bits / 8) + g * (32 * bits / 8);
  for (int byte = 0; byte < 32 / per; ++byte) {
    uint32_t w = 0;
    for (int i = 0; i < per; ++i) {
      float c = rintf((v[byte * per + i] - lo) / s);
      c = fminf(fmaxf(c, 0.f), (float)(levels - 1));
      w |= (uint32_t)c << (i * bits);
    }
    out[byte] = (uint8_t)w;
  }
  store_as(scale, row * ng + g, x_dtype, s);
  store_as(mn, row * ng + g, x_dtype, lo);
}

int bytes_score_keys_pack(const void* x, int x_dtype, int64_t rows, int D, int64_t x_row_stride, int bits,
                          void* packed, void* scale, void* mn, void* stream) {
  if (!x || !packed || !scale || !mn || rows < 0 || D <= 0 || D % 32 != 0 || (bits != 4 && bits != 2) ||
      x_dtype < 0 || x_dtype > 2)
    return (int)hipErrorInvalidValue;
  const int64_t n = rows * (D / 32);
  if (n == 0) return 0;
  const int th = 256;
  hipLaunchKernelGGL(score_pack_kernel, dim3((unsigned)((n + th - 1) / th)), dim3(th), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, rows, D, x_row_stride, bits,
                     static_cast<uint8_t*>(packed), scale, mn);
  return (int)hipGetLastError();
}

}  // extern "C"
