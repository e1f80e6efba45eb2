// Quest page metadata and page bounds.
//
// Replaces the page part of benchmarks/sparse_attention.py:328-364
// (`_quest_select`; dense form benchmarks/eval_ppl.py:54-79):
//  * per-page elementwise min/max of the keys over pages of `page` tokens,
//    the last partial page padded with the last key (:336-341);
//  * bound[b, h, p] = scaling * sum_d max(q_d * kmin_d, q_d * kmax_d) in fp32
//    (:342-345), -inf for pages that start after the query position
//    (:346-348) and +inf for pages overlapping the recent window of
//    `local_w` tokens (:349-355).
// The products of bf16 values are exact in fp32 and every thread sums its
// page's terms in ascending d, so the bounds are bit-identical to a
// sequential fp32 evaluation (up to the sign of an all-zero bound, which
// ranks the same); the page top-k that follows is then bit-exact.
#include "common.h"

namespace bytes_amd {

// NaN-propagating min / max (torch.amin / amax semantics).
__device__ __forceinline__ float nmin(float a, float b) { return (a < b || a != a) ? a : b; }
__device__ __forceinline__ float nmax(float a, float b) { return (a > b || a != a) ? a : b; }

// One thread per (b, hk, page, 8-dim chunk).
__global__ void quest_minmax_kernel(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, int Hk, int S,
                                    int D, int page, int np, uint16_t* kmin, uint16_t* kmax) {
  const int chunks = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (gid >= (int64_t)Hk * np * chunks) return;
  const int c = (int)(gid % chunks);
  const int64_t r = gid / chunks;
  const int p = (int)(r % np);
  const int hk = (int)(r / np);
  const uint16_t* base = k + (int64_t)b * k_sb + (int64_t)hk * k_sh + c * 8;
  float mn[8], mx[8];
  for (int o = 0; o < page; ++o) {
    const int t = min(p * page + o, S - 1);
    const u32x4 raw = ld16(base + (int64_t)t * k_ss);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = bf16_bits_to_f32(h[j]);
      mn[j] = o == 0 ? v : nmin(mn[j], v);
      mx[j] = o == 0 ? v : nmax(mx[j], v);
    }
  }
  u32x4 omn, omx;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // min/max of bf16 values are bf16 values: truncation is exact
    omn[j] = (__float_as_uint(mn[2 * j]) >> 16) | (__float_as_uint(mn[2 * j + 1]) & 0xFFFF0000u);
    omx[j] = (__float_as_uint(mx[2 * j]) >> 16) | (__float_as_uint(mx[2 * j + 1]) & 0xFFFF0000u);
  }
  const int64_t o = (((int64_t)b * Hk + hk) * np + p) * D + c * 8;
  *reinterpret_cast<u32x4*>(kmin + o) = omn;
  *reinterpret_cast<u32x4*>(kmax + o) = omx;
}

constexpr int kQuestThreads = 256;
constexpr int kQuestPages = 32;                    // pages per workgroup
constexpr int kQuestSlots = kQuestThreads / kQuestPages;   // head slots per round

// One workgroup per (b, kv head, head block of 16, 32 pages); thread (page
// t % 32, head slot t / 32).  The pages' min/max rows are widened to fp32 in
// LDS (rows padded by 16 bytes, so the 16 pages a 16-lane group reads at one d
// sit in distinct banks) and q is split into q+ = q (q >= 0 or NaN, else 0)
// and q- = q (q < 0, else 0).  On a page whose min/max rows are finite each
// term is fma(q-_d, kmin_d, q+_d * kmax_d): one of the two products is an
// exact zero, so the term is the rounded product max(q_d*kmin_d,
// q_d*kmax_d) picks (kmax >= kmin).  A page with an infinite or NaN min/max
// entry (a key with one) takes the literal form max(q*kmin, q*kmax), NaN if
// either product is (torch.maximum): there 0 * inf on the side q does not
// pick would otherwise turn the term into NaN.  Terms are summed in
// ascending d.
template <int D>
__global__ __launch_bounds__(kQuestThreads) void quest_score_kernel(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                                                    const uint16_t* kmin, const uint16_t* kmax,
                                                                    int Hk, int G, int HB, int np, int page,
                                                                    int pos, int local_w, float scale,
                                                                    float* bound, int64_t o_sb, int64_t o_sh) {
  constexpr int PITCH = D + 4;                     // floats per padded row
  __shared__ __attribute__((aligned(16))) float mn_s[kQuestPages * PITCH];
  __shared__ __attribute__((aligned(16))) float mx_s[kQuestPages * PITCH];
  __shared__ __attribute__((aligned(16))) float qp_s[16 * D];
  __shared__ __attribute__((aligned(16))) float qm_s[16 * D];
  __shared__ uint32_t bad_s[kQuestPages];          // per page: a non-finite min/max entry
  const int parts = (np + kQuestPages - 1) / kQuestPages;
  const int bhb = blockIdx.x / parts, part = blockIdx.x - (blockIdx.x / parts) * parts;
  const int bh = bhb / HB, hb = bhb - (bhb / HB) * HB;
  const int b = bh / Hk, hk = bh - (bh / Hk) * Hk;
  const int p0 = part * kQuestPages;
  // this workgroup's heads: query heads hk*G + g0 .. + GB - 1 (blocks of 16)
  const int g0 = hb * 16, GB = min(16, G - g0);
  // Every load is issued before any LDS store that consumes one (indices
  // clamped, so no load sits under a lane mask): one memory round trip.
  constexpr int CH = D / 8;                        // 16-byte chunks per row
  constexpr int QPT = (16 * CH + kQuestThreads - 1) / kQuestThreads;   // q chunks per thread (16 heads)
  constexpr int MPT = kQuestPages * CH / kQuestThreads;   // min/max chunks per thread
  static_assert(QPT >= 1 && MPT >= 1, "chunks per thread");
  u32x4 qv[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = min((int)threadIdx.x + u * kQuestThreads, 16 * CH - 1);
    const int g = min(e / CH, GB - 1), c = e - (e / CH) * CH;
    qv[u] = ld16(q + (int64_t)b * q_sb + (int64_t)(hk * G + g0 + g) * q_sh + c * 8);
  }
  const int64_t row0 = ((int64_t)b * Hk + hk) * np;
  u32x4 av[MPT], zv[MPT];
#pragma unroll
  for (int u = 0; u < MPT; ++u) {
    const int e = threadIdx.x + u * kQuestThreads;
    const int pp = e / CH, c = e - (e / CH) * CH;
    const int64_t r = row0 + min(p0 + pp, np - 1);  // pages past np: copies nothing reads
    av[u] = ld16_nt(kmin + r * D + c * 8);
    zv[u] = ld16_nt(kmax + r * D + c * 8);
  }
  auto widen = [](const u32x4& raw, f32x4& lo4, f32x4& hi4) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      lo4[2 * j] = __uint_as_float(raw[j] << 16);
      lo4[2 * j + 1] = __uint_as_float(raw[j] & 0xFFFF0000u);
      hi4[2 * j] = __uint_as_float(raw[2 + j] << 16);
      hi4[2 * j + 1] = __uint_as_float(raw[2 + j] & 0xFFFF0000u);
    }
  };
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = min((int)threadIdx.x + u * kQuestThreads, 16 * CH - 1);   // rows past GB are unused
    const int g = e / CH, c = e - (e / CH) * CH;
    f32x4 x0, x1;
    widen(qv[u], x0, x1);
    f32x4 p0v, p1v, m0v, m1v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p0v[j] = (x0[j] >= 0.f || x0[j] != x0[j]) ? x0[j] : 0.f;
      p1v[j] = (x1[j] >= 0.f || x1[j] != x1[j]) ? x1[j] : 0.f;
      m0v[j] = x0[j] < 0.f ? x0[j] : 0.f;
      m1v[j] = x1[j] < 0.f ? x1[j] : 0.f;
    }
    *reinterpret_cast<f32x4*>(qp_s + g * D + c * 8) = p0v;
    *reinterpret_cast<f32x4*>(qp_s + g * D + c * 8 + 4) = p1v;
    *reinterpret_cast<f32x4*>(qm_s + g * D + c * 8) = m0v;
    *reinterpret_cast<f32x4*>(qm_s + g * D + c * 8 + 4) = m1v;
  }
#pragma unroll
  for (int u = 0; u < MPT; ++u) {
    const int e = threadIdx.x + u * kQuestThreads;
    const int pp = e / CH, c = e - (e / CH) * CH;
    f32x4 a0, a1, z0, z1;
    widen(av[u], a0, a1);
    widen(zv[u], z0, z1);
    *reinterpret_cast<f32x4*>(mn_s + pp * PITCH + c * 8) = a0;
    *reinterpret_cast<f32x4*>(mn_s + pp * PITCH + c * 8 + 4) = a1;
    *reinterpret_cast<f32x4*>(mx_s + pp * PITCH + c * 8) = z0;
    *reinterpret_cast<f32x4*>(mx_s + pp * PITCH + c * 8 + 4) = z1;
    // a bf16 exponent field of all ones: infinity or NaN.  Per half word,
    // (h & 0x7F80) + 0x80 reaches bit 15 only then (no carry crosses halves);
    // a page's CH chunks sit on CH consecutive lanes
    uint32_t ex = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ex |= ((av[u][j] & 0x7F807F80u) + 0x00800080u) | ((zv[u][j] & 0x7F807F80u) + 0x00800080u);
    const unsigned long long m = __ballot((ex & 0x80008000u) != 0u);
    const int lane = threadIdx.x & 63;
    if (c == 0) bad_s[pp] = ((m >> (lane & (64 - CH))) & ((1ull << CH) - 1ull)) ? 1u : 0u;
  }
  __syncthreads();
  const int pp = threadIdx.x % kQuestPages;
  const int p = p0 + pp;
  if (p >= np) return;
  // causal validity and the forced recent window, at page granularity
  const bool valid = (int64_t)p * page <= pos;
  bool recent = false;
  if (local_w > 0) {
    const int lo = max(pos - local_w + 1, 0) / page, hi = pos / page;
    recent = p >= lo && p <= hi;
  }
  const float* mnr = mn_s + pp * PITCH;
  const float* mxr = mx_s + pp * PITCH;
  const uint32_t nonfinite = bad_s[pp];
  for (int g = threadIdx.x / kQuestPages; g < GB; g += kQuestSlots) {
    const float* qpr = qp_s + g * D;
    const float* qmr = qm_s + g * D;
    float acc = 0.f;
    if (!nonfinite) {
#pragma clang fp contract(off)
#pragma unroll 4
      for (int d4 = 0; d4 < D / 4; ++d4) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(mnr + 4 * d4);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(mxr + 4 * d4);
        const f32x4 qp = *reinterpret_cast<const f32x4*>(qpr + 4 * d4);
        const f32x4 qm = *reinterpret_cast<const f32x4*>(qmr + 4 * d4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float hp = qp[e] * hi[e];
          const float t = __builtin_fmaf(qm[e], lo[e], hp);
          acc = (d4 == 0 && e == 0) ? t : acc + t;
        }
      }
    } else {
#pragma clang fp contract(off)
      for (int d = 0; d < D; ++d) {
        const float qd = qpr[d] + qmr[d];          // one of the two is an exact zero
        const float a = qd * mnr[d], z = qd * mxr[d];
        const float t = (a != a || z != z) ? __builtin_nanf("") : (a > z ? a : z);
        acc = d == 0 ? t : acc + t;
      }
    }
    float v = acc * scale;
    if (!valid) v = kNegInf;
    if (recent) v = __builtin_inff();
    bound[(int64_t)b * o_sb + (int64_t)(hk * G + g0 + g) * o_sh + p] = v;
  }
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_quest_page_minmax(const void* k, void* kmin, void* kmax, int B, int Hk, int S, int D, int page,
                            int64_t k_sb, int64_t k_sh, int64_t k_ss, void* stream) {
  if (!k || !kmin || !kmax || B <= 0 || Hk <= 0 || S <= 0 || page <= 0 || D <= 0 || D % 8 != 0)
    return (int)hipErrorInvalidValue;
  if (B > 65535) return (int)hipErrorInvalidConfiguration;
  const int np = (S + page - 1) / page;
  const int64_t per_b = (int64_t)Hk * np * (D / 8);
  const int th = 256;
  dim3 grid((unsigned)((per_b + th - 1) / th), (unsigned)B);
  hipLaunchKernelGGL(quest_minmax_kernel, grid, dim3(th), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(k), k_sb, k_sh, k_ss, Hk, S, D, page, np,
                     static_cast<uint16_t*>(kmin), static_cast<uint16_t*>(kmax));
  return (int)hipGetLastError();
}

int bytes_quest_page_scores(const void* q, const void* kmin, const void* kmax, void* bound, int B, int Hq, int Hk,
                            int np, int D, int page, int pos, int local_w, int64_t q_sb, int64_t q_sh,
                            int64_t o_sb, int64_t o_sh, float scale, void* stream) {
  if (!q || !kmin || !kmax || !bound || B <= 0 || Hk <= 0 || Hq % Hk != 0 || np <= 0 || page <= 0)
    return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  const int parts = (np + kQuestPages - 1) / kQuestPages;
  const long grid = (long)B * Hk * HB * parts;
  if (grid > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* qq = static_cast<const uint16_t*>(q);
  const uint16_t* mn = static_cast<const uint16_t*>(kmin);
  const uint16_t* mx = static_cast<const uint16_t*>(kmax);
  float* o = static_cast<float*>(bound);
  if (D == 128)
    BYTES_LAUNCH(kProfQuest, quest_score_kernel<128>, dim3((unsigned)grid), dim3(kQuestThreads), 0, st, qq, q_sb, q_sh,
                       mn, mx, Hk, G, HB, np, page, pos, local_w, scale, o, o_sb, o_sh);
  else
    BYTES_LAUNCH(kProfQuest, quest_score_kernel<64>, dim3((unsigned)grid), dim3(kQuestThreads), 0, st, qq, q_sb, q_sh,
                       mn, mx, Hk, G, HB, np, page, pos, local_w, scale, o, o_sb, o_sh);
  return (int)hipGetLastError();
}

}  // extern "C"
