// Deterministic merge of split-K flash-decode partials (see splitk.h).
//
// One workgroup per (unit, head): out = sum_s f_s acc_s / sum_s f_s l_s with
// f_s = 2^(m_s - max_s m_s).  Splits are assigned to thread groups by a fixed
// rule and the group sums are added in a fixed order, so the result is
// bit-reproducible run to run.
#include "splitk.h"

namespace bytes_amd {

constexpr int kCombineThreads = 256;
constexpr int kSplitMax = 1024;
constexpr int kSplitPerLane = kSplitMax / 64;

template <int D>
__global__ __launch_bounds__(kCombineThreads) void splitk_combine_kernel(SplitKOut o) {
  constexpr int ITEMS = D / 4;                      // float4 items per head row
  constexpr int GROUPS = kCombineThreads / ITEMS;   // split groups
  constexpr int PF = 8;                             // acc loads per thread issued up front
  __shared__ float fw[kSplitMax];
  __shared__ float red[2][64];
  __shared__ float4 gacc[GROUPS][ITEMS];
  const int unit = blockIdx.x, h = blockIdx.y;
  const int b = unit / (o.Hk * o.HB);
  const int rem = unit - b * o.Hk * o.HB;
  const int hk = rem / o.HB, hb = rem - (rem / o.HB) * o.HB;
  const int nh = min(o.hbs, o.G - hb * o.hbs);
  if (h >= nh) return;
  const int ns = o.nsplit, tid = threadIdx.x, lane = tid & 63;
  const size_t base = (size_t)unit * ns * 16 + h;

  // Issue the first PF acc rows of this thread's splits and (wave 0) every
  // split's (m, l) before consuming any of them: one memory round trip.
  const int item = tid % ITEMS, g = tid / ITEMS;
  const float4* src = reinterpret_cast<const float4*>(o.part_acc + base * D) + item;
  const size_t stride4 = (size_t)16 * D / 4;
  float4 pv[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    const int s = g + u * GROUPS;
    pv[u] = s < ns ? src[(size_t)s * stride4] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float m_loc = kNegInf;
  float mv[kSplitPerLane], lv[kSplitPerLane];
#pragma unroll
  for (int k = 0; k < kSplitPerLane; ++k) {
    const int s = lane + 64 * k;
    if (tid < 64 && s < ns) {
      const float2 ml = *reinterpret_cast<const float2*>(o.part_ml + (base + (size_t)s * 16) * 2);
      mv[k] = ml.x;
      lv[k] = ml.y;
    } else {
      mv[k] = kNegInf;
      lv[k] = 0.f;
    }
    m_loc = fmaxf(m_loc, mv[k]);
  }
  if (tid < 64) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m_loc = fmaxf(m_loc, shfl_xor_f(m_loc, off));
    const float Ms = (m_loc == kNegInf) ? 0.f : m_loc;
    float l_loc = 0.f;
#pragma unroll
    for (int k = 0; k < kSplitPerLane; ++k) {
      const int s = lane + 64 * k;
      if (s < ns) {
        const float f = fast_exp2(mv[k] - Ms);
        fw[s] = f;
        l_loc += f * lv[k];
      }
    }
    red[0][lane] = l_loc;
  }
  __syncthreads();
  if (tid == 0) {
    float L = 0.f;
    for (int i = 0; i < 64; ++i) L += red[0][i];
    red[1][0] = 1.f / L;
  }

  // weighted sum: thread (group g, item) takes splits s = g, g+GROUPS, ... in order
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    const int s = g + u * GROUPS;
    if (s < ns) {
      const float f = fw[s];
      A.x += f * pv[u].x; A.y += f * pv[u].y; A.z += f * pv[u].z; A.w += f * pv[u].w;
    }
  }
  for (int s = g + PF * GROUPS; s < ns; s += GROUPS) {
    const float4 v = src[(size_t)s * stride4];
    const float f = fw[s];
    A.x += f * v.x; A.y += f * v.y; A.z += f * v.z; A.w += f * v.w;
  }
  gacc[g][item] = A;
  __syncthreads();
  if (g == 0) {
    float4 T = gacc[0][item];
    for (int gg = 1; gg < GROUPS; ++gg) {
      const float4 v = gacc[gg][item];
      T.x += v.x; T.y += v.y; T.z += v.z; T.w += v.w;
    }
    const float il = red[1][0];
    const int hq = hk * o.G + hb * o.hbs + h, d = item * 4;
    store_out(o, b, hq, d + 0, T.x * il);
    store_out(o, b, hq, d + 1, T.y * il);
    store_out(o, b, hq, d + 2, T.z * il);
    store_out(o, b, hq, d + 3, T.w * il);
  }
}

int splitk_combine(const SplitKOut& o, long units, int D, hipStream_t stream) {
  if (o.nsplit <= 1) return 0;
  if (o.nsplit > kSplitMax) return (int)hipErrorInvalidValue;
  dim3 grid((unsigned)units, 16);
  if (D == 64)
    hipLaunchKernelGGL(splitk_combine_kernel<64>, grid, dim3(kCombineThreads), 0, stream, o);
  else if (D == 128)
    hipLaunchKernelGGL(splitk_combine_kernel<128>, grid, dim3(kCombineThreads), 0, stream, o);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

}  // namespace bytes_amd
