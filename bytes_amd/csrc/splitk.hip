// Deterministic merge of split-K flash-decode partials (see splitk.h).
//
// out = sum_s f_s acc_s / sum_s f_s l_s with f_s = 2^(m_s - max_s m_s).
//
// One wave per (unit, head, 64-dim slice of the head row), no LDS and no
// barrier.  The waves of a unit run on the XCD that ran its first split (the
// split kernels deal runs of consecutive splits to each XCD, see
// xcd_unit_split), where the partials are still in that XCD's L2: workgroup L
// of the 1-D grid goes to XCD L % 8 and takes that XCD's (L / 8)-th wave.  The
// 64 lanes are 16 float4 items of the slice x 4 split groups; lane (g, item)
// takes splits g, g+4, ... of each block of up to 128 splits, and all of a block's
// loads (the acc rows and every split's (m, l)) are issued before any is
// used, so a block costs one memory round trip.  Lanes are folded by fixed
// DPP rotations and row swaps (no LDS round trips), so the result is
// bit-reproducible run to run.
#include "splitk.h"

namespace bytes_amd {

constexpr int kSplitMax = 1024;
constexpr int kCombItems = 16;                    // float4 items per wave (64 dims)
constexpr int kCombGroups = 64 / kCombItems;      // split groups per wave

// Units whose first split is on XCD x: [first[x], first[x + 1]), for a split
// grid of units * ns workgroups mapped by xcd_unit_split.
struct XcdUnits {
  int first[kXcds + 1];
};

static XcdUnits xcd_units(long units, int ns) {
  XcdUnits m;
  const long N = units * ns, q = N / kXcds, r = N % kXcds;
  for (int x = 0; x < kXcds; ++x) {
    const long start = x * q + (x < r ? x : r);    // first split index dealt to XCD x
    m.first[x] = (int)((start + ns - 1) / ns);
  }
  m.first[kXcds] = (int)units;
  return m;
}

template <int D, int PF>
__global__ __launch_bounds__(64) void splitk_combine_kernel(SplitKOut o, XcdUnits xm) {
  constexpr int BLK = kCombGroups * PF;           // splits per block
  constexpr int MB = (BLK + 63) / 64;             // (m, l) pairs per lane per block
  constexpr int NSL = D / 64;                     // 64-dim slices per head row
  static_assert(BLK <= 128, "at most two (m, l) pairs per lane");
  const int x = blockIdx.x % kXcds, kk = blockIdx.x / kXcds;
  const int wu = (o.G < o.hbs ? o.G : o.hbs) * NSL;                  // waves per unit
  const int uk = kk / wu;
  const int unit = xm.first[x] + uk;
  if (unit >= xm.first[x + 1]) return;
  const int rw = kk - uk * wu;
  const int h = rw / NSL, slice = rw - h * NSL;
  const int b = fast_div(unit, o.dunit);
  const int rem = unit - b * o.Hk * o.HB;
  const int hk = fast_div(rem, o.dhb), hb = rem - hk * o.HB;
  const int nh = min(o.hbs, o.G - hb * o.hbs);
  if (h >= nh) return;
  const int lane = threadIdx.x, item = lane % kCombItems, g = lane / kCombItems;
  const int ns = o.nsplit;
  const size_t hrow = ((size_t)unit * 16 + h) * ns;   // row of split 0 of this head
  const float4* src = reinterpret_cast<const float4*>(o.part_acc + hrow * D) + slice * kCombItems + item;
  const float2* mlp = reinterpret_cast<const float2*>(o.part_ml) + hrow;
  constexpr int ROW4 = D / 4;

  // Block 0: every load unconditional (split index clamped to ns - 1, the
  // surplus weighted by 0), all in flight together.
  float2 mlv[MB];
  float4 pv[PF];
#pragma unroll
  for (int k = 0; k < MB; ++k) mlv[k] = mlp[min(lane + 64 * k, ns - 1)];
#pragma unroll
  for (int u = 0; u < PF; ++u) pv[u] = src[(size_t)min(g + u * kCombGroups, ns - 1) * ROW4];

  float M = kNegInf;
  if (ns <= BLK) {
#pragma unroll
    for (int k = 0; k < MB; ++k) M = fmaxf(M, lane + 64 * k < ns ? mlv[k].x : kNegInf);
  } else {
    for (int s = lane; s < ns; s += 256) {
      float m4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) m4[k] = mlp[min(s + 64 * k, ns - 1)].x;   // clamped repeats are harmless
#pragma unroll
      for (int k = 0; k < 4; ++k) M = fmaxf(M, m4[k]);
    }
  }
  M = wave_max_f32(M);
  if (M == kNegInf) M = 0.f;

  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += BLK) {
    if (s0 > 0) {
#pragma unroll
      for (int k = 0; k < MB; ++k) mlv[k] = mlp[min(s0 + lane + 64 * k, ns - 1)];
#pragma unroll
      for (int u = 0; u < PF; ++u) pv[u] = src[(size_t)min(s0 + g + u * kCombGroups, ns - 1) * ROW4];
    }
    float f[MB];
#pragma unroll
    for (int k = 0; k < MB; ++k) {
      const bool in = s0 + lane + 64 * k < ns;
      f[k] = in ? fast_exp2(mlv[k].x - M) : 0.f;
      L += in ? f[k] * mlv[k].y : 0.f;
    }
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      // split g + 4u of the block: its weight sits in lane (g + 4u) % 64, pair u / 16
      const float w = __shfl(f[u / 16], (g + u * kCombGroups) & 63, 64);   // 0 past ns
      A.x += w * pv[u].x; A.y += w * pv[u].y; A.z += w * pv[u].z; A.w += w * pv[u].w;
    }
  }
  L = wave_sum_f32(L);
  static_assert(kCombItems == 16, "split groups are the four lanes l % 16 + 16 j");
  A.x = col_sum4(A.x); A.y = col_sum4(A.y); A.z = col_sum4(A.z); A.w = col_sum4(A.w);
  if (g == 0) {
    const float il = 1.f / L;
    const int hq = hk * o.G + hb * o.hbs + h, d = (slice * kCombItems + item) * 4;
    store_out(o, b, hq, d + 0, A.x * il);
    store_out(o, b, hq, d + 1, A.y * il);
    store_out(o, b, hq, d + 2, A.z * il);
    store_out(o, b, hq, d + 3, A.w * il);
  }
}

template <int D>
static void launch_combine(const SplitKOut& o, const XcdUnits& xm, dim3 grid, hipStream_t stream) {
  // acc loads per lane per block: enough for min(ns, 128) splits over the 4 groups
  const int need = ((o.nsplit < 128 ? o.nsplit : 128) + kCombGroups - 1) / kCombGroups;
  if (need <= 2)
    hipLaunchKernelGGL((splitk_combine_kernel<D, 2>), grid, dim3(64), 0, stream, o, xm);
  else if (need <= 4)
    hipLaunchKernelGGL((splitk_combine_kernel<D, 4>), grid, dim3(64), 0, stream, o, xm);
  else if (need <= 8)
    hipLaunchKernelGGL((splitk_combine_kernel<D, 8>), grid, dim3(64), 0, stream, o, xm);
  else if (need <= 16)
    hipLaunchKernelGGL((splitk_combine_kernel<D, 16>), grid, dim3(64), 0, stream, o, xm);
  else
    hipLaunchKernelGGL((splitk_combine_kernel<D, 32>), grid, dim3(64), 0, stream, o, xm);
}

int splitk_combine(const SplitKOut& o, long units, int D, hipStream_t stream) {
  if (o.nsplit <= 1) return 0;
  if (o.nsplit > kSplitMax) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  // one wave per (unit, query head of the unit's head block, 64-dim slice),
  // eight interleaved per-XCD lists as long as the longest
  const long wu = (long)(o.G < o.hbs ? o.G : o.hbs) * (D / 64);
  const XcdUnits xm = xcd_units(units, o.nsplit);
  long most = 0;
  for (int x = 0; x < kXcds; ++x) most = xm.first[x + 1] - xm.first[x] > most ? xm.first[x + 1] - xm.first[x] : most;
  if (most * wu * kXcds > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)(most * wu * kXcds));
  if (D == 64)
    launch_combine<64>(o, xm, grid, stream);
  else
    launch_combine<128>(o, xm, grid, stream);
  return (int)hipGetLastError();
}

}  // namespace bytes_amd
