// Exact top-k selection over a short row by one wave or by one workgroup
// (used by the top-k kernels and by kernels that select inside their
// prologue).
//
// The row's n <= 64 * PER order keys (score_order_key) sit in the wave's
// registers, lane l holding elements PER*l .. PER*l + PER - 1.  The selection
// is the top k under one total order: key descending, index ascending on
// equal keys.  wave_select_threshold finds the k-th largest key T and how
// many keys equal to T are taken (the lowest-indexed ones): digit passes of
// 11 bits start at the highest bit in which the row's keys differ, histogram
// the keys matching the prefix so far in the wave's LDS (kBins words) and
// pick the digit from a suffix scan over the lanes.  wave_select_compact then
// lists the selected indices in ascending index order.  Wave-level
// synchronisation only: no workgroup barrier.
// block_select_threshold / block_select_compact do the same with the NT
// threads of a workgroup, thread t holding elements PER*t .. +PER: each pass
// picks the digit from wave suffix sums and the wave totals (one barrier), and
// one scan of packed (equal, greater) counts places the selection.
#pragma once
#include "common.h"

namespace bytes_amd {

constexpr int kBins = 2048;            // digit = 11 bits of the order key

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) { return wave_prefix_sum(v); }

// Inclusive suffix sum over the 64 lanes (lane i: sum over lanes >= i).
__device__ __forceinline__ uint32_t wave_suffix_sum(uint32_t v) {
  const uint32_t incl = wave_prefix_sum(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) - incl + v;
}

template <int PER>
__device__ __forceinline__ void wave_select_threshold(const uint32_t (&key)[PER], int n, int k, uint32_t* hist,
                                                      uint32_t& T, uint32_t& need) {
  const int lane = threadIdx.x & 63;
  const int i0 = PER * lane;
  auto valid = [&](int q) { return i0 + q < n; };
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (valid(q)) {
      kmin = min(kmin, key[q]);
      kmax = max(kmax, key[q]);
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, off, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
  }
  const uint32_t diff = kmin ^ kmax;
  const int hb = diff ? 31 - __builtin_clz(diff) : -1;
  uint32_t pmask = hb < 0 ? 0xFFFFFFFFu : ~(uint32_t)((2ull << hb) - 1ull);
  uint32_t prefix = kmin & pmask, kr = (uint32_t)k;
#pragma unroll 1
  for (int hi = hb; hi >= 0; hi -= 11) {
    const int shift = hi >= 10 ? hi - 10 : 0;
    const uint32_t dmask = (1u << (hi - shift + 1)) - 1u;
    u32x4* h4 = reinterpret_cast<u32x4*>(hist) + lane * 8;      // this lane's 32 bins
#pragma unroll
    for (int q = 0; q < 8; ++q) h4[q] = u32x4{0u, 0u, 0u, 0u};
    wave_lds_sync();
#pragma unroll
    for (int q = 0; q < PER; ++q)
      if (valid(q) && (key[q] & pmask) == prefix) atomicAdd(&hist[(key[q] >> shift) & dmask], 1u);
    wave_lds_sync();
    uint32_t c[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const u32x4 v = h4[q];
      c[4 * q] = v[0]; c[4 * q + 1] = v[1]; c[4 * q + 2] = v[2]; c[4 * q + 3] = v[3];
    }
    uint32_t s = 0;
#pragma unroll
    for (int b = 0; b < 32; ++b) s += c[b];
    // inclusive suffix sum over lanes (bins above this lane's range included)
    const uint32_t suf = wave_suffix_sum(s);
    const uint32_t above_lane = suf - s;         // keys in digits above this lane's bins
    // digit d: count(digits > d) < kr <= count(digits >= d)
    const bool mine = above_lane < kr && kr <= suf;
    uint32_t acc = above_lane, d = 0u, above = 0u;
    bool got = false;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
      if (!got && acc + c[b] >= kr) {
        got = true;
        d = 32u * lane + b;
        above = acc;
      }
      acc += c[b];
    }
    const int src = __ffsll((unsigned long long)__ballot(mine)) - 1;
    d = (uint32_t)__builtin_amdgcn_readlane((int)d, src);
    above = (uint32_t)__builtin_amdgcn_readlane((int)above, src);
    kr -= above;
    prefix |= d << shift;
    pmask |= dmask << shift;
    wave_lds_sync();
  }
  T = prefix;
  need = kr;                                     // keys equal to T to take (>= 1)
}

// Selected indices in ascending order: out[slot] for slot < k, through
// emit(slot, index, key).
template <int PER, class EMIT>
__device__ __forceinline__ void wave_select_compact(const uint32_t (&key)[PER], int n, uint32_t T, uint32_t need,
                                                    EMIT emit) {
  const int lane = threadIdx.x & 63;
  const int i0 = PER * lane;
  auto valid = [&](int q) { return i0 + q < n; };
  uint32_t ne = 0u, ng = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    ne += (valid(q) && key[q] == T) ? 1u : 0u;
    ng += (valid(q) && key[q] > T) ? 1u : 0u;
  }
  uint32_t rank = wave_incl_scan(ne, lane) - ne;          // keys equal to T before this lane
  const uint32_t take_eq = rank >= need ? 0u : (need - rank < ne ? need - rank : ne);
  const uint32_t nt = ng + take_eq;
  uint32_t pos = wave_incl_scan(nt, lane) - nt;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const bool v = valid(q);
    bool take = v && key[q] > T;
    if (v && key[q] == T) {
      take = rank < need;
      ++rank;
    }
    if (take) {
      emit(pos, i0 + q, key[q]);
      ++pos;
    }
  }
}

// LDS words block_select_* need beside the kBins histogram.
constexpr int kSelCand = 64;           // crossing-bin keys ranked directly by one wave
template <int NT>
constexpr int block_select_words() { return 4 * (NT / 64) + 4 + kSelCand; }

template <int NT, int PER>
__device__ void block_select_threshold(const uint32_t (&key)[PER], int n, int k, uint32_t* hist, uint32_t* red,
                                       uint32_t& T, uint32_t& need) {
  constexpr int NW = NT / 64;
  constexpr int BPT = kBins / NT;                // histogram bins per thread
  static_assert(BPT % 4 == 0, "bins per thread");
  uint32_t* wa = red;
  uint32_t* wb = red + NW;
  uint32_t* wc = red + 2 * NW;
  uint32_t* sel = red + 4 * NW;                  // [4]: digit, count above, candidate count, result
  uint32_t* cand = red + 4 * NW + 4;             // [kSelCand]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i0 = PER * tid;
  auto valid = [&](int q) { return i0 + q < n; };
  // key range of the row
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (valid(q)) {
      kmin = min(kmin, key[q]);
      kmax = max(kmax, key[q]);
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, off, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
  }
  if (lane == 0) {
    wa[w] = kmin;
    wb[w] = kmax;
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    kmin = min(kmin, wa[v]);
    kmax = max(kmax, wb[v]);
  }
  const uint32_t diff = kmin ^ kmax;
  const int hb = diff ? 31 - __builtin_clz(diff) : -1;        // highest differing bit
  uint32_t pmask = hb < 0 ? 0xFFFFFFFFu : ~(uint32_t)((2ull << hb) - 1ull);
  uint32_t prefix = kmin & pmask, kr = (uint32_t)k;
  u32x4* h4 = reinterpret_cast<u32x4*>(hist) + tid * (BPT / 4);   // this thread's bins
#pragma unroll 1
  for (int hi = hb; hi >= 0; hi -= 11) {
    const int lo = hi >= 10 ? hi - 10 : 0;
    const uint32_t dmask = (1u << (hi - lo + 1)) - 1u;
#pragma unroll
    for (int q = 0; q < BPT / 4; ++q) h4[q] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PER; ++q)
      if (valid(q) && (key[q] & pmask) == prefix) atomicAdd(&hist[(key[q] >> lo) & dmask], 1u);
    __syncthreads();
    uint32_t c[BPT];
#pragma unroll
    for (int q = 0; q < BPT / 4; ++q) {
      const u32x4 v = h4[q];
      c[4 * q] = v[0]; c[4 * q + 1] = v[1]; c[4 * q + 2] = v[2]; c[4 * q + 3] = v[3];
    }
    uint32_t s = 0u;
#pragma unroll
    for (int b = 0; b < BPT; ++b) s += c[b];
    // inclusive suffix sum over the wave's lanes, then the waves above
    const uint32_t suf = wave_suffix_sum(s);
    if (lane == 0) wc[w] = suf;
    __syncthreads();
    uint32_t acc = suf - s;                      // keys in the bins above this thread's
#pragma unroll
    for (int v = 0; v < NW; ++v) acc += v > w ? wc[v] : 0u;
    // digit d: count(digits > d) < kr <= count(digits >= d); exactly one
    // thread and bin see the crossing
#pragma unroll
    for (int b = BPT - 1; b >= 0; --b) {
      if (acc < kr && acc + c[b] >= kr) {
        sel[0] = (uint32_t)(BPT * tid + b);
        sel[1] = acc;
        sel[2] = c[b];
      }
      acc += c[b];
    }
    if (tid == 0) sel[3] = 0u;                   // candidate slots taken (the picked bin is not this thread's)
    __syncthreads();
    kr -= sel[1];
    prefix |= sel[0] << lo;
    pmask |= dmask << lo;
    const uint32_t nc = sel[2];
    if (lo > 0 && nc <= (uint32_t)kSelCand) {
      // few keys in the crossing bin: list them, then one wave finds the kr-th
      // largest by counting, for each candidate, the candidates above it
#pragma unroll
      for (int q = 0; q < PER; ++q)
        if (valid(q) && (key[q] & pmask) == prefix) cand[atomicAdd(&sel[3], 1u)] = key[q];
      __syncthreads();
      if (w == 0) {
        const uint32_t mine = lane < (int)nc ? cand[lane] : 0u;
        uint32_t gt = 0u, ge = 0u;
        for (uint32_t j = 0; j < nc; ++j) {
          const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)mine, (int)j);
          gt += o > mine ? 1u : 0u;
          ge += o >= mine ? 1u : 0u;
        }
        if (lane < (int)nc && gt < kr && kr <= ge) {   // lanes holding the threshold agree
          sel[0] = mine;
          sel[1] = kr - gt;
        }
      }
      __syncthreads();
      T = sel[0];
      need = sel[1];
      __syncthreads();                           // sel is reused by the caller's next select
      return;
    }
  }
  T = prefix;
  need = kr;                                     // keys equal to T to take (>= 1), lowest indices first
}

// Selected indices in ascending order, through emit(slot, index, key).
template <int NT, int PER, class EMIT>
__device__ void block_select_compact(const uint32_t (&key)[PER], int n, uint32_t T, uint32_t need, uint32_t* red,
                                     EMIT emit) {
  constexpr int NW = NT / 64;
  uint32_t* wd = red + 3 * NW;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i0 = PER * tid;
  auto valid = [&](int q) { return i0 + q < n; };
  // one scan of (equal << 16 | greater), both < 2^16
  uint32_t ne = 0u, ng = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    ne += (valid(q) && key[q] == T) ? 1u : 0u;
    ng += (valid(q) && key[q] > T) ? 1u : 0u;
  }
  const uint32_t packed = (ne << 16) | ng;
  const uint32_t incl = wave_incl_scan(packed, lane);
  if (lane == 63) wd[w] = incl;
  __syncthreads();
  uint32_t before = incl - packed;
#pragma unroll
  for (int v = 0; v < NW; ++v) before += v < w ? wd[v] : 0u;
  uint32_t rank = before >> 16;                  // keys equal to T before this thread
  uint32_t pos = (before & 0xFFFFu) + (rank < need ? rank : need);
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const bool v = valid(q);
    bool take = v && key[q] > T;
    if (v && key[q] == T) {
      take = rank < need;
      ++rank;
    }
    if (take) {
      emit(pos, i0 + q, key[q]);
      ++pos;
    }
  }
}

}  // namespace bytes_amd
