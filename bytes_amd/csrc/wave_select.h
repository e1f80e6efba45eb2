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
// block_select / block_select_emit do the same with the NT threads of a
// workgroup, thread t holding elements PER*t .. +PER (described below).
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

// ---- workgroup selection ----
// Digit passes of 8 bits, starting at the highest bit in which the row's keys
// differ.  Each pass has a histogram of its own (all zeroed up front, so a
// pass needs no clearing barrier); every thread adds each of its keys with an
// unconditional LDS add: a key outside the current prefix, or past n, lands in
// a spare word of its own lane past the bins (no branches, no same-address
// conflicts).  After the pass's one barrier every wave scans the 256 bins
// itself (four per lane, a suffix sum over the lanes), so the digit is known
// to every wave without a second barrier.  The passes stop as soon as the
// crossing bin is taken whole.
constexpr int kSelBins = 256;
constexpr int kSelStride = kSelBins + 64;      // bins + one spare word per lane
constexpr int kSelPasses = 4;                  // 32 bits in digits of 8

// LDS words the workgroup selection needs.
template <int NT>
constexpr int block_select_words() { return kSelStride * kSelPasses + 3 * (NT / 64); }

// The selection's predicate: keys with (key & M) > P are taken; of those with
// (key & M) == P, the `need` lowest-indexed (all of them when `all`).
struct BlockSel {
  uint32_t P, M, need, all;
};

// Wave minimum and maximum, every lane receiving both: rotations within the
// rows of 16 (every source lane in the row), then the row and half swaps.
__device__ __forceinline__ void wave_minmax_u32(uint32_t& mn, uint32_t& mx) {
#define BYTES_ROT(CTRL)                                                                        \
  mn = min(mn, (uint32_t)__builtin_amdgcn_update_dpp((int)mn, (int)mn, CTRL, 0xF, 0xF, false)); \
  mx = max(mx, (uint32_t)__builtin_amdgcn_update_dpp((int)mx, (int)mx, CTRL, 0xF, 0xF, false));
  BYTES_ROT(0x128)   // row_ror:8
  BYTES_ROT(0x124)   // row_ror:4
  BYTES_ROT(0x122)   // row_ror:2
  BYTES_ROT(0x121)   // row_ror:1
#undef BYTES_ROT
  const auto a = __builtin_amdgcn_permlane16_swap(mn, mn, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(mx, mx, false, false);
  mn = min((uint32_t)a[0], (uint32_t)a[1]);
  mx = max((uint32_t)b[0], (uint32_t)b[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(mn, mn, false, false);
  const auto d = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);
  mn = min((uint32_t)c[0], (uint32_t)c[1]);
  mx = max((uint32_t)d[0], (uint32_t)d[1]);
}

// Top k (1 <= k <= n <= NT*PER) of the workgroup's keys, thread t holding
// elements PER*t .. +PER; ws: block_select_words<NT>() LDS words, free for
// the call.  Every thread of the workgroup calls it.
template <int NT, int PER>
__device__ BlockSel block_select(const uint32_t (&key)[PER], int n, int k, uint32_t* ws) {
  constexpr int NW = NT / 64;
  uint32_t* hist = ws;
  uint32_t* wr = ws + kSelStride * kSelPasses;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i0 = PER * tid;
  for (int i = tid; i < kSelStride * kSelPasses / 4; i += NT)
    reinterpret_cast<u32x4*>(hist)[i] = u32x4{0u, 0u, 0u, 0u};
  // key range of the row (the bits above its highest differing bit are common)
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const bool v = i0 + q < n;
    kmin = min(kmin, v ? key[q] : 0xFFFFFFFFu);
    kmax = max(kmax, v ? key[q] : 0u);
  }
  wave_minmax_u32(kmin, kmax);
  if (lane == 0) {
    wr[w] = kmin;
    wr[NW + w] = kmax;
  }
  __syncthreads();                             // also orders the histogram clearing
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    kmin = min(kmin, wr[v]);
    kmax = max(kmax, wr[NW + v]);
  }
  kmin = (uint32_t)__builtin_amdgcn_readfirstlane((int)kmin);
  kmax = (uint32_t)__builtin_amdgcn_readfirstlane((int)kmax);
  const uint32_t diff = kmin ^ kmax;
  const int hb = diff ? 31 - __builtin_clz(diff) : -1;
  uint32_t pmask = hb < 0 ? 0xFFFFFFFFu : ~(uint32_t)((2ull << hb) - 1ull);
  uint32_t prefix = kmin & pmask, kr = (uint32_t)k, all = 0u;
  int pass = 0;
#pragma unroll 1
  for (int hi = hb; hi >= 0; hi -= 8, ++pass) {
    const int lo = hi >= 7 ? hi - 7 : 0;
    const uint32_t nb = 1u << (hi - lo + 1);   // bins of this pass (<= 256)
    const uint32_t base = prefix >> lo;        // keys in the prefix: (key >> lo) - base is the digit
    uint32_t* H = hist + pass * kSelStride;
    const uint32_t spare = nb + (uint32_t)lane;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      uint32_t t = (key[q] >> lo) - base;      // wraps past the bins for keys below the prefix
      t = i0 + q < n ? t : 0xFFFFFFFFu;
      atomicAdd(&H[min(t, spare)], 1u);        // outside the prefix: words nb .. nb+63, never scanned
    }
    lds_barrier();
    const u32x4 c = reinterpret_cast<const u32x4*>(H)[lane];   // bins 4*lane .. +3
    const uint32_t b0 = 4u * lane;
    const uint32_t c0 = b0 < nb ? c[0] : 0u, c1 = b0 + 1 < nb ? c[1] : 0u;
    const uint32_t c2 = b0 + 2 < nb ? c[2] : 0u, c3 = b0 + 3 < nb ? c[3] : 0u;
    const uint32_t s = c0 + c1 + c2 + c3;
    const uint32_t suf = wave_suffix_sum(s);   // keys in bins >= 4*lane
    const uint32_t a3 = suf - s, a2 = a3 + c3, a1 = a2 + c2, a0 = a1 + c1;   // keys above bin 4*lane+e
    // digit d: count(digits > d) < kr <= count(digits >= d); one lane holds it
    const int src = __ffsll((unsigned long long)__ballot(a3 < kr && kr <= suf)) - 1;
    const bool g3 = a2 >= kr, g2 = a1 >= kr, g1 = a0 >= kr;
    const uint32_t e = g3 ? 3u : g2 ? 2u : g1 ? 1u : 0u;
    const uint32_t ab = g3 ? a3 : g2 ? a2 : g1 ? a1 : a0;
    const uint32_t cn = g3 ? c3 : g2 ? c2 : g1 ? c1 : c0;
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)(b0 + e), src);
    kr -= (uint32_t)__builtin_amdgcn_readlane((int)ab, src);
    const uint32_t cnt = (uint32_t)__builtin_amdgcn_readlane((int)cn, src);
    prefix |= d << lo;
    pmask |= (nb - 1u) << lo;
    if (cnt == kr) {                           // the crossing bin is taken whole
      all = 1u;
      break;
    }
  }
  return BlockSel{prefix, pmask, kr, all};
}

// The selection in ascending index order, through emit(slot, index, key);
// one barrier (its words are past the histograms, so it may follow
// block_select directly).
template <int NT, int PER, class EMIT>
__device__ void block_select_emit(const uint32_t (&key)[PER], int n, const BlockSel& s, uint32_t* ws, EMIT emit) {
  constexpr int NW = NT / 64;
  uint32_t* wd = ws + kSelStride * kSelPasses + 2 * NW;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i0 = PER * tid;
  if (s.all) {
    bool take[PER];
    uint32_t cnt = 0u;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      take[q] = i0 + q < n && (key[q] & s.M) >= s.P;
      cnt += take[q] ? 1u : 0u;
    }
    const uint32_t incl = wave_prefix_sum(cnt);
    if (lane == 63) wd[w] = incl;
    lds_barrier();
    uint32_t pos = incl - cnt;
#pragma unroll
    for (int v = 0; v < NW; ++v) pos += v < w ? wd[v] : 0u;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      if (take[q]) emit(pos, i0 + q, key[q]);
      pos += take[q] ? 1u : 0u;
    }
    return;
  }
  // ties at the threshold: the lowest-indexed `need` of them; one scan of
  // packed (equal << 16 | greater) counts, both < 2^16
  uint32_t ne = 0u, ng = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const bool v = i0 + q < n;
    const uint32_t m = key[q] & s.M;
    ne += (v && m == s.P) ? 1u : 0u;
    ng += (v && m > s.P) ? 1u : 0u;
  }
  const uint32_t packed = (ne << 16) | ng;
  const uint32_t incl = wave_prefix_sum(packed);
  if (lane == 63) wd[w] = incl;
  lds_barrier();
  uint32_t before = incl - packed;
#pragma unroll
  for (int v = 0; v < NW; ++v) before += v < w ? wd[v] : 0u;
  uint32_t rank = before >> 16;                  // keys equal to P before this thread
  uint32_t pos = (before & 0xFFFFu) + (rank < s.need ? rank : s.need);
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const bool v = i0 + q < n;
    const uint32_t m = key[q] & s.M;
    bool take = v && m > s.P;
    if (v && m == s.P) {
      take = rank < s.need;
      ++rank;
    }
    if (take) {
      emit(pos, i0 + q, key[q]);
      ++pos;
    }
  }
}

}  // namespace bytes_amd
