// Deterministic top-k over rows of fp32 scores.
//
// Replaces `scores.topk(kb, dim=-1).indices` on the sparse decode paths
// (src/attention_kernels.py:1262, benchmarks/sparse_attention.py:307 and
// :358), whose tie order is unspecified, with one total order: score
// descending, index ascending on equal scores (+0 and -0 are equal; NaN ranks
// above +inf, as in torch.topk).  Output: int32 indices [rows, k] ordered by
// that order, identical run to run.
//
// Three launches:
//  1. histogram: many workgroups per row count the top 11 bits (digit) of the
//     32-bit order keys into a per-row 2048-bin histogram (LDS, then one
//     global atomic per non-empty bin);
//  2. filter: many workgroups per row find the digit d0 holding the k-th
//     largest key and copy every key with a larger digit to the row's
//     "above" list and every key with digit d0 to its candidate list (list
//     order is irrelevant: step 3 sorts);
//  3. select: one workgroup per row sorts the above list plus the candidates
//     by (key desc, index asc) with a bitonic sort in LDS and writes the first
//     k indices.  If the candidates overflow their list (heavily tied rows),
//     the workgroup instead runs an exact radix select over the whole row
//     (11/11/10-bit digits), collects in index order and sorts the k results.
// Step 3 also clears the histogram and list counters, which are zero between
// calls.  Short rows, and selections larger than the lists hold (k > 8192),
// run step 3's exact path alone; for k > 8192 it lists the selection by
// ascending index, and a sorted output then takes two more launches: blocks
// of 8192 selected entries sorted in LDS, then each entry's final slot from
// its rank in its own block plus binary searches in the others.
#include "wave_select.h"

namespace bytes_amd {

constexpr int kTopkThreads = 1024;     // select kernel
constexpr int kPassThreads = 512;      // histogram and filter kernels (four 16-byte loads per thread)
constexpr int kSlice = 8192;           // row elements per histogram / filter workgroup
constexpr int kTopkMaxK = 8192;
constexpr int kCandCap = 8192;         // candidate list capacity per row
constexpr int kSortMax = 16384;        // LDS sort capacity (above list + candidates)
constexpr int kShortRow = 16384;       // rows up to this length take the single-kernel exact path
constexpr int kFullSortRow = 4096;     // ... and up to this length simply sort the whole row
constexpr int kEqMax = 512;            // keys equal to the threshold handled by the bitmap path

__device__ __forceinline__ uint32_t order_key(float x) { return score_order_key(x); }

// Sort value: descending order of (key, ~index) = key desc, index asc.
__device__ __forceinline__ uint64_t sort_val(uint32_t key, int idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// Inclusive prefix sum over the NT threads of the workgroup (thread order).
template <int NT>
__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // the wave's scan on DPP (every lane active), then each thread adds the
  // totals of the waves before its own
  const uint32_t x = wave_prefix_sum(v);
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  uint32_t before = 0u, tot = 0u;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const uint32_t t = wsum[u];
    before += u < w ? t : 0u;
    tot += t;
  }
  total = tot;
  __syncthreads();   // wsum is reused by the next scan
  return x + before;
}

// Buffer resource over the n floats of a row: reads past the row return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* x, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), (short)0, (int)((uint32_t)n * 4u), 0x00020000);
}

// Order keys of elements i .. i+3 of a row and whether each exists.  Loads go
// through the row's buffer resource, unconditionally (past the row they read
// zero), so no load sits under a branch and a thread's loads are all in flight
// together.  VEC: one 16-byte load (the host sets it only for 16-byte-aligned
// rows with n % 4 == 0, so a vector is never partly past the row).
template <bool VEC>
__device__ __forceinline__ void load4(__amdgpu_buffer_rsrc_t rs, int i, int n, uint32_t (&key)[4], bool (&ok)[4]) {
  if constexpr (VEC) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, i * 4, 0, 0));
#pragma unroll
    for (int j = 0; j < 4; ++j) key[j] = order_key(__uint_as_float(v[j]));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) key[j] = order_key(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (i + j) * 4, 0, 0)));
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) ok[j] = i + j < n;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Bitonic merge steps with strides 32 .. 1 on the 64-element segments of buf,
// one segment per wave at a time, in registers (xor shuffles); for the merge
// of blocks of `size`, whose direction is descending where (index & size) == 0.
// size <= 64 runs the whole network up to that size.
template <int NT>
__device__ __forceinline__ void bitonic_wave_steps(uint64_t* buf, int P, int size_lo, int size_hi) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int seg = w; seg < P / 64; seg += NW) {
    const int i = seg * 64 + lane;
    uint64_t x = buf[i];
    for (int size = size_lo; size <= size_hi; size <<= 1) {
      const bool desc = (i & size) == 0;
      for (int stride = (size < 64 ? size : 64) >> 1; stride > 0; stride >>= 1) {
        const uint64_t y = shfl_xor_u64(x, stride);
        const bool keep_max = ((lane & stride) == 0) == desc;
        x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
      }
    }
    buf[i] = x;
  }
}

// In-LDS bitonic sort of buf[0, P) into descending order (P a power of two,
// P >= 64).  Strides below 64 run inside a wave on xor shuffles; only strides
// >= 64 go through LDS with a workgroup barrier.
template <int NT>
__device__ void bitonic_desc(uint64_t* buf, int P) {
  bitonic_wave_steps<NT>(buf, P, 2, 64);
  __syncthreads();
  for (int size = 128; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride >= 64; stride >>= 1) {
      for (int i = threadIdx.x; i < P / 2; i += NT) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t va = buf[lo], vb = buf[hi];
        if ((va < vb) == desc) {
          buf[lo] = vb;
          buf[hi] = va;
        }
      }
      __syncthreads();
    }
    bitonic_wave_steps<NT>(buf, P, size, size);
    __syncthreads();
  }
}

constexpr int kRowBatch = 1024;        // rows per launch group (fixed histogram region, 8 MiB)

// Workspace: a fixed-size region of per-row histograms and list counters for
// kRowBatch rows, zero between calls (the select kernel clears what it used),
// then the lists, whose size depends on (rows, k).  Because the zero region
// never moves, list data of an earlier call can never land in it.
struct TopkWs {
  uint32_t* hist;    // [kRowBatch][kBins]
  uint32_t* cnt;     // [kRowBatch][kCntStride]: above-list length, candidate count
  uint64_t* above;   // [kRowBatch][k]
  uint64_t* cand;    // [kRowBatch][kCandCap]; k > kTopkMaxK: [kRowBatch][kLargeCand]
  uint32_t* sabove;  // k > kTopkMaxK: [kRowBatch][parts] keys above the threshold digit per slice
  uint32_t* soff;    // k > kTopkMaxK: [kRowBatch][parts] output offset of each slice
  uint32_t* par;     // k > kTopkMaxK: [kRowBatch][kLargePar] the row's selection predicate
  uint64_t* sorted;  // k > kTopkMaxK: [rows][kpad] sort values of the selection, sorted per 8192-entry block
};

// A row's two list counters have a 128-byte line of their own: the filter
// workgroups of a row (on every XCD) add to them with device-wide atomics,
// which serialise per cache line.
constexpr int kCntStride = 32;
constexpr size_t kTopkZeroBytes = (size_t)kRowBatch * kBins * 4 + (size_t)kRowBatch * kCntStride * 4;

// k above kTopkMaxK on long rows: the keys of the threshold digit (up to
// kLargeCand per row) are listed and selected among by one workgroup per row,
// which leaves the row's selection predicate and each slice's output offset;
// every slice then writes its selected indices in index order.
constexpr int kLargeCand = 16384;   // 16 per thread of the select workgroup (more spills registers)
constexpr int kLargeMaxParts = 2048;   // slices per row (rows up to 16 Mi elements)
constexpr int kLargePar = 8;

// Lists for the rows of one launch group (min(rows, kRowBatch)) follow the
// fixed zero region.  k above kTopkMaxK: the candidate lists, slice counts
// and predicates of the launch group, then (sorted output) rows * kpad 8-byte
// sort values, kpad = k rounded up to whole 8192-entry sort blocks.
constexpr int kSortBlock = 8192;
__host__ __device__ inline size_t topk_large_pad(int k) { return ((size_t)k + kSortBlock - 1) / kSortBlock * kSortBlock; }

inline int topk_parts(int n) { return (n + kSlice - 1) / kSlice; }

inline size_t topk_large_list_bytes(size_t r, int n) {
  return r * ((size_t)kLargeCand * 8 + (size_t)topk_parts(n) * 8 + kLargePar * 4);
}

inline size_t topk_ws_bytes(int64_t rows, int n, int k) {
  const size_t r = (size_t)(rows < kRowBatch ? (rows > 0 ? rows : 1) : kRowBatch);
  if (k > kTopkMaxK)
    return kTopkZeroBytes + topk_large_list_bytes(r, n) + (size_t)(rows > 0 ? rows : 1) * topk_large_pad(k) * 8;
  return kTopkZeroBytes + r * k * 8 + r * kCandCap * 8;
}

inline TopkWs topk_ws_carve(void* ws, int64_t rows, int n, int k) {
  char* p = static_cast<char*>(ws);
  TopkWs t;
  t.hist = reinterpret_cast<uint32_t*>(p);
  t.cnt = reinterpret_cast<uint32_t*>(p + (size_t)kRowBatch * kBins * 4);
  const size_t r = (size_t)(rows < kRowBatch ? (rows > 0 ? rows : 1) : kRowBatch);
  char* l = p + kTopkZeroBytes;
  if (k > kTopkMaxK) {
    const int parts = topk_parts(n);
    t.above = nullptr;
    t.cand = reinterpret_cast<uint64_t*>(l);
    t.sabove = reinterpret_cast<uint32_t*>(l + r * kLargeCand * 8);
    t.soff = t.sabove + r * parts;
    t.par = t.soff + r * parts;
    t.sorted = reinterpret_cast<uint64_t*>(l + topk_large_list_bytes(r, n));
  } else {
    t.above = reinterpret_cast<uint64_t*>(l);
    t.cand = reinterpret_cast<uint64_t*>(l + r * k * 8);
    t.sabove = t.soff = t.par = nullptr;
    t.sorted = nullptr;
  }
  return t;
}

// ---- 1. per-row digit histogram ----
template <bool VEC>
__global__ __launch_bounds__(kPassThreads) void topk_hist_kernel(const float* scores, int64_t row_stride, int n,
                                                                 int parts, uint32_t* hist) {
  __shared__ uint32_t h[kBins];
  // scores points at the batch's first row; row indexes the batch's workspace rows
  const int row = blockIdx.x / parts, part = blockIdx.x - (blockIdx.x / parts) * parts;
  const float* x = scores + (int64_t)row * row_stride;
  const auto rs = row_rsrc(x, n);
  constexpr int R = kSlice / (kPassThreads * 4);
  uint32_t key[R][4];
  bool ok[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = part * kSlice + (r * kPassThreads + threadIdx.x) * 4;
    load4<VEC>(rs, i, n, key[r], ok[r]);
  }
  for (int b = threadIdx.x; b < kBins; b += kPassThreads) h[b] = 0u;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ok[r][j]) atomicAdd(&h[key[r][j] >> 21], 1u);
  __syncthreads();
  uint32_t* hr = hist + (int64_t)row * kBins;
  for (int b = threadIdx.x; b < kBins; b += kPassThreads)
    if (h[b]) atomicAdd(hr + b, h[b]);
}

// The digit holding the k-th largest key of a row and the count of keys in
// larger digits, from its histogram (thread t owns digits PER*t .. PER*t+PER-1, PER = kBins / NT).
template <int NT>
__device__ __forceinline__ void find_digit(const uint32_t* hr, uint32_t k, uint32_t* wsum, uint32_t* sel) {
  constexpr int PER = kBins / NT;
  if (threadIdx.x == 0) sel[0] = 0xFFFFFFFFu;
  uint32_t hb[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    hb[j] = hr[threadIdx.x * PER + j];
    sum += hb[j];
  }
  uint32_t total;
  const uint32_t incl = block_incl_scan<NT>(sum, wsum, total);
  uint32_t above = total - incl;              // keys in digits > PER*t + PER-1
#pragma unroll
  for (int j = PER - 1; j >= 0; --j) {
    if (above < k && above + hb[j] >= k) {
      sel[0] = threadIdx.x * PER + j;
      sel[1] = above;
    }
    above += hb[j];
  }
  __syncthreads();
}

// ---- 2. filter into the above list and the candidate list ----
template <bool VEC>
__global__ __launch_bounds__(kPassThreads) void topk_filter_kernel(const float* scores, int64_t row_stride, int n,
                                                                   int k, int parts, TopkWs ws) {
  __shared__ uint32_t wsum[kPassThreads / 64];
  __shared__ uint32_t sel[4];
  const int row = blockIdx.x / parts, part = blockIdx.x - (blockIdx.x / parts) * parts;
  const float* x = scores + (int64_t)row * row_stride;
  const auto rs = row_rsrc(x, n);
  constexpr int R = kSlice / (kPassThreads * 4);
  uint32_t key[R][4];
  bool ok[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = part * kSlice + (r * kPassThreads + threadIdx.x) * 4;
    load4<VEC>(rs, i, n, key[r], ok[r]);
  }
  find_digit<kPassThreads>(ws.hist + (int64_t)row * kBins, (uint32_t)k, wsum, sel);
  const uint32_t d0 = sel[0];                   // digits are < kBins: a missing pick keeps every key out
  uint32_t na = 0, nc = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[r][j]) continue;
      const uint32_t d = key[r][j] >> 21;
      na += d > d0 ? 1u : 0u;
      nc += d == d0 ? 1u : 0u;
    }
  // one scan of (candidates << 16 | above): both stay below 2^16 per workgroup
  static_assert(kSlice < 65536, "packed counts");
  uint32_t tp;
  const uint32_t op = block_incl_scan<kPassThreads>((nc << 16) | na, wsum, tp) - ((nc << 16) | na);
  uint32_t oa = op & 0xFFFFu, oc = op >> 16;
  const uint32_t ta = tp & 0xFFFFu, tc = tp >> 16;
  if (threadIdx.x == 0) {
    sel[2] = ta ? atomicAdd(ws.cnt + row * kCntStride + 0, ta) : 0u;
    sel[3] = tc ? atomicAdd(ws.cnt + row * kCntStride + 1, tc) : 0u;
  }
  __syncthreads();
  oa += sel[2];
  oc += sel[3];
  uint64_t* al = ws.above + (int64_t)row * k;
  uint64_t* cl = ws.cand + (int64_t)row * kCandCap;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[r][j]) continue;
      const uint32_t d = key[r][j] >> 21;
      const int idx = part * kSlice + (r * kPassThreads + threadIdx.x) * 4 + j;
      if (d > d0) {
        if (oa < (uint32_t)k) al[oa] = sort_val(key[r][j], idx);
        ++oa;
      } else if (d == d0) {
        if (oc < (uint32_t)kCandCap) cl[oc] = sort_val(key[r][j], idx);
        ++oc;
      }
    }
}

// Over an LDS histogram of 2048 digits (1024 threads, two digits each): the
// digit holding the kr-th largest key and the count of keys in larger digits,
// left in sel[0], sel[1].
__device__ __forceinline__ void pick_digit(const uint32_t* hist, uint32_t kr, uint32_t* wsum, uint32_t* sel) {
  const int tid = threadIdx.x;
  const uint32_t c0 = hist[2 * tid], c1 = hist[2 * tid + 1];
  uint32_t total;
  const uint32_t incl = block_incl_scan<kTopkThreads>(c0 + c1, wsum, total);
  const uint32_t above = total - incl;
  if (above < kr && above + c1 >= kr) {
    sel[0] = 2 * tid + 1;
    sel[1] = above;
  } else if (above + c1 < kr && above + c1 + c0 >= kr) {
    sel[0] = 2 * tid;
    sel[1] = above + c1;
  }
  __syncthreads();
}

// Exact selection over a whole row in one workgroup (used when the candidate
// list overflowed): radix select, then either collection and sort by score or
// (unsorted) collection straight into index order.
template <bool VEC>
__device__ void topk_row_exact(const float* x, int n, int k, int sorted, uint64_t* sortbuf, uint32_t* hist,
                               uint32_t* wsum, uint32_t* sel, int32_t* o) {
  const int tid = threadIdx.x;
  const auto rs = row_rsrc(x, n);
  uint32_t prefix = 0u, pmask = 0u;
  uint32_t kr = (uint32_t)k;
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 0x3FFu : 0x7FFu;
    for (int b = tid; b < kBins; b += kTopkThreads) hist[b] = 0u;
    __syncthreads();
    for (int i = tid * 4; i < n; i += kTopkThreads * 4) {
      uint32_t key[4];
      bool ok[4];
      load4<VEC>(rs, i, n, key, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (ok[j] && (key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & dmask], 1u);
    }
    __syncthreads();
    // digit d with count(digits > d) < kr <= count(digits >= d); shift-relative digits
    pick_digit(hist, kr, wsum, sel);
    kr -= sel[1];
    prefix |= sel[0] << shift;
    pmask |= dmask << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;
  const uint32_t need = kr;                      // keys equal to T to take, >= 1
  if (!sorted) {
    // collection in index order: output slot = selected keys before this one
    if (tid == 0) sel[3] = 0u;                   // keys equal to T taken so far
    if (tid == 0) sel[2] = 0u;                   // output slots used so far
    __syncthreads();
    for (int base = 0; base < n; base += kTopkThreads * 4) {
      const int i = base + tid * 4;
      uint32_t key[4];
      bool ok[4];
      load4<VEC>(rs, i, n, key, ok);
      uint32_t ne = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) ne += (ok[j] && key[j] == T) ? 1u : 0u;
      uint32_t tot_eq;
      uint32_t rank = block_incl_scan<kTopkThreads>(ne, wsum, tot_eq) - ne;
      const uint32_t eq0 = sel[3];
      bool take[4];
      uint32_t nt = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        take[j] = ok[j] && key[j] > T;
        if (ok[j] && key[j] == T) {
          take[j] = eq0 + rank < need;
          ++rank;
        }
        nt += take[j] ? 1u : 0u;
      }
      uint32_t tot_t;
      uint32_t pos = sel[2] + block_incl_scan<kTopkThreads>(nt, wsum, tot_t) - nt;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (take[j]) o[pos++] = i + j;
      __syncthreads();
      if (tid == 0) {
        sel[3] = eq0 + tot_eq;
        sel[2] += tot_t;
      }
      __syncthreads();
    }
    return;
  }
  int P = 64;
  while (P < k) P <<= 1;
  for (int i = tid; i < P; i += kTopkThreads) sortbuf[i] = 0ull;
  if (tid == 0) {
    sel[2] = 0u;
    sel[3] = 0u;
  }
  __syncthreads();
  for (int base = 0; base < n; base += kTopkThreads * 4) {
    const int i = base + tid * 4;
    uint32_t key[4];
    bool ok[4];
    load4<VEC>(rs, i, n, key, ok);
    uint32_t ne = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) ne += (ok[j] && key[j] == T) ? 1u : 0u;
    uint32_t rank = 0, tot = 0;
    if (__syncthreads_or(ne != 0)) rank = block_incl_scan<kTopkThreads>(ne, wsum, tot) - ne;
    const uint32_t eq0 = sel[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[j]) continue;
      bool take = key[j] > T;
      if (key[j] == T) {
        take = eq0 + rank < need;
        ++rank;
      }
      if (take) sortbuf[atomicAdd(&sel[2], 1u)] = sort_val(key[j], i + j);
    }
    __syncthreads();
    if (tid == 0) sel[3] = eq0 + tot;
    __syncthreads();
  }
  bitonic_desc<kTopkThreads>(sortbuf, P);
  for (int i = tid; i < k; i += kTopkThreads) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sortbuf[i]);
}

// ---- 3. per-row selection and sort ----
// sorted: output ordered by (score desc, index asc); else by index ascending.
template <bool VEC>
__global__ __launch_bounds__(kTopkThreads) void topk_select_kernel(const float* scores, int64_t row_stride, int n,
                                                                   int k, TopkWs ws, int32_t* out,
                                                                   int64_t out_stride, int exact, int sorted,
                                                                   int hist_ready) {
  extern __shared__ uint64_t sortbuf[];          // [kSortMax]
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wsum[kTopkThreads / 64];
  __shared__ uint32_t sel[8];
  const int row = blockIdx.x, tid = threadIdx.x;
  int32_t* o = out + (int64_t)row * out_stride;
  const float* x = scores + (int64_t)row * row_stride;
  const auto rs = row_rsrc(x, n);
  if (exact) {                                   // short rows: one pass of this kernel only
    if (sorted && n <= kFullSortRow) {
      // sort the whole row by (key desc, index asc)
      int P = 64;
      while (P < n) P <<= 1;
      for (int i = tid; i < P; i += kTopkThreads) sortbuf[i] = i < n ? sort_val(order_key(x[i]), i) : 0ull;
      __syncthreads();
      bitonic_desc<kTopkThreads>(sortbuf, P);
      for (int i = tid; i < k; i += kTopkThreads) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sortbuf[i]);
    } else {
      topk_row_exact<VEC>(x, n, k, sorted, sortbuf, hist, wsum, sel, o);
    }
    if (hist_ready) {                            // a histogram the caller built: leave it at zero
      uint32_t* hr = ws.hist + (int64_t)row * kBins;
      for (int b = tid; b < kBins; b += kTopkThreads) hr[b] = 0u;
    }
    return;
  }
  const uint32_t A = ws.cnt[row * kCntStride + 0], Cn = ws.cnt[row * kCntStride + 1];
  bool fallback = true;
  // lists are complete and consistent: fewer than k keys above the digit, the
  // candidates fill the rest and fit their list
  if (A < (uint32_t)k && A + Cn >= (uint32_t)k && Cn <= (uint32_t)kCandCap) {
    fallback = false;
    const uint64_t* al = ws.above + (int64_t)row * k;
    const uint64_t* cl = ws.cand + (int64_t)row * kCandCap;
    // refine among the candidates (which share the top 11 key bits) on bits
    // 20..10: keep the ones in larger digits and all of the threshold digit
    constexpr int PC = kCandCap / kTopkThreads;
    uint64_t cv[PC];
#pragma unroll
    for (int j = 0; j < PC; ++j) {
      const int i = tid + j * kTopkThreads;
      cv[j] = i < (int)Cn ? cl[i] : 0ull;
    }
    auto live = [&](int j) { return tid + j * kTopkThreads < (int)Cn; };
    auto dg1 = [&](int j) { return (uint32_t)(cv[j] >> 42) & 0x7FFu; };     // key bits 20..10
    auto dg2 = [&](int j) { return (uint32_t)(cv[j] >> 32) & 0x3FFu; };     // key bits 9..0
    for (int b = tid; b < kBins; b += kTopkThreads) hist[b] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PC; ++j)
      if (live(j)) atomicAdd(&hist[dg1(j)], 1u);
    __syncthreads();
    pick_digit(hist, (uint32_t)k - A, wsum, sel);
    const uint32_t d1 = sel[0], above1 = sel[1];
    if (sorted) {
      uint32_t nk = 0;
#pragma unroll
      for (int j = 0; j < PC; ++j) nk += (live(j) && dg1(j) >= d1) ? 1u : 0u;
      uint32_t kept;
      uint32_t off = block_incl_scan<kTopkThreads>(nk, wsum, kept) - nk;
      const int m = (int)(A + kept);
      int P = 64;
      while (P < m) P <<= 1;
      for (int i = tid; i < P; i += kTopkThreads) sortbuf[i] = i < (int)A ? al[i] : 0ull;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < PC; ++j)
        if (live(j) && dg1(j) >= d1) sortbuf[A + off++] = cv[j];
      __syncthreads();
      bitonic_desc<kTopkThreads>(sortbuf, P);
      for (int i = tid; i < k; i += kTopkThreads) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sortbuf[i]);
    } else {
      // exact threshold: bits 9..0 among the candidates of digit d1
      const uint32_t need1 = (uint32_t)k - A - above1;
      for (int b = tid; b < kBins; b += kTopkThreads) hist[b] = 0u;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < PC; ++j)
        if (live(j) && dg1(j) == d1) atomicAdd(&hist[dg2(j)], 1u);
      __syncthreads();
      pick_digit(hist, need1, wsum, sel);
      const uint32_t d2 = sel[0];
      const uint32_t need = need1 - sel[1];        // keys equal to T to take (lowest indices)
      if (tid == 0) sel[4] = (uint32_t)(cl[0] >> 53);   // the candidates' common top digit
      if (tid == 0) sel[5] = 0u;
      __syncthreads();
      const uint32_t T = (sel[4] << 21) | (d1 << 10) | d2;
      uint32_t* eql = reinterpret_cast<uint32_t*>(sortbuf);            // [kEqMax] indices equal to T
      uint32_t* bits = eql + kEqMax;                                    // [ceil(n/32)] selection bitmap
      const int W = (n + 31) / 32;
      const bool fits = (size_t)(kEqMax + W) * 4 <= (size_t)kSortMax * 8;   // bitmap fits the LDS buffer
#pragma unroll
      for (int j = 0; j < PC; ++j)
        if (live(j) && (uint32_t)(cv[j] >> 32) == T) {
          const uint32_t slot = atomicAdd(&sel[5], 1u);
          if (slot < (uint32_t)kEqMax) eql[slot] = 0xFFFFFFFFu - (uint32_t)cv[j];
        }
      if (fits)
        for (int w = tid; w < W; w += kTopkThreads) bits[w] = 0u;
      __syncthreads();
      const uint32_t ceq = sel[5];
      if (ceq <= (uint32_t)kEqMax && fits) {
        for (int i = tid; i < (int)A; i += kTopkThreads) {
          const uint32_t idx = 0xFFFFFFFFu - (uint32_t)al[i];
          atomicOr(&bits[idx >> 5], 1u << (idx & 31));
        }
#pragma unroll
        for (int j = 0; j < PC; ++j) {
          if (!live(j)) continue;
          const uint32_t key = (uint32_t)(cv[j] >> 32);
          const uint32_t idx = 0xFFFFFFFFu - (uint32_t)cv[j];
          bool take = key > T;
          if (key == T) {
            uint32_t r = 0;
            for (uint32_t e = 0; e < ceq; ++e) r += eql[e] < idx ? 1u : 0u;
            take = r < need;
          }
          if (take) atomicOr(&bits[idx >> 5], 1u << (idx & 31));
        }
        __syncthreads();
        // compaction: thread t owns bitmap words [t*WPT, (t+1)*WPT)
        const int WPT = (W + kTopkThreads - 1) / kTopkThreads;
        uint32_t cnt = 0;
        for (int w = tid * WPT; w < min(W, (tid + 1) * WPT); ++w) cnt += __popc(bits[w]);
        uint32_t tot;
        uint32_t pos = block_incl_scan<kTopkThreads>(cnt, wsum, tot) - cnt;
        for (int w = tid * WPT; w < min(W, (tid + 1) * WPT); ++w) {
          uint32_t m = bits[w];
          while (m) {
            const int bpos = __ffs(m) - 1;
            m &= m - 1;
            if (pos < (uint32_t)k) o[pos] = w * 32 + bpos;
            ++pos;
          }
        }
      } else {
        fallback = true;
      }
    }
  }
  if (fallback) {
    __syncthreads();
    topk_row_exact<VEC>(x, n, k, sorted, sortbuf, hist, wsum, sel, o);
  }
  // leave the row's histogram and list counters at zero for the next call
  uint32_t* hr = ws.hist + (int64_t)row * kBins;
  for (int b = tid; b < kBins; b += kTopkThreads) hr[b] = 0u;
  if (tid == 0) {
    ws.cnt[row * kCntStride + 0] = 0u;
    ws.cnt[row * kCntStride + 1] = 0u;
  }
}

// ---- short rows: one wave per row ----
// Many rows of at most kWaveRow elements with k <= kWaveK: the row's order keys
// stay in the wave's registers (lane holds elements PER*lane .. +PER), the
// three digit passes histogram them in the wave's LDS and pick the digit with
// a suffix scan over the lanes, and the selection is compacted in index order
// (unsorted) or into an LDS list that an in-wave bitonic sort orders by
// (score desc, index asc).  No workgroup barrier anywhere.
constexpr int kWaveRow = 4096;
constexpr int kWaveK = 256;
constexpr int kWaveRowsPerWG = 4;

template <bool VEC, int PER>
__global__ __launch_bounds__(64 * kWaveRowsPerWG) void topk_wave_kernel(const float* scores, int64_t row_stride,
                                                                        int64_t rows, int n, int k, int32_t* out,
                                                                        int64_t out_stride, int sorted,
                                                                        uint32_t* ghist) {
  static_assert(PER % 4 == 0 && 64 * PER <= kWaveRow, "keys per lane");
  __shared__ __attribute__((aligned(16))) uint32_t hist_s[kWaveRowsPerWG][kBins];
  __shared__ uint64_t sb_s[kWaveRowsPerWG][kWaveK];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaveRowsPerWG + w;
  if (row >= rows) return;                       // wave-uniform
  uint32_t* hist = hist_s[w];
  uint64_t* sb = sb_s[w];
  const float* x = scores + row * row_stride;
  const auto rs = row_rsrc(x, n);
  int32_t* o = out + row * out_stride;

  uint32_t key[PER];
  const int i0 = PER * lane;                     // this lane's first element
#pragma unroll
  for (int j = 0; j < PER / 4; ++j) {
    uint32_t kq[4];
    bool okq[4];
    load4<VEC>(rs, i0 + 4 * j, n, kq, okq);
#pragma unroll
    for (int e = 0; e < 4; ++e) key[4 * j + e] = kq[e];
  }
  uint32_t T, need;
  wave_select_threshold<PER>(key, n, k, hist, T, need);
  if (ghist) {                                   // a histogram the caller built: leave it at zero
    u32x4* gh = reinterpret_cast<u32x4*>(ghist + row * kBins) + lane * 8;
#pragma unroll
    for (int q = 0; q < 8; ++q) gh[q] = u32x4{0u, 0u, 0u, 0u};
  }
  // compaction in index order (lane, q): slot = selected keys before this one
  wave_select_compact<PER>(key, n, T, need, [&](uint32_t pos, int idx, uint32_t kk) {
    if (sorted) sb[pos] = sort_val(kk, idx);
    else o[pos] = idx;
  });
  if (!sorted) return;

  // in-wave bitonic sort of sb[0, P) into descending order (padding zeros sort last)
  int P = 64;
  while (P < k) P <<= 1;
  for (int i = k + lane; i < P; i += 64) sb[i] = 0ull;
  wave_lds_sync();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      for (int p = lane; p < P / 2; p += 64) {
        const int lo = ((p & ~(stride - 1)) << 1) | (p & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t va = sb[lo], vb = sb[hi];
        if ((va < vb) == desc) {
          sb[lo] = vb;
          sb[hi] = va;
        }
      }
      wave_lds_sync();
    }
  }
  for (int i = lane; i < k; i += 64) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sb[i]);
}

// Rows of at most kSmallRow elements that the wave kernel does not take (few
// rows, or larger k): one 256-thread workgroup per row, the row's order keys
// in registers (thread t holds elements PER*t .. +PER, read from memory once),
// selected by block_select (8-bit digit passes from the highest bit in which
// the row's keys differ, one barrier per pass); one scan of the per-thread
// counts places the selection in index order, or into an LDS list sorted by
// (score desc, index asc).
constexpr int kSmallThreads = 256;
constexpr int kSmallRow = 4096;
constexpr int kSmallSortK = 1024;

template <bool VEC, int PER>
__global__ __launch_bounds__(kSmallThreads) void topk_small_kernel(const float* scores, int64_t row_stride, int n,
                                                                   int k, int32_t* out, int64_t out_stride,
                                                                   int sorted, uint32_t* ghist) {
  constexpr int NT = kSmallThreads;
  constexpr int BPT = kBins / NT;                // caller histogram words cleared per thread
  static_assert(PER % 4 == 0 && NT * PER <= kSmallRow && BPT % 4 == 0, "keys and bins per thread");
  __shared__ __attribute__((aligned(16))) uint32_t ws[block_select_words<NT>()];
  __shared__ uint64_t sb[kSmallSortK];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* x = scores + row * row_stride;
  const auto rs = row_rsrc(x, n);
  int32_t* o = out + row * out_stride;

  uint32_t key[PER];
  const int i0 = PER * tid;                      // this thread's first element
#pragma unroll
  for (int j = 0; j < PER / 4; ++j) {
    uint32_t kq[4];
    bool okq[4];
    load4<VEC>(rs, i0 + 4 * j, n, kq, okq);
#pragma unroll
    for (int e = 0; e < 4; ++e) key[4 * j + e] = kq[e];
  }
  const BlockSel sel = block_select<NT, PER>(key, n, k, ws);
  if (ghist) {                                   // a histogram the caller built: leave it at zero
    u32x4* gh = reinterpret_cast<u32x4*>(ghist + row * kBins) + tid * (BPT / 4);
#pragma unroll
    for (int q = 0; q < BPT / 4; ++q) gh[q] = u32x4{0u, 0u, 0u, 0u};
  }
  // placement in index order
  block_select_emit<NT, PER>(key, n, sel, ws, [&](uint32_t pos, int idx, uint32_t kk) {
    if (sorted) sb[pos] = sort_val(kk, idx);
    else o[pos] = idx;
  });
  if (!sorted) return;
  int P = 64;
  while (P < k) P <<= 1;
  for (int i = k + tid; i < P; i += NT) sb[i] = 0ull;   // padding sorts last
  __syncthreads();
  bitonic_desc<NT>(sb, P);
  for (int i = tid; i < k; i += NT) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sb[i]);
}

// ---- k > kTopkMaxK on long rows: the selection in index order ----
// 1. filter (many workgroups per row): the digit d0 holding the k-th largest
//    key (from the row's histogram); each slice records how many of its keys
//    lie in larger digits and appends the keys of digit d0 to the row's
//    candidate list (any order);
// 2. select (one workgroup per row): among the candidates, block_select finds
//    the (k - above)-th largest; ties at the threshold are ranked by index in a
//    second block_select over the tied keys' complemented indices.  The result
//    is a predicate on (key, index) that holds for exactly k elements, plus
//    every slice's output offset (its above count and selected candidates,
//    summed over the slices before it).  Rows whose candidates overflow the
//    list run the one-workgroup exact path instead and are marked done;
// 3. write (many workgroups per row): each slice writes the indices that
//    satisfy the predicate, in index order, from its offset.
template <bool VEC>
__global__ __launch_bounds__(kPassThreads) void topk_large_filter_kernel(const float* scores, int64_t row_stride,
                                                                         int n, int k, int parts, TopkWs ws) {
  __shared__ uint32_t wsum[kPassThreads / 64];
  __shared__ uint32_t sel[4];
  const int row = blockIdx.x / parts, part = blockIdx.x - (blockIdx.x / parts) * parts;
  const float* x = scores + (int64_t)row * row_stride;
  const auto rs = row_rsrc(x, n);
  constexpr int R = kSlice / (kPassThreads * 4);
  uint32_t key[R][4];
  bool ok[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = part * kSlice + (r * kPassThreads + threadIdx.x) * 4;
    load4<VEC>(rs, i, n, key[r], ok[r]);
  }
  find_digit<kPassThreads>(ws.hist + (int64_t)row * kBins, (uint32_t)k, wsum, sel);
  const uint32_t d0 = sel[0];
  uint32_t na = 0, nc = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[r][j]) continue;
      const uint32_t d = key[r][j] >> 21;
      na += d > d0 ? 1u : 0u;
      nc += d == d0 ? 1u : 0u;
    }
  static_assert(kSlice < 65536, "packed counts");
  uint32_t tp;
  const uint32_t packed = (nc << 16) | na;
  const uint32_t op = block_incl_scan<kPassThreads>(packed, wsum, tp) - packed;
  uint32_t oc = op >> 16;
  const uint32_t tc = tp >> 16;
  if (threadIdx.x == 0) {
    ws.sabove[row * parts + part] = tp & 0xFFFFu;
    sel[3] = tc ? atomicAdd(ws.cnt + row * kCntStride + 1, tc) : 0u;
  }
  __syncthreads();
  oc += sel[3];
  uint64_t* cl = ws.cand + (int64_t)row * kLargeCand;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[r][j] || (key[r][j] >> 21) != d0) continue;
      if (oc < (uint32_t)kLargeCand) cl[oc] = sort_val(key[r][j], part * kSlice + (r * kPassThreads + threadIdx.x) * 4 + j);
      ++oc;
    }
}

// One row's selection among its Cn <= NT*PER candidates (see above); thread t
// holds candidates PER*t .. +PER.
template <int PER>
__device__ void topk_large_choose(const uint64_t* cl, uint32_t Cn, uint32_t kc, int parts, const uint32_t* sabove,
                                  uint32_t* soff, uint32_t* pr, uint32_t* lws, uint32_t* sc, uint32_t* wsum) {
  constexpr int NT = kTopkThreads;
  const int tid = threadIdx.x;
  uint32_t key[PER], idx[PER];
#pragma unroll
  for (int j = 0; j < PER; j += 2) {
    const int e = PER * tid + j;                 // even: one 16-byte load holds entries e, e+1
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (e < (int)Cn) v = ld16(cl + e);
    if (e + 1 >= (int)Cn) v[2] = v[3] = 0u;
    key[j] = v[1];
    idx[j] = 0xFFFFFFFFu - v[0];
    key[j + 1] = v[3];
    idx[j + 1] = 0xFFFFFFFFu - v[2];
  }
  const BlockSel bs = block_select<NT, PER>(key, (int)Cn, (int)kc, lws);
  uint32_t P2 = 0u, M2 = 0u;
  if (!bs.all) {
    // keys equal to the threshold (bs.M is full here): the bs.need lowest
    // indices are the largest complemented indices
    uint32_t k2[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) k2[j] = (PER * tid + j < (int)Cn && key[j] == bs.P) ? ~idx[j] : 0u;
    __syncthreads();                             // every thread is done with lws
    const BlockSel b2 = block_select<NT, PER>(k2, (int)Cn, (int)bs.need, lws);
    P2 = b2.P;
    M2 = b2.M;
  }
  for (int i = tid; i < parts; i += NT) sc[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (PER * tid + j >= (int)Cn) continue;
    const uint32_t m = key[j] & bs.M;
    const bool take = m > bs.P || (m == bs.P && (bs.all || ((~idx[j] & M2) >= P2)));
    if (take) atomicAdd(&sc[idx[j] / kSlice], 1u);
  }
  __syncthreads();
  // slice offsets: thread t owns slices 2t, 2t+1 (parts <= 2 * NT)
  static_assert(kLargeMaxParts <= 2 * NT, "slices per thread");
  const int s0 = 2 * tid, s1 = 2 * tid + 1;
  const uint32_t v0 = s0 < parts ? sabove[s0] + sc[s0] : 0u;
  const uint32_t v1 = s1 < parts ? sabove[s1] + sc[s1] : 0u;
  uint32_t total;
  const uint32_t excl = block_incl_scan<NT>(v0 + v1, wsum, total) - v0 - v1;
  if (s0 < parts) soff[s0] = excl;
  if (s1 < parts) soff[s1] = excl + v0;
  if (tid == 0) {
    pr[0] = bs.P;
    pr[1] = bs.M;
    pr[2] = P2;
    pr[3] = M2;
    pr[4] = bs.all;
    pr[5] = 1u;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kTopkThreads) void topk_large_select_kernel(const float* scores, int64_t row_stride,
                                                                         int n, int k, int parts, TopkWs ws,
                                                                         int32_t* out, int64_t out_stride) {
  constexpr int NT = kTopkThreads;
  __shared__ __attribute__((aligned(16))) uint32_t lws[block_select_words<NT>()];
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wsum[NT / 64];
  __shared__ uint32_t sel[8];
  __shared__ uint32_t sc[kLargeMaxParts];
  const int row = blockIdx.x, tid = threadIdx.x;
  uint32_t* pr = ws.par + row * kLargePar;
  find_digit<NT>(ws.hist + (int64_t)row * kBins, (uint32_t)k, wsum, sel);
  const uint32_t kc = (uint32_t)k - sel[1];      // to take among the candidates (keys above the digit: sel[1])
  const uint32_t Cn = ws.cnt[row * kCntStride + 1];
  const uint64_t* cl = ws.cand + (int64_t)row * kLargeCand;
  const uint32_t* sa = ws.sabove + row * parts;
  uint32_t* so = ws.soff + row * parts;
  // as few candidates per thread as the list needs: every slot costs a
  // histogram add in each digit pass
  if (Cn <= (uint32_t)(NT * 4)) topk_large_choose<4>(cl, Cn, kc, parts, sa, so, pr, lws, sc, wsum);
  else if (Cn <= (uint32_t)(NT * 8)) topk_large_choose<8>(cl, Cn, kc, parts, sa, so, pr, lws, sc, wsum);
  else if (Cn <= (uint32_t)kLargeCand) topk_large_choose<kLargeCand / NT>(cl, Cn, kc, parts, sa, so, pr, lws, sc, wsum);
  else {
    // the threshold digit holds more keys than the list: exact path over the row
    __syncthreads();
    topk_row_exact<VEC>(scores + (int64_t)row * row_stride, n, k, 0, nullptr, hist, wsum, sel,
                        out + (int64_t)row * out_stride);
    if (tid == 0) pr[5] = 0u;                    // written: the write pass skips the row
  }
  // leave the row's histogram and list counters at zero for the next call
  uint32_t* hr = ws.hist + (int64_t)row * kBins;
  for (int b = tid; b < kBins; b += NT) hr[b] = 0u;
  if (tid == 0) ws.cnt[row * kCntStride + 1] = 0u;
}

template <bool VEC>
__global__ __launch_bounds__(kPassThreads) void topk_large_write_kernel(const float* scores, int64_t row_stride,
                                                                        int n, int k, int parts, TopkWs ws,
                                                                        int32_t* out, int64_t out_stride) {
  __shared__ uint32_t wsum[kPassThreads / 64];
  const int row = blockIdx.x / parts, part = blockIdx.x - (blockIdx.x / parts) * parts;
  const uint32_t* pr = ws.par + row * kLargePar;
  if (pr[5] == 0u) return;                       // the select kernel wrote this row itself
  const float* x = scores + (int64_t)row * row_stride;
  const auto rs = row_rsrc(x, n);
  constexpr int R = kSlice / (kPassThreads * 4);
  static_assert(R == 4, "two packed scans of four 16-bit counts");
  uint32_t key[R][4];
  bool ok[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = part * kSlice + (r * kPassThreads + threadIdx.x) * 4;
    load4<VEC>(rs, i, n, key[r], ok[r]);
  }
  const uint32_t P = pr[0], M = pr[1], P2 = pr[2], M2 = pr[3], all = pr[4];
  bool take[R][4];
  uint32_t c[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    c[r] = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t idx = (uint32_t)(part * kSlice + (r * kPassThreads + threadIdx.x) * 4 + j);
      const uint32_t m = key[r][j] & M;
      take[r][j] = ok[r][j] && (m > P || (m == P && (all || ((~idx & M2) >= P2))));
      c[r] += take[r][j] ? 1u : 0u;
    }
  }
  // element order is (r, thread, j): scans of the per-r counts, two packed per
  // scan (each total <= 2048 < 2^16)
  uint32_t t01, t23;
  const uint32_t p01 = c[0] | (c[1] << 16), p23 = c[2] | (c[3] << 16);
  const uint32_t e01 = block_incl_scan<kPassThreads>(p01, wsum, t01) - p01;
  const uint32_t e23 = block_incl_scan<kPassThreads>(p23, wsum, t23) - p23;
  const uint32_t tot[R] = {t01 & 0xFFFFu, t01 >> 16, t23 & 0xFFFFu, t23 >> 16};
  const uint32_t ex[R] = {e01 & 0xFFFFu, e01 >> 16, e23 & 0xFFFFu, e23 >> 16};
  int32_t* o = out + (int64_t)row * out_stride;
  uint32_t base = ws.soff[row * parts + part];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t pos = base + ex[r];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (take[r][j]) {
        if (pos < (uint32_t)k) o[pos] = part * kSlice + (r * kPassThreads + threadIdx.x) * 4 + j;
        ++pos;
      }
    base += tot[r];
  }
}

// ---- sorted output for k > kTopkMaxK ----
// Block j of a row's selection (entries j*8192 .. +8192 of `out`, listed by
// ascending index): sort values (order key, index) sorted descending in LDS
// and written to the row's part of `sorted`.
__global__ __launch_bounds__(kTopkThreads) void topk_sort_block_kernel(const float* scores, int64_t row_stride,
                                                                      int k, const int32_t* out,
                                                                      int64_t out_stride, uint64_t* sorted,
                                                                      int nblk) {
  extern __shared__ uint64_t sortbuf[];          // [kSortBlock]
  const int64_t row = blockIdx.x / nblk;
  const int blk = (int)(blockIdx.x - row * nblk);
  const int j0 = blk * kSortBlock, cnt = min(kSortBlock, k - j0);
  const float* x = scores + row * row_stride;
  const int32_t* o = out + row * out_stride + j0;
  for (int i = threadIdx.x; i < kSortBlock; i += kTopkThreads) {
    uint64_t v = 0ull;                           // padding sorts last (every real value is > 0)
    if (i < cnt) {
      const int idx = o[i];
      v = sort_val(order_key(x[idx]), idx);
    }
    sortbuf[i] = v;
  }
  __syncthreads();
  bitonic_desc<kTopkThreads>(sortbuf, kSortBlock);
  uint64_t* dst = sorted + row * (int64_t)topk_large_pad(k) + j0;
  for (int i = threadIdx.x; i < cnt; i += kTopkThreads) dst[i] = sortbuf[i];
}

// Final slot of each selected entry: its rank in its own sorted block plus,
// for every other block, the number of that block's values above it (binary
// search; values are distinct, since the index is part of each).
constexpr int kRankThreads = 256;
__global__ __launch_bounds__(kRankThreads) void topk_rank_merge_kernel(const uint64_t* sorted, int k, int32_t* out,
                                                                      int64_t out_stride, int64_t per_row) {
  const int64_t row = blockIdx.x / per_row;
  const int j = (int)((blockIdx.x - row * per_row) * kRankThreads + threadIdx.x);
  if (j >= k) return;
  const uint64_t* srow = sorted + row * (int64_t)topk_large_pad(k);
  const uint64_t v = srow[j];
  const int own = j / kSortBlock;
  int rank = j - own * kSortBlock;
  const int nblk = (k + kSortBlock - 1) / kSortBlock;
  for (int b = 0; b < nblk; ++b) {
    if (b == own) continue;
    const uint64_t* blk = srow + b * kSortBlock;
    int lo = 0, hi = min(kSortBlock, k - b * kSortBlock);
    while (lo < hi) {                            // count of values > v (blocks are descending)
      const int mid = (lo + hi) >> 1;
      if (blk[mid] > v) lo = mid + 1;
      else hi = mid;
    }
    rank += lo;
  }
  out[row * out_stride + rank] = (int32_t)(0xFFFFFFFFu - (uint32_t)v);
}

static int topk_sort_large(const float* scores, int64_t rows, int64_t row_stride, int k, int32_t* out,
                           int64_t out_stride, const TopkWs& ws, hipStream_t st) {
  static bool lds_set = false;   // 64 KB of dynamic LDS: at the default limit, set once to be explicit
  if (!lds_set) {
    int rc = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_sort_block_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kSortBlock * 8);
    if (rc) return rc;
    lds_set = true;
  }
  const int nblk = (k + kSortBlock - 1) / kSortBlock;
  const int64_t per_row = (k + kRankThreads - 1) / kRankThreads;
  if (rows * nblk > 0x7FFFFFFFL || rows * per_row > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(topk_sort_block_kernel, dim3((unsigned)(rows * nblk)), dim3(kTopkThreads), kSortBlock * 8, st,
                     scores, row_stride, k, out, out_stride, ws.sorted, nblk);
  hipLaunchKernelGGL(topk_rank_merge_kernel, dim3((unsigned)(rows * per_row)), dim3(kRankThreads), 0, st, ws.sorted,
                     k, out, out_stride, per_row);
  return (int)hipGetLastError();
}

template <bool VEC>
static int topk_launch(const float* scores, int64_t rows, int n, int64_t row_stride, int k, int32_t* out,
                       int64_t out_stride, int sorted, int hist_ready, const TopkWs& ws, hipStream_t st) {
  static bool lds_set = false;   // the select kernel's dynamic LDS exceeds the 64 KB default
  if (!lds_set) {
    int rc = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_select_kernel<VEC>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kSortMax * 8);
    if (rc) return rc;
    lds_set = true;
  }
  const int parts = (n + kSlice - 1) / kSlice;
  // one wave per row when there are more rows than CUs: the one-workgroup
  // path (16 waves per row, one workgroup per CU at a time) then runs in
  // several generations, while four rows per workgroup all stay resident;
  // with fewer rows the 16-wave workgroups finish each row sooner
  if (n <= kWaveRow && k <= kWaveK && rows > device_cu_count()) {
    const int64_t g = (rows + kWaveRowsPerWG - 1) / kWaveRowsPerWG;
    if (g > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
    uint32_t* gh = hist_ready ? ws.hist : nullptr;
    if (n <= 2048)
      hipLaunchKernelGGL((topk_wave_kernel<VEC, 32>), dim3((unsigned)g), dim3(64 * kWaveRowsPerWG), 0, st, scores,
                         row_stride, rows, n, k, out, out_stride, sorted, gh);
    else
      hipLaunchKernelGGL((topk_wave_kernel<VEC, 64>), dim3((unsigned)g), dim3(64 * kWaveRowsPerWG), 0, st, scores,
                         row_stride, rows, n, k, out, out_stride, sorted, gh);
    return (int)hipGetLastError();
  }
  // other rows of at most kSmallRow elements: a 256-thread workgroup per row
  if (n <= kSmallRow && (!sorted || k <= kSmallSortK)) {
    if (rows > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
    uint32_t* gh = hist_ready ? ws.hist : nullptr;
    const dim3 grid((unsigned)rows), block(kSmallThreads);
    if (n <= 1024)
      hipLaunchKernelGGL((topk_small_kernel<VEC, 4>), grid, block, 0, st, scores, row_stride, n, k, out, out_stride,
                         sorted, gh);
    else if (n <= 2048)
      hipLaunchKernelGGL((topk_small_kernel<VEC, 8>), grid, block, 0, st, scores, row_stride, n, k, out, out_stride,
                         sorted, gh);
    else
      hipLaunchKernelGGL((topk_small_kernel<VEC, 16>), grid, block, 0, st, scores, row_stride, n, k, out,
                         out_stride, sorted, gh);
    return (int)hipGetLastError();
  }
  // k beyond the list capacity on long rows: filter, per-row select, ordered write
  if (k > kTopkMaxK && n > kShortRow && parts <= kLargeMaxParts) {
    for (int64_t r0 = 0; r0 < rows; r0 += kRowBatch) {
      const int nr = (int)(rows - r0 < kRowBatch ? rows - r0 : kRowBatch);
      const float* s = scores + r0 * row_stride;
      int32_t* o = out + r0 * out_stride;
      const unsigned grid = (unsigned)(nr * parts);
      if (!hist_ready)
        hipLaunchKernelGGL(topk_hist_kernel<VEC>, dim3(grid), dim3(kPassThreads), 0, st, s, row_stride, n, parts,
                           ws.hist);
      hipLaunchKernelGGL(topk_large_filter_kernel<VEC>, dim3(grid), dim3(kPassThreads), 0, st, s, row_stride, n, k,
                         parts, ws);
      hipLaunchKernelGGL(topk_large_select_kernel<VEC>, dim3((unsigned)nr), dim3(kTopkThreads), 0, st, s, row_stride,
                         n, k, parts, ws, o, out_stride);
      hipLaunchKernelGGL(topk_large_write_kernel<VEC>, dim3(grid), dim3(kPassThreads), 0, st, s, row_stride, n, k,
                         parts, ws, o, out_stride);
      const int rc = (int)hipGetLastError();
      if (rc) return rc;
    }
    return 0;
  }
  // short rows, and k beyond the list capacity (unsorted output: the exact
  // path writes the selection straight to `out` in index order)
  const int exact = (n <= kShortRow || k > kTopkMaxK) ? 1 : 0;
  if (exact) {
    if (rows > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(topk_select_kernel<VEC>, dim3((unsigned)rows), dim3(kTopkThreads), kSortMax * 8, st, scores,
                       row_stride, n, k, ws, out, out_stride, exact, sorted, hist_ready);
    return (int)hipGetLastError();
  }
  for (int64_t r0 = 0; r0 < rows; r0 += kRowBatch) {
    const int nr = (int)(rows - r0 < kRowBatch ? rows - r0 : kRowBatch);
    const float* s = scores + r0 * row_stride;
    int32_t* o = out + r0 * out_stride;
    const unsigned grid = (unsigned)(nr * parts);
    if (!hist_ready)
      hipLaunchKernelGGL(topk_hist_kernel<VEC>, dim3(grid), dim3(kPassThreads), 0, st, s, row_stride, n, parts,
                         ws.hist);
    hipLaunchKernelGGL(topk_filter_kernel<VEC>, dim3(grid), dim3(kPassThreads), 0, st, s, row_stride, n, k, parts,
                       ws);
    hipLaunchKernelGGL(topk_select_kernel<VEC>, dim3((unsigned)nr), dim3(kTopkThreads), kSortMax * 8, st, s,
                       row_stride, n, k, ws, o, out_stride, exact, sorted, hist_ready);
    const int rc = (int)hipGetLastError();
    if (rc) return rc;
  }
  return 0;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_topk_workspace_size(int64_t rows, int n, int k, size_t* bytes) {
  if (!bytes || rows < 0 || n <= 0 || k <= 0 || k > n) return (int)hipErrorInvalidValue;
  *bytes = topk_ws_bytes(rows, n, k);
  return 0;
}

int bytes_topk(const void* scores, int64_t rows, int n, int64_t row_stride, int k, int sorted, int hist_ready,
               void* out, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  if (!scores || !out || rows < 0 || n <= 0 || k <= 0 || k > n) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  const long parts = (n + kSlice - 1) / kSlice;
  if (kRowBatch * parts > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  if (!workspace || workspace_bytes < topk_ws_bytes(rows, n, k)) return (int)hipErrorInvalidValue;
  if (hist_ready && rows > kRowBatch) return (int)hipErrorInvalidValue;
  const TopkWs ws = topk_ws_carve(workspace, rows, n, k);
  const bool vec = (reinterpret_cast<uintptr_t>(scores) % 16 == 0) && (row_stride % 4 == 0) && (n % 4 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float* s = static_cast<const float*>(scores);
  int32_t* o = static_cast<int32_t*>(out);
  // k > kTopkMaxK sorted: the selection by ascending index, then sorted
  const bool large_sorted = sorted && k > kTopkMaxK;
  const int so = (sorted && !large_sorted) ? 1 : 0, hr = hist_ready ? 1 : 0;
  prof_begin(kProfTopk, st);
  int rc = vec ? topk_launch<true>(s, rows, n, row_stride, k, o, out_stride, so, hr, ws, st)
               : topk_launch<false>(s, rows, n, row_stride, k, o, out_stride, so, hr, ws, st);
  if (rc == 0 && large_sorted) rc = topk_sort_large(s, rows, row_stride, k, o, out_stride, ws, st);
  prof_end(kProfTopk, st);
  return rc;
}

}  // extern "C"
