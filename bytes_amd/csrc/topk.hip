// Deterministic top-k over rows of fp32 scores.
//
// Replaces `scores.topk(kb, dim=-1).indices` on the sparse decode paths
// (src/attention_kernels.py:1262, benchmarks/sparse_attention.py:307 and
// :358), whose tie order is unspecified, with one total order: score
// descending, index ascending on equal scores (+0 and -0 are equal; NaN ranks
// above +inf, as in torch.topk).  Output: int32 indices [rows, k] ordered by
// that order, identical run to run.
//
// One 1024-thread workgroup per row:
//  1. radix select on 32-bit order keys, 11/11/10-bit digits from the top:
//     each pass builds an LDS histogram of the digit among the keys that
//     still match the selected prefix and picks the digit holding the k-th
//     largest key, so after three passes the k-th key T is known exactly,
//     along with how many keys equal to T are needed;
//  2. collection in index order: every key > T, plus the first `need` keys
//     equal to T (a workgroup scan gives each thread its rank among them);
//  3. bitonic sort of the k selected (key, ~index) pairs in LDS.
#include "common.h"

namespace bytes_amd {

constexpr int kTopkThreads = 1024;
constexpr int kTopkMaxK = 8192;
constexpr int kBins = 2048;

// Monotone key: larger score -> larger key.  NaN -> 0xFFFFFFFF, -0 -> +0.
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0xFFFFFFFFu;
  uint32_t u = __float_as_uint(x);
  if (x == 0.f) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 1024 threads of the workgroup (thread order).
__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  if (w == 0) {
    uint32_t s = lane < kTopkThreads / 64 ? wsum[lane] : 0u;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const uint32_t y = __shfl_up(s, off, 64);
      if (lane >= off) s += y;
    }
    if (lane < kTopkThreads / 64) wsum[lane] = s;
  }
  __syncthreads();
  total = wsum[kTopkThreads / 64 - 1];
  const uint32_t r = x + (w > 0 ? wsum[w - 1] : 0u);
  __syncthreads();   // wsum is reused by the next scan
  return r;
}

template <bool VEC>
__device__ __forceinline__ void load4(const float* x, int i, int n, uint32_t (&key)[4], bool (&ok)[4]) {
  if (VEC && i + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    key[0] = order_key(v.x); key[1] = order_key(v.y); key[2] = order_key(v.z); key[3] = order_key(v.w);
    ok[0] = ok[1] = ok[2] = ok[3] = true;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ok[j] = i + j < n;
      key[j] = ok[j] ? order_key(x[i + j]) : 0u;
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* scores, int64_t row_stride, int n, int k,
                                                            int P, int32_t* out, int64_t out_stride) {
  extern __shared__ uint64_t sortbuf[];          // [P] (key << 32) | ~index
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wsum[kTopkThreads / 64];
  __shared__ uint32_t sel[4];                    // digit, count above, slot counter, eq base
  const int tid = threadIdx.x;
  const float* x = scores + (int64_t)blockIdx.x * row_stride;

  // ---- 1. radix select ----
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
      load4<VEC>(x, i, n, key, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (ok[j] && (key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & dmask], 1u);
    }
    __syncthreads();
    // thread t owns digits 2t, 2t+1; count of keys in digits above 2t+1
    const uint32_t c0 = hist[2 * tid], c1 = hist[2 * tid + 1];
    uint32_t total;
    const uint32_t incl = block_incl_scan(c0 + c1, wsum, total);
    const uint32_t above = total - incl;     // digits > 2*tid + 1
    if (above < kr && above + c1 >= kr) {
      sel[0] = 2 * tid + 1;
      sel[1] = above;
    } else if (above + c1 < kr && above + c1 + c0 >= kr) {
      sel[0] = 2 * tid;
      sel[1] = above + c1;
    }
    __syncthreads();
    const uint32_t d = sel[0];
    kr -= sel[1];
    prefix |= d << shift;
    pmask |= dmask << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;
  const uint32_t need = kr;                      // keys equal to T to take, >= 1

  // ---- 2. collection (index order decides among keys equal to T) ----
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
    load4<VEC>(x, i, n, key, ok);
    uint32_t ne = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) ne += (ok[j] && key[j] == T) ? 1u : 0u;
    uint32_t rank = 0, tot = 0;
    if (__syncthreads_or(ne != 0)) {
      const uint32_t incl = block_incl_scan(ne, wsum, tot);
      rank = incl - ne;
    }
    const uint32_t eq0 = sel[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!ok[j]) continue;
      bool take = key[j] > T;
      if (key[j] == T) {
        take = eq0 + rank < need;
        ++rank;
      }
      if (take) {
        const uint32_t slot = atomicAdd(&sel[2], 1u);
        sortbuf[slot] = ((uint64_t)key[j] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(i + j));
      }
    }
    __syncthreads();
    if (tid == 0) sel[3] = eq0 + tot;
    __syncthreads();
  }

  // ---- 3. bitonic sort, descending ----
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P / 2; i += kTopkThreads) {
        const int lo = (i / stride) * stride * 2 + (i % stride);
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t va = sortbuf[lo], vb = sortbuf[hi];
        if ((va < vb) == desc) {
          sortbuf[lo] = vb;
          sortbuf[hi] = va;
        }
      }
      __syncthreads();
    }
  }
  int32_t* o = out + (int64_t)blockIdx.x * out_stride;
  for (int i = tid; i < k; i += kTopkThreads) o[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)sortbuf[i]);
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_topk(const void* scores, int64_t rows, int n, int64_t row_stride, int k, void* out, int64_t out_stride,
               void* stream) {
  if (!scores || !out || rows < 0 || n <= 0 || k <= 0 || k > n) return (int)hipErrorInvalidValue;
  if (k > kTopkMaxK) return (int)hipErrorNotSupported;
  if (rows == 0) return 0;
  if (rows > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  int P = 1;
  while (P < k) P <<= 1;
  if (P < 2) P = 2;
  const size_t lds = (size_t)P * 8;
  const bool vec = (reinterpret_cast<uintptr_t>(scores) % 16 == 0) && (row_stride % 4 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec) {
    int rc = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel<true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (rc) return rc;
    hipLaunchKernelGGL(topk_kernel<true>, dim3((unsigned)rows), dim3(kTopkThreads), lds, st,
                       static_cast<const float*>(scores), row_stride, n, k, P, static_cast<int32_t*>(out), out_stride);
  } else {
    int rc = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel<false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (rc) return rc;
    hipLaunchKernelGGL(topk_kernel<false>, dim3((unsigned)rows), dim3(kTopkThreads), lds, st,
                       static_cast<const float*>(scores), row_stride, n, k, P, static_cast<int32_t*>(out), out_stride);
  }
  return (int)hipGetLastError();
}

}  // extern "C"
