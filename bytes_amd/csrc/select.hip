// Row-wise steps of the reference's selection functions for query chunks of
// Qc >= 1 rows (benchmarks/sparse_attention.py:226-387), around the score,
// top-k and gather kernels:
//  * select_mask_kernel: the causal mask and the forced recent window of
//    select_topk (:248-256, :298-300) and _quest_select (:346-355), applied in
//    place to fp32 scores of token or page candidates;
//  * select_fill_kernel: index lists with the sentinel rule (:288-293, :376):
//    an entry that is past the row's query position, negative, or at/after S
//    becomes S, and slots past the input width are filled with S;
//  * select_pages_kernel: page ids -> the token ids of their rows, clamped to
//    S - 1 (:358-363).
// Row r of a [.., Qc, n] tensor belongs to query row r % Qc, whose position is
// pos[r % Qc] (int64 on the device, the reference's q_pos).
#include "common.h"

namespace bytes_amd {

constexpr int kSelThreads = 256;

// Candidate t stands for position t * unit (unit 1: tokens; page size: pages).
// Causally valid iff t * unit <= pos; forced (+inf) iff local_w > 0 and
// t lies in [max(pos - local_w + 1, 0) / unit, pos / unit].
__global__ __launch_bounds__(kSelThreads) void select_mask_kernel(float* s, int64_t rows, int n, int64_t rs,
                                                                  const int64_t* pos, int Qc, int unit,
                                                                  int local_w, int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int64_t t = (blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x;
  if (r >= rows || t >= n) return;
  const int64_t p = pos[r % Qc];
  float* row = s + r * rs;
  float v = row[t];
  if (t * unit > p) v = kNegInf;
  if (local_w > 0) {
    const int64_t lo = (p - local_w + 1 > 0 ? p - local_w + 1 : 0) / unit, hi = p / unit;
    if (t >= lo && t <= hi) v = __builtin_inff();
  }
  row[t] = v;
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kSelThreads) void select_fill_kernel(const TI* in, int64_t in_rs, int k_in, TO* out,
                                                                  int64_t out_rs, int k_out, int64_t rows,
                                                                  const int64_t* pos, int Qc, int64_t S,
                                                                  int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int j = (int)((blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x);
  if (r >= rows || j >= k_out) return;
  const int64_t p = pos[r % Qc];
  int64_t v = S;
  if (j < k_in) {
    const int64_t x = (int64_t)in[r * in_rs + j];
    if (x >= 0 && x < S && x <= p) v = x;
  }
  out[r * out_rs + j] = (TO)v;
}

__global__ __launch_bounds__(kSelThreads) void select_pages_kernel(const int32_t* pid, int64_t rows, int npick,
                                                                   int page, int64_t S, int64_t* out,
                                                                   int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int j = (int)((blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x);
  if (r >= rows || j >= npick * page) return;
  const int64_t t = (int64_t)pid[r * npick + j / page] * page + j % page;
  out[r * (int64_t)npick * page + j] = t < S - 1 ? t : S - 1;
}

static bool grid_of(int64_t rows, int64_t width, int64_t* bpr, int64_t* blocks) {
  *bpr = (width + kSelThreads - 1) / kSelThreads;
  *blocks = rows * *bpr;
  return *blocks > 0 && *blocks <= 0x7FFFFFFFL;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_select_mask(void* scores, int64_t rows, int n, int64_t row_stride, const void* pos, int Qc, int unit,
                      int local_w, void* stream) {
  if (!scores || !pos || rows <= 0 || n <= 0 || Qc <= 0 || unit <= 0 || local_w < 0 || row_stride < n)
    return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, n, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(select_mask_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<float*>(scores), rows, n, row_stride,
                     static_cast<const int64_t*>(pos), Qc, unit, local_w, bpr);
  return (int)hipGetLastError();
}

// in_dtype / out_dtype: 0 int32, 1 int64.
int bytes_select_fill(const void* in, int in_dtype, int64_t in_rs, int k_in, void* out, int out_dtype,
                      int64_t out_rs, int k_out, int64_t rows, const void* pos, int Qc, int64_t S, void* stream) {
  if (!out || !pos || rows <= 0 || k_out <= 0 || k_in < 0 || (k_in > 0 && !in) || Qc <= 0 || S <= 0)
    return (int)hipErrorInvalidValue;
  if ((in_dtype != 0 && in_dtype != 1) || (out_dtype != 0 && out_dtype != 1)) return (int)hipErrorInvalidValue;
  if (out_dtype == 0 && S > 0x7FFFFFFFL) return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, k_out, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t* p = static_cast<const int64_t*>(pos);
  dim3 g((unsigned)blocks), b(kSelThreads);
#define SEL_FILL(TI, TO)                                                                                    \
  hipLaunchKernelGGL((select_fill_kernel<TI, TO>), g, b, 0, st, static_cast<const TI*>(in), in_rs, k_in, \
                     static_cast<TO*>(out), out_rs, k_out, rows, p, Qc, S, bpr)
  if (in_dtype == 0 && out_dtype == 0) SEL_FILL(int32_t, int32_t);
  else if (in_dtype == 0) SEL_FILL(int32_t, int64_t);
  else if (out_dtype == 0) SEL_FILL(int64_t, int32_t);
  else SEL_FILL(int64_t, int64_t);
#undef SEL_FILL
  return (int)hipGetLastError();
}

int bytes_select_pages(const void* page_ids, int64_t rows, int npick, int page, int64_t S, void* out,
                       void* stream) {
  if (!page_ids || !out || rows <= 0 || npick <= 0 || page <= 0 || S <= 0) return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, (int64_t)npick * page, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(select_pages_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const int32_t*>(page_ids), rows, npick, page,
                     S, static_cast<int64_t*>(out), bpr);
  return (int)hipGetLastError();
}

}  // extern "C"
