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
//    S - 1 (:358-363);
//  * select_merge_kernel: one step of the streaming top-k over key chunks
//    (:286-309): the top-k positions of a row's [running list | chunk]
//    candidates become the next running list of (score, key index) pairs;
//  * select_recent_kernel: the "recent" selector (:261-265), idx =
//    max(pos - j, 0).
// Row r of a [.., Qc, n] tensor belongs to query row r % Qc, whose position is
// pos[r % Qc] (int64 on the device, the reference's q_pos).
#include "common.h"

namespace bytes_amd {

constexpr int kSelThreads = 256;

// Candidate t stands for position (key0 + t) * unit (unit 1: tokens; page
// size: pages; key0: the first candidate's index, for a chunk of keys).
// Causally valid iff t * unit <= pos; forced (+inf) iff local_w > 0 and
// t lies in [max(pos - local_w + 1, 0) / unit, pos / unit].
__global__ __launch_bounds__(kSelThreads) void select_mask_kernel(float* s, int64_t rows, int n, int64_t rs,
                                                                  int64_t key0, const int64_t* pos, int Qc,
                                                                  int unit, int local_w, int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int64_t j = (blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x;
  if (r >= rows || j >= n) return;
  const int64_t t = key0 + j;
  const int64_t p = pos[r % Qc];
  float* row = s + r * rs;
  float v = row[j];
  if (t * unit > p) v = kNegInf;
  if (local_w > 0) {
    const int64_t lo = (p - local_w + 1 > 0 ? p - local_w + 1 : 0) / unit, hi = p / unit;
    if (t >= lo && t <= hi) v = __builtin_inff();
  }
  row[j] = v;
}

// Row r's candidates are cand[r][off .. off + nrun + n): its running list of
// nrun (score, key index) pairs (indices in ridx[r]) followed by the scores
// of keys kc0, kc0 + 1, ...  sel[r] holds the top-ksel candidate positions;
// entry i < ksel of the next running list is the candidate at sel[r][i],
// entries ksel <= i < kout are fillers (-inf, S).
__global__ __launch_bounds__(kSelThreads) void select_merge_kernel(const float* cand, int64_t cand_rs, int off,
                                                                   int nrun, const int32_t* ridx, int64_t ridx_rs,
                                                                   const int32_t* sel, int64_t sel_rs, int ksel,
                                                                   int kc0, int S, int64_t rows, float* out_v,
                                                                   int64_t out_v_rs, int out_off, int32_t* out_i,
                                                                   int64_t out_i_rs, int kout,
                                                                   int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int i = (int)((blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x);
  if (r >= rows || i >= kout) return;
  float v = kNegInf;
  int idx = S;
  if (i < ksel) {
    const int p = sel[r * sel_rs + i];
    v = cand[r * cand_rs + off + p];
    idx = p < nrun ? ridx[r * ridx_rs + p] : kc0 + (p - nrun);
  }
  if (out_v) out_v[r * out_v_rs + out_off + i] = v;
  out_i[r * out_i_rs + i] = idx;
}

// "recent": the kb most recent causal positions of row r, pos - j clamped at 0.
__global__ __launch_bounds__(kSelThreads) void select_recent_kernel(const int64_t* pos, int Qc, int64_t rows, int kb,
                                                                    int64_t* out, int64_t blocks_per_row) {
  const int64_t r = blockIdx.x / blocks_per_row;
  const int j = (int)((blockIdx.x - r * blocks_per_row) * kSelThreads + threadIdx.x);
  if (r >= rows || j >= kb) return;
  const int64_t v = pos[r % Qc] - j;
  out[r * kb + j] = v > 0 ? v : 0;
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

int bytes_select_mask_at(void* scores, int64_t rows, int n, int64_t row_stride, int64_t key0, const void* pos,
                         int Qc, int unit, int local_w, void* stream) {
  if (!scores || !pos || rows <= 0 || n <= 0 || Qc <= 0 || unit <= 0 || local_w < 0 || row_stride < n || key0 < 0)
    return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, n, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(select_mask_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<float*>(scores), rows, n, row_stride, key0,
                     static_cast<const int64_t*>(pos), Qc, unit, local_w, bpr);
  return (int)hipGetLastError();
}

int bytes_select_mask(void* scores, int64_t rows, int n, int64_t row_stride, const void* pos, int Qc, int unit,
                      int local_w, void* stream) {
  return bytes_select_mask_at(scores, rows, n, row_stride, 0, pos, Qc, unit, local_w, stream);
}

int bytes_select_merge(const void* cand, int64_t cand_rs, int off, int nrun, const void* ridx, int64_t ridx_rs,
                       const void* sel, int64_t sel_rs, int ksel, int kc0, int S, int64_t rows, void* out_vals,
                       int64_t out_vals_rs, int out_off, void* out_idx, int64_t out_idx_rs, int kout,
                       void* stream) {
  if (!cand || !sel || !out_idx || rows <= 0 || ksel <= 0 || kout < ksel || nrun < 0 || off < 0 || kc0 < 0 ||
      S <= 0 || out_off < 0 || (nrun > 0 && !ridx))
    return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, kout, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(select_merge_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(cand), cand_rs, off, nrun,
                     static_cast<const int32_t*>(ridx), ridx_rs, static_cast<const int32_t*>(sel), sel_rs, ksel,
                     kc0, S, rows, static_cast<float*>(out_vals), out_vals_rs, out_off,
                     static_cast<int32_t*>(out_idx), out_idx_rs, kout, bpr);
  return (int)hipGetLastError();
}

int bytes_select_recent(const void* pos, int Qc, int64_t rows, int kb, void* out, void* stream) {
  if (!pos || !out || Qc <= 0 || rows <= 0 || kb <= 0) return (int)hipErrorInvalidValue;
  int64_t bpr, blocks;
  if (!grid_of(rows, kb, &bpr, &blocks)) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(select_recent_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const int64_t*>(pos), Qc, rows, kb,
                     static_cast<int64_t*>(out), bpr);
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
