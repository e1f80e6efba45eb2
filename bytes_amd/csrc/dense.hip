// Dense bf16 GQA single-query decode attention (split-K flash-decode).
//
// Replaces src/attention_kernels.py:8-92 (`_decode_attn_bf16_kernel` /
// `decode_attn_bf16`).  The reference launches one program per (b, h_q) and
// so streams each KV head G times; here one workgroup serves all query heads
// of a GQA group for one chunk of the token axis, so K and V are read once.
//
// Per wave, per 32-token tile (waves of a workgroup take interleaved tiles):
//   S^T[t][h] = K[t][:] . Q[h][:]    two 16x16 MFMA blocks over D; A = K rows
//                                    loaded straight into VGPRs, B = Q in VGPRs
//   fp32 online softmax per head     lane l owns head l%16
//   O^T[d][h] += V^T[d][t] P^T[t][h] MFMA; V is staged through a
//                                    wave-private LDS buffer (XOR-swizzled
//                                    16-byte chunks, so the transposed reads
//                                    are bank-conflict free)
// The next tile's K and V loads are issued before the current tile is
// computed (two-stage software pipeline).
//
// The fp8 entry point (src/attention_kernels.py:156-182, `decode_attn_fp8`:
// OCP e4m3fn K and V, bf16 q, output in q's dtype, no scale) runs the same
// kernel with K/V rows widened to bf16 (exactly) as they are staged in LDS.
#include <mutex>

#include "dense_tile.h"

namespace bytes_amd {

struct DenseArgs {
  const uint16_t* q;
  const void* k;             // bf16 or fp8 e4m3fn rows
  const void* v;
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int Hk, G, S, HB, chunk;
  float scale_log2;
  SplitKOut o;
};

template <int D, bool FP8>
__global__ __launch_bounds__(kDenseWaves * 64, 2) void dense_decode_kernel(DenseArgs a) {
  PREFETCH_ARGS(a);
  using C = DenseCfg<D>;
  __shared__ __attribute__((aligned(16))) char smem_raw[C::kSmem];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const UnitLoc loc = splitk_locate(a.o);
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk, hb = loc.hb;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);

  bf16x8 qb[C::KK];
  load_q_bf16<D>(a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh, a.q_sh, nh, lane, qb);

  const int t_begin = split * a.chunk;
  const int t_end = min(t_begin + a.chunk, a.S);
  char* wbuf = smem_raw + w * C::WAVE;

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (FP8) {
    const uint8_t* kbase = static_cast<const uint8_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
    const uint8_t* vbase = static_cast<const uint8_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
    dense_wave_loop_fp8<D>(kbase, vbase, a.k_ss, a.v_ss, a.S, t_begin, t_end, w, lane, a.scale_log2, qb, wbuf,
                           m_run, l_run, acc);
  } else {
    const uint16_t* kbase = static_cast<const uint16_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
    const uint16_t* vbase = static_cast<const uint16_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
    dense_wave_loop<D>(kbase, vbase, a.k_ss, a.v_ss, a.S, t_begin, t_end, w, lane, a.scale_log2, qb, wbuf, m_run,
                       l_run, acc);
  }

  splitk_epilogue<D, kDenseWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b,
                                  hq0, nh);
}

// Device-resident scratch of the no-allocation entry point: the split-K
// partials of one call (each device holds its own copy for the life of the
// process).  Host code never uses the symbol's name as an address: its
// device address is looked up once per device and kept in g_scratch.
constexpr size_t kNoAllocScratchBytes = 16u << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::once_flag g_scratch_once[kMaxDevices];
static void* g_scratch[kMaxDevices];
static int g_scratch_rc[kMaxDevices];

// This device's address of `scratch` (nullptr and a status on failure).
static void* scratch_address(int* rc) {
  int dev = 0;
  *rc = (int)hipGetDevice(&dev);
  if (*rc) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = (int)hipErrorInvalidDevice;
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_scratch_rc[dev] ? nullptr : p;
  });
  *rc = g_scratch_rc[dev];
  return g_scratch[dev];
}

// Host-side split choice: chunk is a multiple of (waves * tile) tokens; aim
// for per_cu workgroups per CU: one for bf16 K/V (measured faster than two at
// L = 16K and 32K: half the partials to merge, longer pipelines per wave),
// two for fp8 (whose rows are widened to bf16 as they are staged).  More
// workgroups per CU never means fewer splits, so the workspace query plans
// for two.
static void dense_plan(int S, long units, int chunk_req, int per_cu, int* chunk, int* nsplit) {
  const int step = kDenseWaves * kTile;
  int c;
  if (chunk_req > 0) {
    c = (chunk_req + step - 1) / step * step;
  } else {
    const long target = (long)per_cu * device_cu_count();
    long per = ((long)S * units + target - 1) / target;
    c = (int)((per + step - 1) / step * step);
    if (c < step) c = step;
  }
  int ns = (S + c - 1) / c;
  if (ns > 1024) {  // the merge keeps one weight per split in LDS
    c = ((S + 1023) / 1024 + step - 1) / step * step;
    ns = (S + c - 1) / c;
  }
  *chunk = c;
  *nsplit = ns;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_decode_attn_bf16_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk_req, size_t* bytes) {
  if (!bytes || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0 || (D != 64 && D != 128)) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  int chunk, ns;
  dense_plan(S, units, chunk_req, 2, &chunk, &ns);
  *bytes = splitk_workspace_bytes(units, ns, D);
  return 0;
}

static int dense_decode(bool fp8, const void* q, const void* k, const void* v, void* out, int B, int Hq, int Hk,
                        int S, int D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                        int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scale,
                        int chunk_req, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  if (units > 65535) return (int)hipErrorInvalidConfiguration;
  DenseArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = k;
  a.v = v;
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.Hk = Hk; a.G = G; a.S = S; a.HB = HB;
  a.scale_log2 = scale * kLog2e;
  int ns;
  dense_plan(S, units, chunk_req, fp8 ? 2 : 1, &a.chunk, &ns);
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  a.o.out = out;
  a.o.out_dtype = kOutBF16;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  a.o.Hk = Hk; a.o.HB = HB; a.o.G = G;
  splitk_carve(workspace, units, ns, a.o);
  dim3 grid((unsigned)(ns * units));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 block(kDenseWaves * 64);
  if (D == 64) {
    if (fp8) BYTES_LAUNCH(kProfDense, (dense_decode_kernel<64, true>), grid, block, 0, st, a);
    else BYTES_LAUNCH(kProfDense, (dense_decode_kernel<64, false>), grid, block, 0, st, a);
  } else {
    if (fp8) BYTES_LAUNCH(kProfDense, (dense_decode_kernel<128, true>), grid, block, 0, st, a);
    else BYTES_LAUNCH(kProfDense, (dense_decode_kernel<128, false>), grid, block, 0, st, a);
  }
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

int bytes_decode_attn_bf16(const void* q, const void* k, const void* v, void* out, int B, int Hq, int Hk, int S,
                           int D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scale,
                           int chunk_req, void* workspace, size_t workspace_bytes, void* stream) {
  return dense_decode(false, q, k, v, out, B, Hq, Hk, S, D, q_sb, q_sh, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb,
                      o_sh, scale, chunk_req, workspace, workspace_bytes, stream);
}

// The bf16 decode with its split-K partials in this device's `scratch`
// instead of a caller workspace: no allocation of any kind, so it serves
// callers that cannot allocate.  Every partial the merge reads is written
// earlier in the same call, so nothing in the scratch has to start at zero.
// Calls that overlap on one device share the scratch and race.
int bytes_decode_attn_bf16_noalloc(const void* q, const void* k, const void* v, void* out, int B, int Hq, int Hk,
                                   int S, int D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh,
                                   int64_t k_ss, int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb,
                                   int64_t o_sh, float scale, int chunk_req, void* stream) {
  size_t need = 0;
  int rc = bytes_decode_attn_bf16_workspace_size(B, Hq, Hk, S, D, chunk_req, &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes) return (int)hipErrorOutOfMemory;
  void* ws = scratch_address(&rc);
  if (rc) return rc;
  return dense_decode(false, q, k, v, out, B, Hq, Hk, S, D, q_sb, q_sh, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb,
                      o_sh, scale, chunk_req, ws, kNoAllocScratchBytes, stream);
}

// K/V element strides are in fp8 elements (bytes).
int bytes_decode_attn_fp8(const void* q, const void* k, const void* v, void* out, int B, int Hq, int Hk, int S,
                          int D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                          int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, float scale,
                          int chunk_req, void* workspace, size_t workspace_bytes, void* stream) {
  return dense_decode(true, q, k, v, out, B, Hq, Hk, S, D, q_sb, q_sh, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb,
                      o_sh, scale, chunk_req, workspace, workspace_bytes, stream);
}

}  // extern "C"
