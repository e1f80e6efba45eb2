// Microkernels of the study harnesses.
//
// gather_reduce_kernel: the access-pattern probe of
// benchmarks/bench_access_pattern.py:25-52 (`_gather_reduce_kernel`): for each
// of H (batch x KV head) rows of an fp16 cache [H, S, D], the sum over the K
// listed token rows, out[h, d] = sum_k v[h, idx[h, k], d] in fp32 (entries
// outside [0, S) read the nearest row, so no index can leave the cache).  Only the
// index pattern changes between runs, so its achieved bandwidth isolates what
// the pattern costs.  One workgroup per h (the reference's program per h):
// the index list is staged in LDS, then each thread owns one 16-byte column
// chunk of the rows it visits and keeps two batches of eight rows in flight;
// the chunk sums are reduced through LDS in a fixed order.
//
// stream_read_kernel / empty_kernel: the floor probes the decode kernels are
// measured against.  G workgroups each read their own contiguous slice of a
// buffer in 16-byte loads, NL per thread in flight at a time, fold the words
// and write one float per thread; empty_kernel is a launch that does nothing.
// Together they give the fixed cost of a launch, the first HBM round trip and
// the streaming-read ceiling at a given grid.
//
// packed_stage_kernel: the staged packed-score probe of
// benchmarks/bench_unpack_ablation.py:19-53 (`_packed_stage_kernel`): per
// (b, query head) and key row t of packed 4/2-bit keys (the layout of
// quantize_and_pack_score_keys), with codes c, bf16 scale s and zero z per 32
// dims and the query q:
//   stage 0: sum over the D columns of the packed byte each column lives in
//   stage 1: sum_c code_c
//   stage 2: sum_c (code_c * s_g + z_g)
//   stage 3: sum_c (code_c * s_g + z_g) * q_c
// so the time of each stage adds one step (load, unpack, dequant, dot) of the
// score pass's work, on the vector ALUs.  A group of CPR lanes shares a row,
// one 16-byte chunk each (consecutive lanes, consecutive chunks), and folds
// its partial sums with lane shuffles.
#include "common.h"

namespace bytes_amd {

constexpr int kGrThreads = 256;
constexpr int kGrIdxMax = 16384;    // index-list entries staged in LDS at a time
constexpr int kGrUnroll = 8;

template <int CPR>
__global__ __launch_bounds__(kGrThreads) void gather_reduce_kernel(const uint16_t* v, int64_t v_sh, int64_t v_ss,
                                                                   const int32_t* idx, int64_t i_sh, int K,
                                                                   int S, float* out, int D) {
  __shared__ int32_t rows[kGrIdxMax];
  __shared__ float red[kGrThreads * 8];
  constexpr int R = kGrThreads / CPR;           // rows per pass of the workgroup
  const int h = blockIdx.x;
  const int c = threadIdx.x % CPR, r0 = threadIdx.x / CPR;
  const uint16_t* vh = v + (int64_t)h * v_sh + c * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int seg = 0; seg < K; seg += kGrIdxMax) {
    const int n = min(kGrIdxMax, K - seg);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kGrThreads) rows[i] = idx[(int64_t)h * i_sh + seg + i];
    __syncthreads();
    // batches of kGrUnroll rows per thread; the next batch is requested before
    // the current one is summed (rows past n read row 0 and are not summed)
    constexpr int BATCH = R * kGrUnroll;
    u32x4 cur[kGrUnroll], nxt[kGrUnroll];
    auto issue = [&](int j0, u32x4 (&dst)[kGrUnroll]) {
#pragma unroll
      for (int u = 0; u < kGrUnroll; ++u) {
        const int j = j0 + r0 + u * R;
        const int row = j < n ? min(max(rows[j], 0), S - 1) : 0;   // entries outside [0, S) read a clamped row
        dst[u] = ld16(vh + (int64_t)row * v_ss);
      }
    };
    issue(0, cur);
    for (int j0 = 0; j0 < n; j0 += BATCH) {
      issue(j0 + BATCH < n ? j0 + BATCH : 0, nxt);
#pragma unroll
      for (int u = 0; u < kGrUnroll; ++u) {
        if (j0 + r0 + u * R < n) {
          const _Float16* e = reinterpret_cast<const _Float16*>(&cur[u]);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += (float)e[i];
        }
      }
#pragma unroll
      for (int u = 0; u < kGrUnroll; ++u) cur[u] = nxt[u];
    }
  }
  // reduce over the threads of each column chunk, in thread order
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) red[threadIdx.x * 8 + i] = acc[i];
  __syncthreads();
  for (int e = threadIdx.x; e < CPR * 8; e += kGrThreads) {
    const int cc = e / 8, i = e % 8;
    float s = 0.f;
    for (int t = cc; t < kGrThreads; t += CPR) s += red[t * 8 + i];
    if (cc * 8 + i < D) out[(int64_t)h * D + cc * 8 + i] = s;
  }
}

constexpr int kSrThreads = 256;
constexpr int kSrLoads = 8;         // 16-byte loads per thread in flight

template <bool NT>
__global__ __launch_bounds__(kSrThreads) void stream_read_kernel(const u32x4* src, int64_t vec_per_wg, float* out) {
  const u32x4* p = src + (int64_t)blockIdx.x * vec_per_wg;
  uint32_t acc = 0;
  for (int64_t base = 0; base < vec_per_wg; base += (int64_t)kSrThreads * kSrLoads) {
    u32x4 r[kSrLoads];
#pragma unroll
    for (int i = 0; i < kSrLoads; ++i) {
      const int64_t e = base + threadIdx.x + (int64_t)i * kSrThreads;
      const u32x4* a = p + (e < vec_per_wg ? e : vec_per_wg - 1);
      r[i] = NT ? ld16_nt(a) : ld16(a);
    }
#pragma unroll
    for (int i = 0; i < kSrLoads; ++i) acc ^= r[i][0] ^ r[i][1] ^ r[i][2] ^ r[i][3];
  }
  out[(int64_t)blockIdx.x * kSrThreads + threadIdx.x] = (float)acc;
}

__global__ __launch_bounds__(kSrThreads) void empty_kernel() {}

constexpr int kPsThreads = 256;
constexpr int kPsRowsPerThread = 4;

template <int BITS, int D, int STAGE>
__global__ __launch_bounds__(kPsThreads) void packed_stage_kernel(
    const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint8_t* kp, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    const uint16_t* sc, const uint16_t* zr, int64_t m_sb, int64_t m_sh, int64_t m_ss, float* out, int64_t o_sb,
    int64_t o_sh, int Hq, int G, int S) {
  constexpr int RB = D * BITS / 8;             // packed bytes per row
  constexpr int CPR = RB / 16;                 // 16-byte chunks per row
  constexpr int CODES = 128 / BITS;            // codes per chunk
  constexpr int EPB = 8 / BITS;                // codes per byte
  constexpr int R = kPsThreads / CPR;          // rows per pass
  __shared__ float qs[D];
  const int bh = blockIdx.y;
  const int b = bh / Hq, hq = bh - (bh / Hq) * Hq, hk = hq / G;
  if (STAGE == 3) {
    for (int i = threadIdx.x; i < D; i += kPsThreads) qs[i] = bf16_bits_to_f32(q[(int64_t)b * q_sb + (int64_t)hq * q_sh + i]);
    __syncthreads();
  }
  const int c = threadIdx.x % CPR, r0 = threadIdx.x / CPR;
  const uint8_t* kb = kp + (int64_t)b * k_sb + (int64_t)hk * k_sh + c * 16;
  const uint16_t* sb = sc + (int64_t)b * m_sb + (int64_t)hk * m_sh;
  const uint16_t* zb = zr + (int64_t)b * m_sb + (int64_t)hk * m_sh;
  const int t0 = blockIdx.x * (R * kPsRowsPerThread);
  u32x4 raw[kPsRowsPerThread];
  float sv[kPsRowsPerThread][CODES / 32], zv[kPsRowsPerThread][CODES / 32];
#pragma unroll
  for (int u = 0; u < kPsRowsPerThread; ++u) {
    const int t = min(t0 + r0 + u * R, S - 1);
    raw[u] = ld16(kb + (int64_t)t * k_ss);
    if (STAGE >= 2) {
#pragma unroll
      for (int g = 0; g < CODES / 32; ++g) {
        const int grp = c * (CODES / 32) + g;
        sv[u][g] = bf16_bits_to_f32(sb[(int64_t)t * m_ss + grp]);
        zv[u][g] = bf16_bits_to_f32(zb[(int64_t)t * m_ss + grp]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kPsRowsPerThread; ++u) {
    const uint8_t* by = reinterpret_cast<const uint8_t*>(&raw[u]);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CODES; ++j) {
      const uint32_t byte = by[j / EPB];
      float x;
      if (STAGE == 0) {
        x = (float)byte;
      } else {
        x = (float)((byte >> ((j % EPB) * BITS)) & ((1u << BITS) - 1u));
        if (STAGE >= 2) x = x * sv[u][j / 32] + zv[u][j / 32];
        if (STAGE == 3) x = x * qs[c * CODES + j];
      }
      s += x;
    }
#pragma unroll
    for (int m = 1; m < CPR; m <<= 1) s += __shfl_xor(s, m, 64);
    const int t = t0 + r0 + u * R;
    if (c == 0 && t < S) out[(int64_t)b * o_sb + (int64_t)hq * o_sh + t] = s;
  }
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_gather_reduce(const void* v, int64_t v_sh, int64_t v_ss, const void* idx, int64_t i_sh, void* out, int H,
                        int S, int K, int D, void* stream) {
  if (!v || !idx || !out || H <= 0 || S <= 0 || K <= 0 || D <= 0 || D % 8 != 0 || D > 256)
    return (int)hipErrorInvalidValue;
  const int cpr = D / 8;
  const dim3 g((unsigned)H), blk(kGrThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* vv = static_cast<const uint16_t*>(v);
  const int32_t* ii = static_cast<const int32_t*>(idx);
  float* o = static_cast<float*>(out);
#define GR(C) hipLaunchKernelGGL((gather_reduce_kernel<C>), g, blk, 0, st, vv, v_sh, v_ss, ii, i_sh, K, S, o, D)
  switch (cpr) {
    case 1: GR(1); break;
    case 2: GR(2); break;
    case 4: GR(4); break;
    case 8: GR(8); break;
    case 16: GR(16); break;
    case 32: GR(32); break;
    default: return (int)hipErrorNotSupported;      // D in {8, 16, 32, 64, 128, 256}
  }
#undef GR
  return (int)hipGetLastError();
}

int bytes_packed_stage(const void* q, int64_t q_sb, int64_t q_sh, const void* kp, int64_t k_sb, int64_t k_sh,
                       int64_t k_ss, const void* scale, const void* zero, int64_t m_sb, int64_t m_sh, int64_t m_ss,
                       void* out, int64_t o_sb, int64_t o_sh, int B, int Hq, int Hk, int S, int D, int bits,
                       int stage, void* stream) {
  if (!q || !kp || !scale || !zero || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || S <= 0)
    return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || (bits != 4 && bits != 2) || stage < 0 || stage > 3) return (int)hipErrorInvalidValue;
  const int cpr = D * bits / 8 / 16;
  const int rows_per_block = kPsThreads / cpr * kPsRowsPerThread;
  const long bhs = (long)B * Hq;
  if (bhs > 65535) return (int)hipErrorInvalidConfiguration;
  const dim3 g((unsigned)((S + rows_per_block - 1) / rows_per_block), (unsigned)bhs), blk(kPsThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* qq = static_cast<const uint16_t*>(q);
  const uint8_t* kk = static_cast<const uint8_t*>(kp);
  const uint16_t* ss = static_cast<const uint16_t*>(scale);
  const uint16_t* zz = static_cast<const uint16_t*>(zero);
  float* o = static_cast<float*>(out);
  const int G = Hq / Hk;
#define PS(BB, DD, ST) \
  hipLaunchKernelGGL((packed_stage_kernel<BB, DD, ST>), g, blk, 0, st, qq, q_sb, q_sh, kk, k_sb, k_sh, k_ss, ss, \
                     zz, m_sb, m_sh, m_ss, o, o_sb, o_sh, Hq, G, S)
#define PS_STAGES(BB, DD)            \
  switch (stage) {                   \
    case 0: PS(BB, DD, 0); break;    \
    case 1: PS(BB, DD, 1); break;    \
    case 2: PS(BB, DD, 2); break;    \
    default: PS(BB, DD, 3); break;   \
  }
  if (bits == 4 && D == 128) {
    PS_STAGES(4, 128)
  } else if (bits == 4) {
    PS_STAGES(4, 64)
  } else if (D == 128) {
    PS_STAGES(2, 128)
  } else {
    PS_STAGES(2, 64)
  }
#undef PS_STAGES
#undef PS
  return (int)hipGetLastError();
}


// Floor probes (see stream_read_kernel): `wgs` workgroups of 256 threads read
// bytes / wgs each from src (bytes a multiple of 16 * wgs; src 16-byte
// aligned); out holds wgs * 256 floats.  nontemporal != 0 issues the loads
// with the non-temporal hint, as the decode kernels stream K/V rows.
int bytes_stream_read(const void* src, int64_t bytes, int wgs, int nontemporal, void* out, void* stream) {
  if (!src || !out || wgs <= 0 || bytes <= 0 || bytes % (16LL * wgs) != 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(nontemporal ? stream_read_kernel<true> : stream_read_kernel<false>, dim3((unsigned)wgs),
                     dim3(kSrThreads), 0, static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     bytes / 16 / wgs, static_cast<float*>(out));
  return (int)hipGetLastError();
}

int bytes_empty_launch(int wgs, void* stream) {
  if (wgs <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(empty_kernel, dim3((unsigned)wgs), dim3(kSrThreads), 0, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

}  // extern "C"
