// Shared device helpers for the bytes_amd gfx950 (CDNA4) kernels.
//
// Conventions used by every kernel in this directory:
//  * wave64; MFMA operand layouts are those of v_mfma_f32_16x16x32_{bf16,f16}:
//      A[m][k]: lane l holds m = l%16, k = (l/16)*8 + j   (j = 0..7)
//      B[k][n]: lane l holds n = l%16, k = (l/16)*8 + j
//      C[m][n]: lane l holds n = l%16, m = (l/16)*4 + i   (i = 0..3)
//  * softmax runs in the log2 domain: x = score * scale * log2(e), p = 2^(x - m).
//  * every entry point returns 0 or a hipError_t and never throws.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bytes_amd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16-byte global load (caller guarantees 16-byte alignment).
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// 16-byte global load with the non-temporal hint, for data streamed once in
// whole cache lines per instruction (consecutive lanes, consecutive 16-byte
// chunks): measured ~7.0 TB/s against ~6.1 for plain loads on MI355X.  (A
// pattern that reads half of each line per instruction refetches the other
// half and gets slower with it.)
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// 16-byte load issued by every lane (p must be readable for all of them),
// zeroed afterwards where !live.  A load under a lane mask makes the compiler
// merge its result with the masked-off value right after the load, which waits
// for every load issued before it; loading unconditionally keeps such loads in
// flight together.
__device__ __forceinline__ u32x4 ld16_live(const void* p, bool live) {
  const u32x4 v = ld16(p);
  return live ? v : u32x4{0, 0, 0, 0};
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Division by a run-time constant d >= 1, for numerators n in [0, 2^31):
// floor(n / d) = (mulhi(m, n) + n) >> l with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (the round-up method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994).
// The host sets it up once per launch; on the device a quotient costs two
// scalar instructions instead of a reciprocal-and-correct sequence.
struct FastDiv {
  uint32_t m = 1, l = 0, d = 1;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d < 1 ? 1 : d;
  uint32_t l = 0;
  while ((1ull << l) < f.d) ++l;
  f.l = l;
  f.m = (uint32_t)((((1ull << l) - f.d) << 32) / f.d + 1);
  return f;
}
__device__ __forceinline__ int fast_div(int n, const FastDiv& f) {
  return (int)((__umulhi(f.m, (uint32_t)n) + (uint32_t)n) >> f.l);
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Cache-policy operand of a buffer load with the non-temporal hint (nt), for
// the same streamed, whole-line reads as ld16_nt.
constexpr int kNonTemporal = 2;

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// Reductions over the four lanes l % 16 + 16 j (j = 0..3) of a wave, the lanes
// that hold one column of an MFMA output: gfx950 row swaps (v_permlane16_swap
// exchanges 16-lane rows 2i and 2i+1, v_permlane32_swap the two 32-lane
// halves; with both operands equal, each lane then holds its own value and its
// partner's) instead of LDS permutes.  Every lane receives the result, the
// same on all four lanes; the maximum is IEEE maximum (no NaN quieting).
__device__ __forceinline__ float col_max4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// Maximum (fmaxf) over all 64 lanes, every lane receiving it: rotations by
// 8, 4, 2, 1 within each row of 16 (every source lane is in the row), then
// the row and half swaps.  All 64 lanes must be active.
__device__ __forceinline__ float wave_max_f32(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x128, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x124, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x122, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x121, 0xF, 0xF, false)));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// Sum over all 64 lanes, every lane receiving the same value; the same
// rotations and swaps as wave_max_f32.  The rotations add in a different
// order on each lane, so the lanes' sums can differ in the last bits: the
// result is lane 0's sum, broadcast (bit-reproducible run to run).
__device__ __forceinline__ float wave_sum_f32(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x128, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x124, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x122, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x121, 0xF, 0xF, false));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
__device__ __forceinline__ float col_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 2^x on the hardware exp unit (v_exp_f32).  Used for softmax weights, whose
// arguments are <= 0: results below the normal range flush towards zero,
// which does not change a softmax numerator or denominator at fp32 precision.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- wave-wide reductions and scans on DPP (no LDS round trip) ----
// dpp_u32<CTRL, ROWS>: lane i reads the lane CTRL names; lanes whose source
// lies outside their row of 16, or whose row is not in ROWS, read 0.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xF, true);
}

// Inclusive prefix sum over the 64 lanes: shifts of 1, 2, 4, 8 within each
// row of 16, then each row adds the totals of the rows before it (row
// broadcasts of lanes 15 and 31).
__device__ __forceinline__ uint32_t wave_prefix_sum(uint32_t x) {
  x += dpp_u32<0x111>(x);         // row_shr:1
  x += dpp_u32<0x112>(x);         // row_shr:2
  x += dpp_u32<0x114>(x);         // row_shr:4
  x += dpp_u32<0x118>(x);         // row_shr:8
  x += dpp_u32<0x142, 0xA>(x);    // row_bcast:15 into rows 1 and 3
  x += dpp_u32<0x143, 0xC>(x);    // row_bcast:31 into rows 2 and 3
  return x;
}

// Wave-scope ordering point for wave-private LDS buffers: keeps the compiler
// from moving LDS accesses across it and orders them at wavefront scope.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Monotone 32-bit ranking key of an fp32 score: larger score -> larger key;
// every NaN -> 0xFFFFFFFF (above +inf), -0 -> the key of +0.
__device__ __forceinline__ uint32_t score_order_key(float x) {
  if (x != x) return 0xFFFFFFFFu;
  uint32_t u = __float_as_uint(x);
  if (x == 0.f) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Workgroup barrier that orders LDS only: outstanding global loads stay in
// flight across it (a plain __syncthreads also waits for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One 16-byte-per-lane LDS-DMA request: lane l's 16 bytes at byte voff of the
// buffer land at lds + 16 l (NT: with the non-temporal hint, for bytes read
// once in whole cache lines).  Issued from inline assembly so
// that the compiler does not track it: the compiler cannot tell LDS-DMA
// destinations apart where a read's offset varies per lane, and would make
// every LDS read wait for every such load in flight.  The caller waits for
// these requests itself (vmcnt) before the LDS they fill is read.  lds is
// wave-uniform (its first lane's value is used) and goes to M0; one wait state
// before the load uses it.  r must be wave-uniform too (scalar registers).
template <bool NT>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, const char* lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds);
  if (NT)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(m0), "v"(voff), "s"(r)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Kernel families of the timing hook (bytes_set_kernel_events).
enum ProfFamily : int { kProfNone = 0, kProfDense = 1, kProfKivi = 2, kProfPq = 3, kProfGather = 4,
                        kProfScore = 5, kProfQuest = 6, kProfTopk = 7 };
constexpr int kProfFamilies = 7;
void prof_begin(int family, hipStream_t st);
void prof_end(int family, hipStream_t st);
bool prof_events(int family, hipEvent_t* start, hipEvent_t* stop);

// Launch a family's main kernel.  While the timing hook is set for the
// family, the launch carries the hook's event pair, which the runtime stamps
// with the dispatch's own start and end (the kernel's execution time, as a
// profiler measures it).
#define BYTES_LAUNCH(FAM, K, G, B, SH, ST, ...)                                  \
  do {                                                                         \
    hipEvent_t bytes_e0_, bytes_e1_;                                           \
    if (prof_events(FAM, &bytes_e0_, &bytes_e1_))                              \
      hipExtLaunchKernelGGL(K, G, B, SH, ST, bytes_e0_, bytes_e1_, 0, __VA_ARGS__); \
    else                                                                       \
      hipLaunchKernelGGL(K, G, B, SH, ST, __VA_ARGS__);                        \
  } while (0)

// Touch every 8-byte word of a kernel's argument block at entry: the scalar
// loads of the whole block are then issued together, one scalar-cache round
// trip, instead of in batches at each first use (each a round trip of its
// own before the first memory request can go out).  A macro, expanded in the
// kernel body: reading the block through a helper's reference parameter makes
// the compiler address every pointer the block holds as a flat pointer.
#define PREFETCH_ARGS(args)                                                          \
  do {                                                                               \
    static_assert(sizeof(args) % 8 == 0, "argument block in 8-byte words");          \
    constexpr int pf_n = (int)(sizeof(args) / 8);                                    \
    u32x2 pf_v[pf_n];                                                                \
    _Pragma("unroll") for (int pf_i = 0; pf_i < pf_n; ++pf_i)                        \
      pf_v[pf_i] = reinterpret_cast<const u32x2*>(&(args))[pf_i];                    \
    _Pragma("unroll") for (int pf_i = 0; pf_i < pf_n; ++pf_i)                        \
      asm volatile("" : : "s"(pf_v[pf_i]));                                          \
  } while (0)

}  // namespace bytes_amd
