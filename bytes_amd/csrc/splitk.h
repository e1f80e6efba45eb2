// Split-K flash-decode epilogue shared by the dense, KIVI, PQ and gather kernels.
//
// A "unit" is one (b, kv-head, head-block) triple: up to 16 query heads of one
// GQA group that read the same K/V rows.  The token axis of a unit is cut into
// `nsplit` chunks, one workgroup each.  Every workgroup merges its waves'
// online-softmax states in LDS and then either writes the final output
// (nsplit == 1) or writes an fp32 partial (m, l, acc[D]) per head to the
// workspace.
//
// Merging the partials (nsplit <= kFusedSplitMax) happens in the same kernel:
// each workgroup writes its partial with device-coherent stores (cache policy
// sc1, the bits the compiler emits for agent-scope atomic stores: written
// through the per-XCD L2), waits for them to complete, and bumps a per-unit
// arrival counter with a relaxed agent-scope atomic.  The workgroup that
// arrives last reads every partial back with device-coherent loads and merges
// them in split order, so results are deterministic and no release/acquire
// fence (an L2 writeback + invalidate on gfx950) is ever executed.  The last
// workgroup also resets the counter, so counters are zero between calls.
// Larger split counts fall back to a second kernel (splitk_combine).
#pragma once
#include "common.h"

namespace bytes_amd {

enum OutDtype : int { kOutBF16 = 0, kOutF16 = 1, kOutF32 = 2 };

struct SplitKOut {
  void* out;            // [B, Hq, D] with element strides o_sb, o_sh (d stride 1)
  int out_dtype;        // OutDtype
  int64_t o_sb, o_sh;
  float* part_acc;      // [units][nsplit][16][D]
  float* part_ml;       // [units][nsplit][16][2]
  unsigned* counter;    // [kMaxUnits] arrival counters, zero between calls
  int nsplit;
  int fused;            // 1: the last-arriving workgroup of a unit merges
  int Hk, HB, G;        // unit u -> b = u / (Hk*HB), hk, hb; query head = hk*G + hb*hbs + h
  int hbs = 16;         // query heads per head block
};

constexpr int kFusedSplitMax = 256;       // largest split count merged in-kernel
constexpr long kMaxUnits = 65535;         // grid.y limit
constexpr size_t kCounterBytes = 65536 * 4;

// Workspace layout: counters (fixed size, so every call finds its counters in
// the zeroed region whatever an earlier call wrote elsewhere), part_ml, part_acc.
inline size_t splitk_workspace_bytes(long units, long nsplit, int D) {
  if (nsplit <= 1) return 256;
  size_t ml = ((size_t)units * nsplit * 16 * 2 * 4 + 255) / 256 * 256;
  size_t acc = (size_t)units * nsplit * 16 * D * 4;
  return kCounterBytes + ml + acc;
}

// allow_fused = 0 keeps the separate merge kernel even for small split counts
// (the dense kernel: its workgroups then exit right after their partial stores).
inline void splitk_carve(void* ws, long units, long nsplit, SplitKOut& o, bool allow_fused = true) {
  char* p = static_cast<char*>(ws);
  size_t ml = ((size_t)units * nsplit * 16 * 2 * 4 + 255) / 256 * 256;
  o.counter = reinterpret_cast<unsigned*>(p);
  o.part_ml = reinterpret_cast<float*>(p + kCounterBytes);
  o.part_acc = reinterpret_cast<float*>(p + kCounterBytes + ml);
  o.nsplit = (int)nsplit;
  o.fused = allow_fused && nsplit > 1 && nsplit <= kFusedSplitMax;
}

// Workgroups of a 1-D grid are dealt round-robin over the XCDs (8 on MI355X),
// each with its own L2.  Map hardware workgroup L to a (unit, split) pair so
// that every XCD receives a run of consecutive splits of one unit: neighbouring
// splits share cache lines of per-channel rows and metadata, which are then
// fetched into one L2 instead of several.  A bijection for any grid size.
constexpr int kXcds = 8;
__device__ __forceinline__ void xcd_unit_split(int nsplit, int& unit, int& split) {
  const int L = blockIdx.x, N = gridDim.x;
  const int x = L % kXcds, k = L / kXcds;
  const int q = N / kXcds, r = N % kXcds;
  const int idx = x * q + min(x, r) + k;
  unit = idx / nsplit;
  split = idx - unit * nsplit;
}

// Raw buffer resource over [base, base + bytes) (out-of-range lanes read 0 and
// drop stores).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr int kCoherent = 16;   // cache policy sc1: device-coherent access

__device__ __forceinline__ void store_out(const SplitKOut& o, int b, int hq, int d, float v) {
  int64_t off = (int64_t)b * o.o_sb + (int64_t)hq * o.o_sh + d;
  if (o.out_dtype == kOutBF16) {
    reinterpret_cast<uint16_t*>(o.out)[off] = f32_to_bf16_bits(v);
  } else if (o.out_dtype == kOutF16) {
    reinterpret_cast<_Float16*>(o.out)[off] = (_Float16)v;
  } else {
    reinterpret_cast<float*>(o.out)[off] = v;
  }
}

// LDS floats needed by splitk_epilogue (wave merge, then the in-kernel split merge).
template <int D, int NW>
constexpr int splitk_smem_floats() {
  constexpr int wave = NW * 16 * 2 + NW * D * 16 + NW * 16 + 16 + 4;
  constexpr int merge = kFusedSplitMax * 16 + 16 + 16;
  return wave > merge ? wave : merge;
}

// Head-dim position of accumulator element acc[db][i] held by lane group lg.
//   kDmapDense: d = db*16 + lg*4 + i           (dense, KIVI 4-bit, PQ, gather)
//   kDmapKivi2: d = 32*(db/2) + 8*lg + 2*i + db%2  (KIVI 2-bit value layout)
enum : int { kDmapDense = 0, kDmapKivi2 = 1 };
__device__ __forceinline__ int acc_d(int dmap, int db, int lg, int i) {
  return dmap == kDmapKivi2 ? 32 * (db >> 1) + 8 * lg + 2 * i + (db & 1) : db * 16 + lg * 4 + i;
}

// m_run: running max (log2 domain) of this lane's head l%16, identical across
// the four lanes l%16 + 16*j; l_run: this lane's partial denominator;
// acc[db][i]: O^T[d = acc_d(dmap, db, l/16, i)][h = l%16].
// All threads of the workgroup must call this (it contains barriers).
template <int D, int NW>
__device__ void splitk_epilogue(float m_run, float l_run, f32x4 (&acc)[D / 16], float* smem,
                                const SplitKOut& o, int unit, int split, int b, int hq0, int nh,
                                int dmap = kDmapDense) {
  static_assert(NW == 4, "the split merge maps 16 threads to each of 16 heads");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  constexpr int NT = NW * 64;
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);
  float* wm = smem;
  float* wl = wm + NW * 16;
  float* wacc = wl + NW * 16;
  __syncthreads();
  if (lg == 0) {
    wm[w * 16 + l16] = m_run;
    wl[w * 16 + l16] = l_run;
  }
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) wacc[(w * D + acc_d(dmap, db, lg, i)) * 16 + l16] = acc[db][i];
  __syncthreads();

  // per-head merge factors of the waves, computed once
  float* wf = wacc + NW * D * 16;   // [NW][16] factors, then [16] L
  if (threadIdx.x < 16) {
    const int h = threadIdx.x;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, wm[ww * 16 + h]);
    const float Ms = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = fast_exp2(wm[ww * 16 + h] - Ms);
      wf[ww * 16 + h] = f;
      L += f * wl[ww * 16 + h];
    }
    wf[NW * 16 + h] = L;
    wm[h] = M;   // wave 0's slot is free now: holds the merged max
  }
  __syncthreads();
  if (o.nsplit <= 1) {
    for (int e = threadIdx.x; e < nh * D; e += NT) {
      const int h = e / D, d = e - h * D;
      float A = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) A += wf[ww * 16 + h] * wacc[(ww * D + d) * 16 + h];
      store_out(o, b, hq0 + h, d, A / wf[NW * 16 + h]);
    }
    return;
  }
  const size_t row0 = ((size_t)unit * o.nsplit + split) * 16;
  if (!o.fused) {
    for (int e = threadIdx.x; e < nh * D; e += NT) {
      const int h = e / D, d = e - h * D;
      float A = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) A += wf[ww * 16 + h] * wacc[(ww * D + d) * 16 + h];
      o.part_acc[(row0 + h) * D + d] = A;
      if (d == 0) {
        o.part_ml[(row0 + h) * 2 + 0] = wm[h];
        o.part_ml[(row0 + h) * 2 + 1] = wf[NW * 16 + h];
      }
    }
    return;
  }

  // ---- fused: write this split's partial with device-coherent stores ----
  constexpr int D4 = D / 4;
  {
    const __amdgpu_buffer_rsrc_t racc = buf_rsrc(o.part_acc + row0 * D, 16 * D * 4);
    for (int e = threadIdx.x; e < nh * D4; e += NT) {
      const int h = e / D4, d0 = (e - h * D4) * 4;
      f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = wf[ww * 16 + h];
#pragma unroll
        for (int j = 0; j < 4; ++j) A[j] += f * wacc[(ww * D + d0 + j) * 16 + h];
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, A), racc, (h * D + d0) * 4, 0, kCoherent);
    }
    if (threadIdx.x < nh) {
      const int h = threadIdx.x;
      const __amdgpu_buffer_rsrc_t rml = buf_rsrc(o.part_ml + row0 * 2, 16 * 2 * 4);
      const u32x2 ml = {__float_as_uint(wm[h]), __float_as_uint(wf[NW * 16 + h])};
      __builtin_amdgcn_raw_buffer_store_b64(ml, rml, h * 8, 0, kCoherent);
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);          // this thread's partial stores have completed
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  int* flag = reinterpret_cast<int*>(wf + NW * 16 + 16);
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(o.counter + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == (unsigned)(o.nsplit - 1);
    if (last) __hip_atomic_store(o.counter + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // ---- last workgroup of the unit: merge every split in split order ----
  // Each thread owns float4 items e = tid, tid + NT, ... of the [nh][D] output
  // and sums its splits in order s = 0, 1, ...; the first PF splits of its
  // first item are requested before the (m, l) pass, so for nsplit <= PF the
  // whole merge is one memory round trip.  Loads past the partial buffer
  // (s >= nsplit) return zero through the buffer range check.
  const int ns = o.nsplit;
  const size_t urow = (size_t)unit * ns * 16;
  constexpr int PF = 32;
  const __amdgpu_buffer_rsrc_t racc = buf_rsrc(o.part_acc + urow * D, (uint32_t)((size_t)ns * 16 * D * 4));
  const int e0 = threadIdx.x;
  const int h0 = e0 / D4;
  const int off00 = (h0 * D + (e0 - h0 * D4) * 4) * 4;
  u32x4 v[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(racc, off00 + k * 16 * D * 4, 0, kCoherent);

  float* fwt = smem;                        // [ns][16] split weights
  float* il = smem + kFusedSplitMax * 16;   // [16] 1 / total denominator
  {
    // 16 threads per head (consecutive lanes), each taking splits j, j+16, ...
    const int h = threadIdx.x >> 4, j = threadIdx.x & 15;
    constexpr int PER = kFusedSplitMax / 16;
    const __amdgpu_buffer_rsrc_t rml = buf_rsrc(o.part_ml + urow * 2, (uint32_t)(ns * 16 * 2 * 4));
    u32x2 ml[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int s = j + 16 * k;
      ml[k] = (s < ns && h < nh) ? __builtin_amdgcn_raw_buffer_load_b64(rml, (s * 16 + h) * 8, 0, kCoherent)
                                 : u32x2{__float_as_uint(kNegInf), 0u};
    }
    float M = kNegInf;
#pragma unroll
    for (int k = 0; k < PER; ++k) M = fmaxf(M, __uint_as_float(ml[k][0]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) M = fmaxf(M, shfl_xor_f(M, off));
    const float Ms = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int s = j + 16 * k;
      if (s < ns) {
        const float f = fast_exp2(__uint_as_float(ml[k][0]) - Ms);
        fwt[s * 16 + h] = f;
        L += f * __uint_as_float(ml[k][1]);
      }
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) L += shfl_xor_f(L, off);
    if (j == 0) il[h] = 1.f / L;
  }
  lds_barrier();
  for (int e = e0; e < nh * D4; e += NT) {
    const int h = e / D4, d0 = (e - h * D4) * 4;
    const int off0 = (h * D + d0) * 4;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += PF) {
      if (e != e0 || s0 != 0) {
#pragma unroll
        for (int k = 0; k < PF; ++k)
          v[k] = __builtin_amdgcn_raw_buffer_load_b128(racc, off0 + (s0 + k) * 16 * D * 4, 0, kCoherent);
      }
#pragma unroll
      for (int k = 0; k < PF; ++k) {
        if (s0 + k < ns) {
          const float f = fwt[(s0 + k) * 16 + h];
          const f32x4 x = __builtin_bit_cast(f32x4, v[k]);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) A[jj] += f * x[jj];
        }
      }
    }
    const float inv = il[h];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) store_out(o, b, hq0 + h, d0 + jj, A[jj] * inv);
  }
}

// Launch the partial merge when it is not fused (no-op otherwise).  units = B*Hk*HB.
int splitk_combine(const SplitKOut& o, long units, int D, hipStream_t stream);

}  // namespace bytes_amd
