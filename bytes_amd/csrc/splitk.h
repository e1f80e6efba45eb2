// Split-K flash-decode epilogue shared by the dense, KIVI, PQ and gather kernels.
//
// A "unit" is one (b, kv-head, head-block) triple: up to 16 query heads of one
// GQA group that read the same K/V rows.  The token axis of a unit is cut into
// `nsplit` chunks, one workgroup each.  Every workgroup merges its waves'
// online-softmax states in LDS and then either writes the final output
// (nsplit == 1) or writes an fp32 partial (m, l, acc[D]) per head to the
// workspace, which splitk_combine_kernel (a second launch) merges in split
// order.  (A merge inside the same kernel - partials written through to
// memory, an arrival counter, the last workgroup merging - was measured
// slower on MI355X for every configuration: one workgroup reading all
// partials is bound by its own outstanding misses.)
#pragma once
#include "common.h"

namespace bytes_amd {

enum OutDtype : int { kOutBF16 = 0, kOutF16 = 1, kOutF32 = 2 };

struct SplitKOut {
  void* out;            // [B, Hq, D] with element strides o_sb, o_sh (d stride 1)
  int out_dtype;        // OutDtype
  int64_t o_sb, o_sh;
  float* part_acc;      // [units][16][nsplit][D]: a head's splits are contiguous
  float* part_ml;       // [units][16][nsplit][2]
  int nsplit;
  int Hk, HB, G;        // unit u -> b = u / (Hk*HB), hk, hb; query head = hk*G + hb*hbs + h
  int hbs = 16;         // query heads per head block
  int nwg = 0;          // workgroups of the split grid (units * nsplit)
  FastDiv dsplit, dunit, dhb;   // division by nsplit, Hk * HB and HB (set by splitk_carve)
};

constexpr long kMaxUnits = 65535;         // grid.y limit

// Workspace layout: part_ml, then part_acc.
inline size_t splitk_workspace_bytes(long units, long nsplit, int D) {
  if (nsplit <= 1) return 256;
  size_t ml = ((size_t)units * nsplit * 16 * 2 * 4 + 255) / 256 * 256;
  size_t acc = (size_t)units * nsplit * 16 * D * 4;
  return ml + acc;
}

inline void splitk_carve(void* ws, long units, long nsplit, SplitKOut& o) {
  char* p = static_cast<char*>(ws);
  size_t ml = ((size_t)units * nsplit * 16 * 2 * 4 + 255) / 256 * 256;
  o.part_ml = reinterpret_cast<float*>(p);
  o.part_acc = reinterpret_cast<float*>(p + ml);
  o.nsplit = (int)nsplit;
  o.nwg = (int)(units * nsplit);
  o.dsplit = make_fastdiv((uint32_t)nsplit);
  o.dunit = make_fastdiv((uint32_t)(o.Hk * o.HB));
  o.dhb = make_fastdiv((uint32_t)o.HB);
}

// Workgroups of a 1-D grid are dealt round-robin over the XCDs (8 on MI355X),
// each with its own L2.  Map hardware workgroup L to a (unit, split) pair so
// that every XCD receives a run of consecutive splits of one unit: neighbouring
// splits share cache lines of per-channel rows and metadata, which are then
// fetched into one L2 instead of several.  A bijection for any grid size.
constexpr int kXcds = 8;
__device__ __forceinline__ void xcd_unit_split(int nsplit, int N, int& unit, int& split) {
  const int L = blockIdx.x;
  const int x = L % kXcds, k = L / kXcds;
  const int q = N / kXcds, r = N % kXcds;
  const int idx = x * q + min(x, r) + k;
  unit = idx / nsplit;
  split = idx - unit * nsplit;
}

// The same mapping with the divisions set up on the host, and the unit's
// (b, hk, hb): unit = (b * Hk + hk) * HB + hb.
struct UnitLoc {
  int unit, split, b, hk, hb;
};
__device__ __forceinline__ UnitLoc splitk_locate(const SplitKOut& o) {
  const int L = blockIdx.x;
  const int x = L % kXcds, k = L / kXcds;
  const int q = o.nwg / kXcds, r = o.nwg % kXcds;
  const int idx = x * q + min(x, r) + k;
  UnitLoc u;
  u.unit = fast_div(idx, o.dsplit);
  u.split = idx - u.unit * o.nsplit;
  u.b = fast_div(u.unit, o.dunit);
  const int rem = u.unit - u.b * (int)o.dunit.d;
  u.hk = fast_div(rem, o.dhb);
  u.hb = rem - u.hk * (int)o.dhb.d;
  return u;
}


// Raw buffer resource over [base, base + bytes) (out-of-range lanes read 0 and
// drop stores).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same over a base and size the caller knows to be wave-uniform, built
// from their first lane's values so that the resource sits in scalar
// registers (an LDS-DMA request in inline assembly takes it there).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_uniform(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p), hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return buf_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}

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

// Floats per (wave, head) row of the epilogue's accumulator copy: D plus four
// pad floats, so the 16-byte writes of lanes with consecutive heads (row
// pitch = 4 banks mod 64) and the merge's reads at consecutive d fall in
// distinct LDS banks.
template <int D>
constexpr int acc_pitch() { return D + 4; }

// LDS floats needed by splitk_epilogue (the wave merge).
template <int D, int NW>
constexpr int splitk_smem_floats() {
  return NW * 16 * 2 + NW * 16 * acc_pitch<D>();
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
//
// Every wave copies its state to LDS (acc as 16-byte runs of four consecutive
// d), then each thread merges four consecutive d of one head over the waves,
// computing that head's wave factors itself (no third barrier), in wave order.
// smem holds the maxima, denominators and the accumulator rows of every wave,
// splitk_smem_floats<D, NW>() floats; with smem_hi set, the rows of waves
// NW/2.. go there instead (NW/2 * 16 * acc_pitch<D>() floats each side), for
// kernels whose LDS is two separate arrays.
template <int D, int NW>
__device__ void splitk_epilogue(float m_run, float l_run, f32x4 (&acc)[D / 16], float* smem,
                                const SplitKOut& o, int unit, int split, int b, int hq0, int nh,
                                int dmap = kDmapDense, float* smem_hi = nullptr) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  constexpr int NT = NW * 64;
  constexpr int P = acc_pitch<D>();
  constexpr int D4 = D / 4;
  l_run = col_sum4(l_run);
  float* wm = smem;
  float* wl = wm + NW * 16;
  float* wacc = wl + NW * 16;
  // accumulator rows of wave ww
  auto wrow = [&](int ww) { return smem_hi && ww >= NW / 2 ? smem_hi + (ww - NW / 2) * 16 * P : wacc + ww * 16 * P; };
  __syncthreads();
  if (lg == 0) {
    wm[w * 16 + l16] = m_run;
    wl[w * 16 + l16] = l_run;
  }
  // rows of head columns past nh are never read: not written
  f32x4* row = reinterpret_cast<f32x4*>(wrow(w) + l16 * P);
  if (l16 < nh) {
    if (dmap == kDmapKivi2) {
      // acc[2k][i], acc[2k+1][i] hold d = 32k + 8lg + 2i + {0, 1}
#pragma unroll
      for (int k = 0; k < D / 32; ++k) {
        row[8 * k + 2 * lg] = f32x4{acc[2 * k][0], acc[2 * k + 1][0], acc[2 * k][1], acc[2 * k + 1][1]};
        row[8 * k + 2 * lg + 1] = f32x4{acc[2 * k][2], acc[2 * k + 1][2], acc[2 * k][3], acc[2 * k + 1][3]};
      }
    } else {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) row[4 * db + lg] = acc[db];
    }
  }
  __syncthreads();

  for (int e = threadIdx.x; e < nh * D4; e += NT) {
    const int h = e / D4, d4 = e - h * D4;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, wm[ww * 16 + h]);
    const float Ms = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = fast_exp2(wm[ww * 16 + h] - Ms);
      L += f * wl[ww * 16 + h];
      A += f * reinterpret_cast<const f32x4*>(wrow(ww) + h * P)[d4];
    }
    if (o.nsplit <= 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) store_out(o, b, hq0 + h, 4 * d4 + j, A[j] / L);
    } else {
      const size_t r = ((size_t)unit * 16 + h) * o.nsplit + split;
      reinterpret_cast<f32x4*>(o.part_acc + r * D)[d4] = A;
      if (d4 == 0) {
        o.part_ml[r * 2 + 0] = M;
        o.part_ml[r * 2 + 1] = L;
      }
    }
  }
}

// Launch the partial merge (no-op for nsplit <= 1).  units = B*Hk*HB.
int splitk_combine(const SplitKOut& o, long units, int D, hipStream_t stream);

}  // namespace bytes_amd
