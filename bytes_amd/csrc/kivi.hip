// KIVI-style quantized-KV decode attention, plus the KIVI pack / dequant helpers.
//
// Replaces benchmarks/kivi_latency.py:59-90 (`kivi_decode_attn`, whose device
// work is KIVI's external `cuda_bmm_fA_qB_outer` GEMV twice plus a residual
// matmul, softmax and cat) with one split-K flash-decode kernel, and the
// external `triton_quantize_and_pack_along_last_dim` (kivi_latency.py:123,127)
// plus the in-repo inverse `unpack_tensor_last_dim`/`dequant_k`/`dequant_v`
// (kivi_latency.py:26-57) with pack/dequant kernels.
//
// Cache layout (the reference's): codes packed 32/bits per int32 along the
// last dim, element i of word w at bits [i*bits, (i+1)*bits).
//   keys   Kq [B,Hk,D,Sq*bits/32], K_scale/K_mn fp16 [B,Hk,D,Sq/32]  (per channel,
//          groups of 32 tokens)
//   values Vq [B,Hk,Sq,D*bits/32], V_scale/V_mn fp16 [B,Hk,Sq,D/32]  (per token,
//          groups of 32 channels)
//   residual K_res/V_res bf16 [B,Hk,R,D]
//
// Decode data path, per wave and 64-token tile:
//  * packed key and value words go HBM -> LDS untouched (buffer loads with the
//    LDS bit, issued from inline assembly with explicit vmcnt waits); key and
//    value scales/zeros go through VGPRs into transposed LDS layouts;
//  * ds_read_b64_tr_b4 transposes the packed words at 4-bit granularity, which
//    turns "16 tokens of one channel" (keys) / "16 channels of one token"
//    (values) into the per-lane K-contiguous layout MFMA operands need;
//  * two masks split each nibble into fp4 (2-bit codes, value c/2) or fp8
//    (4-bit codes, value c*2^-9) operands that v_cvt_scalef32_pk_f16_{fp4,fp8}
//    turn into exact fp16 codes, which enter the MFMAs unscaled: key scales
//    multiply Q per 32-token group, value scales multiply P per 32-channel
//    group, and both zero terms are MFMA chains of their own;
//  * S^T = K_dq Q^T and O^T += V_dq^T P^T run on v_mfma_f32_16x16x32_f16 with
//    fp32 accumulation and an fp32 online softmax (kivi_tile_at).
// Three kernels share that tile: the two-half kernel (a workgroup stages its
// chunk in two halves, one tile per wave each), the pipelined kernel for long
// caches (runs of 256-token granules through a two-stage LDS ring) and the
// streaming kernel for caches with an odd number of 32-token key groups
// (which has a tile of its own, 32-token granular).  The bf16 residual window
// runs with the dense tile loop, on splits of its own or in pieces on the last
// splits after their quantized tiles.
#include "dense_tile.h"

namespace bytes_amd {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef int v2i_vs __attribute__((__vector_size__(2 * sizeof(int))));
typedef __attribute__((address_space(3))) v2i_vs* tr_ptr_t;

// ============================================================================
// pack / dequant along the last dim
// ============================================================================
__device__ __forceinline__ float load_elem(const void* p, int dt, int64_t i) {
  if (dt == 0) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == 1) return (float)static_cast<const _Float16*>(p)[i];
  return static_cast<const float*>(p)[i];
}

// One thread per (row, group).  Arithmetic follows src/quantization.py:432-442
// in fp32: scale = max(max-min, 1e-8)/(2^bits-1), code = clamp(rint((x-min)/scale)).
__global__ void kivi_pack_kernel(const void* x, int dt, int64_t rows, int T, int64_t x_rs, int gs, int bits,
                                 uint32_t* code, _Float16* scale, _Float16* mn) {
  const int ngr = T / gs;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * ngr) return;
  const int64_t row = gid / ngr;
  const int grp = (int)(gid - row * ngr);
  const int64_t base = row * x_rs + (int64_t)grp * gs;
  float lo = __builtin_inff(), hi = -__builtin_inff();
  for (int i = 0; i < gs; ++i) {
    const float v = load_elem(x, dt, base + i);
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
  const int levels = 1 << bits;
  const float s = fmaxf(hi - lo, 1e-8f) / (float)(levels - 1);
  const int fpi = 32 / bits;
  uint32_t* cw = code + row * (int64_t)(T / fpi) + (int64_t)grp * (gs / fpi);
  for (int w = 0; w < gs / fpi; ++w) {
    uint32_t word = 0;
    for (int i = 0; i < fpi; ++i) {
      const float v = load_elem(x, dt, base + w * fpi + i);
      float c = rintf((v - lo) / s);
      c = fminf(fmaxf(c, 0.f), (float)(levels - 1));
      word |= (uint32_t)c << (i * bits);
    }
    cw[w] = word;
  }
  scale[row * ngr + grp] = (_Float16)s;
  mn[row * ngr + grp] = (_Float16)lo;
}

// out[row, t] = code * scale + mn, in fp32 (fp16_math=0) or in the reference's
// fp16 arithmetic (fp16_math=1: product rounded to fp16, then sum rounded).
__global__ void kivi_dequant_kernel(const uint32_t* code, const _Float16* scale, const _Float16* mn, int64_t rows,
                                    int T, int gs, int bits, int fp16_math, void* out, int out_dt) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * T) return;
  const int64_t row = gid / T;
  const int t = (int)(gid - row * T);
  const int fpi = 32 / bits, ngr = T / gs;
  const uint32_t w = code[row * (T / fpi) + t / fpi];
  const uint32_t c = (w >> ((t % fpi) * bits)) & ((1u << bits) - 1u);
  const _Float16 s = scale[row * ngr + t / gs], m = mn[row * ngr + t / gs];
  float v;
  if (fp16_math) {
#pragma clang fp contract(off)
    const _Float16 p = (_Float16)c * s;   // rounded to fp16, then the sum rounded again
    v = (float)(_Float16)(p + m);
  } else {
    v = (float)c * (float)s + (float)m;
  }
  if (out_dt == kOutBF16)
    static_cast<uint16_t*>(out)[gid] = f32_to_bf16_bits(v);
  else if (out_dt == kOutF16)
    static_cast<_Float16*>(out)[gid] = (_Float16)v;
  else
    static_cast<float*>(out)[gid] = v;
}

// ============================================================================
// decode
// ============================================================================
struct KiviArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint32_t* kq;       // contiguous [B,Hk,D,Sq*BITS/32]
  const _Float16* ks;       // contiguous [B,Hk,D,Sq/32]
  const _Float16* km;
  const uint32_t* vq;       // contiguous [B,Hk,Sq,D*BITS/32]
  const _Float16* vs;       // contiguous [B,Hk,Sq,D/32]
  const _Float16* vm;
  const uint16_t* kr;       // residual [B,Hk,R,D] bf16
  const uint16_t* vr;
  int64_t kr_sb, kr_sh, kr_ss, vr_sb, vr_sh, vr_ss;
  int Hk, G, HB, Sq, R, chunk, nsq;
  int rsplit;               // > 0: the residual window has splits nsq .. nsq+rsplit-1 of its own (128 tokens each)
  int rchunk;               // rsplit == 0: residual tokens per piece (<= 128; pieces ride on the last splits)
  float scale_log2;
  SplitKOut o;
};

// Waves per workgroup (template NW): 4 (512-token chunks, two workgroups per CU) or 8
// (1024-token chunks, one per CU).  Chunk = waves * 128 tokens, staged in two
// halves of one 64-token tile per wave.
constexpr int kKiviTile = 64;
constexpr int kResidPerSplit = 128;  // residual tokens per split at most (one 32-token tile per wave)
constexpr int kKiviOnes = 128;       // LDS bytes of f16 ones after a wave's value scales/zeros (the softmax row sums)

template <int D, int BITS, int NW = 4>
struct KiviCfg {
  static constexpr int CHUNK = NW * 2 * kKiviTile;         // tokens per workgroup
  static constexpr int KK = D / 32;                        // MFMA k-steps over channels
  // Key codes are staged per half chunk ([half][channel][row]) so that the
  // first half's block, read by no wave once the second half is staged, can
  // hold the dense residual tiles of the first waves (RES_EARLY of them).  A
  // channel row of a half is NPC 16-byte pieces (piece p: the half's tokens
  // [p * 128 / BITS, (p + 1) * 128 / BITS)) in the slots kslot_swz<NPC> maps
  // them to, with no pad, so that a half arrives by LDS-DMA, 1 KB (KROWS_DMA
  // rows) per request.
  static constexpr int NPC = CHUNK * BITS / 256;           // key pieces per channel row of a half
  static constexpr int KROW = NPC * 16;
  static constexpr int KROWS_DMA = 1024 / KROW;
  static constexpr int KHALF = D * KROW;
  static constexpr int KDMA = KHALF / (NW * 1024);          // key LDS-DMA requests per wave per half
  static constexpr int KCBYTES = 2 * KHALF;                // staged key codes of one chunk
  static constexpr int RES_EARLY = KHALF / DenseCfg<D>::WAVE;
  static constexpr int KMG = CHUNK / 32;                   // key groups per chunk
  // staged key scales + zeros, one row of KMP fp16 per (scale|zero, group): the
  // 8-halfword pad puts the staging stores of a wave's eight groups in
  // distinct banks (4-bit caches on 4-wave workgroups go without it, to fit
  // two workgroups per CU)
  static constexpr int KMP = (BITS == 4 && NW == 4) ? D : D + 8;
  static constexpr int KMETA = 2 * KMG * KMP * 2;
  static constexpr int VROW = D * BITS / 8;                // LDS bytes of one token's value codes
  static constexpr int VBYTES = kKiviTile * VROW;
  static constexpr int VDMA = VBYTES / 1024;               // value LDS-DMA requests per wave per tile
  static constexpr int NGV = D / 32;                        // value groups per token
  static constexpr int VMBYTES = 2 * kKiviTile * NGV * 2;   // value scale + zero of one tile
  // per wave: the value codes of its two tiles (each half's arrive while the
  // other's tile may still be read), then one tile's value scales/zeros
  static constexpr int WAVE_BYTES = 2 * VBYTES + VMBYTES;
  // Q of the unit's 16 head columns as the fp16 B operand (scaled, k-slot
  // order within each 8-channel chunk), staged once per workgroup: row pitch
  // D*2 + 16 bytes so the 16 head rows a 16-lane group reads sit in distinct
  // banks, where that still fits two 4-wave workgroups per CU
  static constexpr int QBASE = KCBYTES + KMETA + NW * WAVE_BYTES;
  static constexpr int QP = (NW == 4 && QBASE + 16 * (D * 2 + 16) > 80 * 1024) ? D * 2 : D * 2 + 16;
  static constexpr int QOFF = QBASE;
  static constexpr int kQuant = QOFF + 16 * QP;
  static constexpr int kDense = DenseCfg<D>::kSmem;        // residual tiles of waves 0-3 (and their merge)
  static constexpr int kEpi = splitk_smem_floats<D, NW>() * 4;
  static constexpr int kSmem0 = kQuant > kDense ? kQuant : kDense;
  static constexpr int kSmem = kSmem0 > kEpi ? kSmem0 : kEpi;
  static_assert(KROWS_DMA * KROW == 1024 && KDMA * NW * 1024 == KHALF && VDMA * 1024 == VBYTES,
                "whole LDS-DMA requests");
  static_assert(NW == 8 ? kSmem <= 160 * 1024 : kSmem <= 80 * 1024, "workgroups per CU of the launch bounds");
};

// Position of the k-slot order inside an 8-channel block (4-bit keys interleave
// even/odd channels: slots hold channels 0,2,4,6,1,3,5,7).
template <int BITS>
__device__ __forceinline__ int kslot_pos(int ch) {
  if (BITS == 2) return ch;
  const int r = ch & 7;
  return (ch & ~7) | ((r & 1) ? 4 + (r >> 1) : (r >> 1));
}
template <int BITS>
__device__ __forceinline__ int kslot_ch(int jj) {  // channel offset held by k-slot jj
  return BITS == 2 ? jj : (jj < 4 ? 2 * jj : 2 * (jj - 4) + 1);
}

// Value-meta slot of tile token tau for (sm, g): [sm][g][sg][lg][jj] (fp16 index).
template <int D, int BITS>
__device__ __forceinline__ int vmeta_slot(int sm, int g, int tau) {
  constexpr int NGV = D / 32;
  const int sg = tau >> 5, r = tau & 31;
  int lg, jj;
  if (BITS == 2) {
    lg = r >> 3;
    jj = r & 7;
  } else {
    const int hf = r >> 4, r2 = r & 15;
    lg = r2 >> 2;
    jj = hf * 4 + (r2 & 3);
  }
  return (((sm * NGV + g) * 2 + sg) * 4 + lg) * 8 + jj;
}

__device__ __forceinline__ u32x2 tr4(const char* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr4_b64_v2i32((tr_ptr_t)p));
}

__device__ __forceinline__ h2 u2h(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// 8 fp4 nibbles (2-bit codes c -> value c/2) -> 8 fp16 c*scale + zero.
__device__ __forceinline__ f16x8 deq_fp4(uint32_t dw, u32x4 s, u32x4 z) {
  u32x4 r;
  r[0] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 0)), u2h(s[0]), u2h(z[0])));
  r[1] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 1)), u2h(s[1]), u2h(z[1])));
  r[2] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 2)), u2h(s[2]), u2h(z[2])));
  r[3] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 3)), u2h(s[3]), u2h(z[3])));
  return __builtin_bit_cast(f16x8, r);
}

// lo/hi: 4 bytes each holding a 4-bit code (fp8 e4m3 value c*2^-9).  Output
// k-slots: lo bytes 0,1 | lo bytes 2,3 | hi bytes 0,1 | hi bytes 2,3.
__device__ __forceinline__ f16x8 deq_fp8(uint32_t lo, uint32_t hi, u32x4 s, u32x4 z) {
  u32x4 r;
  r[0] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false)), u2h(s[0]), u2h(z[0])));
  r[1] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true)), u2h(s[1]), u2h(z[1])));
  r[2] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false)), u2h(s[2]), u2h(z[2])));
  r[3] = h2u(__builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true)), u2h(s[3]), u2h(z[3])));
  return __builtin_bit_cast(f16x8, r);
}

// 8 fp4 nibbles (2-bit codes c -> value c/2) -> the 8 codes as fp16 (exact).
__device__ __forceinline__ f16x8 codes_fp4(uint32_t dw) {
  const u32x4 r = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 0)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 1)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 2)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 3))};
  return __builtin_bit_cast(f16x8, r);
}

// lo/hi: 4 bytes each holding a 4-bit code (fp8 e4m3 value c*2^-9) -> the 8
// codes as fp16, k-slots in the order of deq_fp8.
__device__ __forceinline__ f16x8 codes_fp8(uint32_t lo, uint32_t hi) {
  const u32x4 r = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true))};
  return __builtin_bit_cast(f16x8, r);
}

// Elementwise fp16 product of an operand and 8 fp16 scales.
__device__ __forceinline__ f16x8 scale8(f16x8 x, u32x4 s) { return x * __builtin_bit_cast(f16x8, s); }

template <int D>
using VMetaReg = typename std::conditional<(D >= 128), u32x4, u32x2>::type;

// Online softmax of one 64-token tile with a lazy running maximum.
//
// On entry sc[u][i] holds s - m_run for its (token, head), where m_run is the
// head's frame (0 before the wave's first tile, when m_run = -inf): the
// zero-term chain of the scores starts from negm = -m_run.  The frame moves
// only when some score of the head's tile exceeds it - always on the first
// tile - and then to the tile maximum plus kKiviLazy (log2 units), so the
// tiles after it whose scores climb by up to kKiviLazy skip the rescale of the
// accumulators (and its exp).  Every probability p = exp2(s - m_run) is at
// most 1, so its fp16 products with the value scales are at most the scale
// itself and stay finite for every finite fp16 scale.  The softmax
// denominators are not summed here: the value zero-term MFMA has rows of ones
// (rows >= NGV of its A operand) and accumulates sum_t p[h][t] in zv row
// kKiviOnesRow, rescaled with the accumulators.  The accumulators, the
// denominator and m_run handed to the residual tiles and the split merge are
// all in the frame.  p receives exp2(s - m_run) in sc's order.
constexpr float kKiviLazy = 4.f;
constexpr int kKiviOnesRow = 12;     // zv row read back as the denominator (lanes 48-63, element 0)
template <int D>
__device__ __forceinline__ void kivi_softmax(f32x4 (&sc)[4], float& m_run, f32x4& negm, f32x4 (&acc)[D / 16],
                                             f32x4& zv, float (&p)[16]) {
  float mx = kNegInf;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = __builtin_elementwise_maximum(mx, sc[u][i]);
  mx = col_max4(mx);
  const bool first = m_run == kNegInf;            // the same on every lane of the wave
  if (__ballot(first || mx > 0.f) != 0) {
    const float m_new = first ? mx + kKiviLazy : (mx > 0.f ? m_run + mx + kKiviLazy : m_run);
    const float shift = first ? m_new : m_new - m_run;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[u][i] -= shift;
    if (__ballot(!first) != 0) {
      const float alpha = fast_exp2(m_run - m_new);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) acc[db] *= alpha;
      zv *= alpha;
    }
    m_run = m_new;
    negm = f32x4{-m_new, -m_new, -m_new, -m_new};
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) p[u * 4 + i] = fast_exp2(sc[u][i]);
}

// After a wave's last quantized tile: the value zero term added to the
// accumulators (acc[db][i] holds a channel of value group db / 2 in both
// layouts; group g's term is held by lane l16 of row group 0 at element g)
// and the lane's share of the denominator (the ones row, on lanes 48-63).
template <int D>
__device__ __forceinline__ void kivi_finish(int lane, const f32x4& zv, f32x4 (&acc)[D / 16], float& l_run) {
  const int l16 = lane & 15;
#pragma unroll
  for (int g = 0; g < D / 32; ++g) {
    const float zg = __shfl(zv[g], l16, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * g][i] += zg;
      acc[2 * g + 1][i] += zg;
    }
  }
  static_assert(kKiviOnesRow % 4 == 0, "the ones row is element 0 of its lane group");
  l_run = (lane >> 4) == kKiviOnesRow / 4 ? zv[0] : 0.f;
}

// Buffer resources over one unit's quantized cache.  A split without
// quantized tokens gets zero-sized resources: its requests are issued like
// any other (every wait counts the same requests on every path) and read
// zeros without touching memory.  Offsets are 32-bit (a unit's cache is far
// below 4 GiB), so every request is a buffer load with a per-lane offset
// computed once and a uniform offset in a scalar register.
struct KiviRsrc {
  __amdgpu_buffer_rsrc_t kq, ks, kz, vq;
  const char* vs;          // the unit's value scales and zeros (a readable dummy when
  const char* vz;          // the split has no quantized tokens)
};

// Value scales (lanes 0-31) / zeros (32-63) of tokens o + 2(l % 32), +1 of the
// tile at token o: contiguous in HBM.
template <int D>
__device__ __forceinline__ VMetaReg<D> kivi_load_vmeta(const KiviRsrc& rs, bool quant, int o, int lane) {
  const char* mb = lane < 32 ? rs.vs : rs.vz;
  return __builtin_nontemporal_load(
      reinterpret_cast<const VMetaReg<D>*>(mb + (quant ? (uint32_t)(o + 2 * (lane & 31)) * (D / 32) * 2 : 0u)));
}

// Write one tile's value scales/zeros to the wave's LDS buffer (vmeta_slot layout).
template <int D, int BITS>
__device__ __forceinline__ void kivi_stage_vmeta(int lane, const VMetaReg<D>& vm, char* vmeta_lds) {
  constexpr int NGV = D / 32;
  const _Float16* hv = reinterpret_cast<const _Float16*>(&vm);
  const int sm = lane >> 5, tau0 = 2 * (lane & 31);
  _Float16* dst = reinterpret_cast<_Float16*>(vmeta_lds);
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int g = 0; g < NGV; ++g) dst[vmeta_slot<D, BITS>(sm, g, tau0 + u)] = hv[u * NGV + g];
}

// Slot of 16-byte key piece p in a staged key channel row r of NPC pieces
// (rows 16 * NPC bytes apart): the 16 rows a transposed read touches (r =
// 16k .. 16k + 15) then sit in distinct banks of the 256-byte bank cycle, and
// the slot depends on r % 16 only.  An involution in p, so it also maps a
// slot to the piece it holds.
template <int NPC>
__device__ __forceinline__ int kslot_swz(int p, int r) {
  static_assert(NPC == 4 || NPC == 8 || NPC == 16, "64-, 128- or 256-byte rows");
  return NPC == 4 ? p ^ ((r >> 2) & 3) : NPC == 8 ? p ^ ((r >> 1) & 7) : p ^ (r & 15);
}

// One 64-token tile: scores from staged key codes, online softmax, value
// accumulation from staged value codes.
//
// Scales are folded into the other MFMA operand, so codes enter the MFMAs as
// exact fp16 integers:
//   keys   s[t][h] = sum_c (q[h][c] sc[c][g]) code[t][c] + sum_c q[h][c] zero[c][g]
//          (g = key group of t; the second sum is one MFMA chain on the zeros,
//          whose A rows are all equal, started from -m_run, and initialises
//          the score tile, so the scores come out shifted by the running
//          maximum; see kivi_softmax);
//   values o[c][h] += sum_t code[t][c] (p[h][t] vs[t][g]) + sum_t p[h][t] vm[t][g]
//          (g = value group of channel c; the second sum accumulates in zv,
//          rows = groups, and is added to acc once after the last tile; rows
//          of ones in the same MFMA sum p, the softmax denominator).
//
// Operands:
// kb[sg] is this lane's byte of key channel row l16 for the tile's tokens
// [32sg, 32sg + 32) (rows KPR bytes apart; 8 bytes for 2-bit caches, 16 - two
// 16-token blocks of 8 - for 4-bit), kms the staged key scales ([group][KMP]
// fp16, k-slot channel order) with the zeros kzo bytes on and grp0 the tile's
// first group there, vst / vml the tile's value codes and value scales/zeros
// (vmeta_slot layout).  The value zero-term MFMA's rows past the value groups
// are ones (the softmax denominators).
template <int D, int BITS, int KPR, int KMP>
__device__ __forceinline__ void kivi_tile_at(int lane, const f16x8 (&qh)[D / 32], const char* const (&kb)[2],
                                             const char* kms, int kzo, int grp0, const char* vst, const char* vml,
                                             float& m_run, f32x4& negm, f32x4 (&acc)[D / 16], f32x4& zv) {
  constexpr int KK = D / 32, NGV = D / 32, VROW = D * BITS / 8;
  const int l16 = lane & 15, lg = lane >> 4;

  // 2-bit: sc[sg*2 + p][i] is tile token 32sg + 8lg + 2i + p
  // 4-bit: sc[tb][i]       is tile token 16tb + 4lg + i
  f32x4 sc[4];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    const int grp = grp0 + sg;
    f16x8 qs[KK];
    f32x4 z = negm;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int off = (grp * KMP + lg * (D / 4) + kk * 8) * 2;
      const u32x4 ks = *reinterpret_cast<const u32x4*>(kms + off);
      const u32x4 kz = *reinterpret_cast<const u32x4*>(kms + kzo + off);
      qs[kk] = scale8(qh[kk], ks);
      z = mfma_f16(__builtin_bit_cast(f16x8, kz), qh[kk], z);
    }
    sc[sg * 2 + 0] = z;
    sc[sg * 2 + 1] = z;
#pragma unroll
    for (int bb = 0; bb < (BITS == 2 ? 1 : 2); ++bb)
#pragma unroll
      for (int rd = 0; rd < KK / 2; ++rd) {
        const u32x2 x = tr4(kb[sg] + (lg * (D / 4) + rd * 16) * KPR + bb * 8);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int kk = rd * 2 + half;
          if (BITS == 2) {
            const uint32_t e = x[half] & 0x33333333u, od = (x[half] >> 2) & 0x33333333u;
            sc[sg * 2 + 0] = mfma_f16(codes_fp4(e), qs[kk], sc[sg * 2 + 0]);
            sc[sg * 2 + 1] = mfma_f16(codes_fp4(od), qs[kk], sc[sg * 2 + 1]);
          } else {
            const uint32_t lo = x[half] & 0x0F0F0F0Fu, hi = (x[half] >> 4) & 0x0F0F0F0Fu;
            sc[sg * 2 + bb] = mfma_f16(codes_fp8(lo, hi), qs[kk], sc[sg * 2 + bb]);
          }
        }
      }
  }

  float p[16];
  kivi_softmax<D>(sc, m_run, negm, acc, zv, p);
  // P^T as the B operand, k-slot jj of sub-tile sg (the orders of kivi_tile)
  f16x8 pb[2];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      pb[sg][jj] = (_Float16)p[BITS == 2 ? (sg * 2 + (jj & 1)) * 4 + (jj >> 1) : (2 * sg + (jj >> 2)) * 4 + (jj & 3)];

  constexpr uint32_t kOnes = 0x3C003C00u;
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    f16x8 pg[NGV];
#pragma unroll
    for (int g = 0; g < NGV; ++g)
      pg[g] = scale8(pb[sg], *reinterpret_cast<const u32x4*>(vml + vmeta_slot<D, BITS>(0, g, sg * 32) * 2 + lg * 16));
    {
      u32x4 vz = *reinterpret_cast<const u32x4*>(vml + vmeta_slot<D, BITS>(1, min(l16, NGV - 1), sg * 32) * 2 + lg * 16);
      if (l16 >= NGV) vz = u32x4{kOnes, kOnes, kOnes, kOnes};
      zv = mfma_f16(__builtin_bit_cast(f16x8, vz), pb[sg], zv);
    }
    if (BITS == 2) {
#pragma unroll
      for (int rd = 0; rd < D / 64; ++rd) {
        const int r = l16 & 7, cbr = 2 * rd + (l16 >> 3);
        const int tok = 32 * sg + 8 * lg + r;
        const u32x2 x = tr4(vst + tok * VROW + cbr * 8);
        const int ca = 2 * rd, cbb = 2 * rd + 1;
        const uint32_t e0 = x[0] & 0x33333333u, e1 = x[1] & 0x33333333u;
        const uint32_t o0 = (x[0] >> 2) & 0x33333333u, o1 = (x[1] >> 2) & 0x33333333u;
        acc[ca * 2 + 0] = mfma_f16(codes_fp4(e0), pg[ca], acc[ca * 2 + 0]);
        acc[cbb * 2 + 0] = mfma_f16(codes_fp4(e1), pg[cbb], acc[cbb * 2 + 0]);
        acc[ca * 2 + 1] = mfma_f16(codes_fp4(o0), pg[ca], acc[ca * 2 + 1]);
        acc[cbb * 2 + 1] = mfma_f16(codes_fp4(o1), pg[cbb], acc[cbb * 2 + 1]);
      }
    } else {
#pragma unroll
      for (int rd = 0; rd < D / 32; ++rd) {
        const int r = l16 & 7, cbr = 2 * rd + (l16 >> 3);
        const int tok = (r & 1) ? 32 * sg + 16 + 4 * lg + (r >> 1) : 32 * sg + 4 * lg + (r >> 1);
        const u32x2 x = tr4(vst + tok * VROW + cbr * 8);
        const uint32_t lo0 = x[0] & 0x0F0F0F0Fu, hi0 = (x[0] >> 4) & 0x0F0F0F0Fu;
        const uint32_t lo1 = x[1] & 0x0F0F0F0Fu, hi1 = (x[1] >> 4) & 0x0F0F0F0Fu;
        acc[2 * rd] = mfma_f16(codes_fp8(lo0, hi0), pg[rd], acc[2 * rd]);
        acc[2 * rd + 1] = mfma_f16(codes_fp8(lo1, hi1), pg[rd], acc[2 * rd + 1]);
      }
    }
  }
}

// ============================================================================
// Streaming decode (caches with an odd number of key groups): phases of 512
// tokens, one 64-token tile per wave
// ============================================================================
// A workgroup of eight waves walks its split's quantized tokens in phases of
// 512 (one 64-token tile, two key groups, per wave per phase).  The requests
// of DEPTH phases are in flight at once, held in registers: every thread
// loads a slice of the phase's key codes and key scales/zeros (staged in a
// workgroup-shared LDS buffer) and every wave loads its own tile's value codes
// and value scales/zeros (a wave-private LDS buffer).  When phase p's
// registers have arrived and every wave is done with phase p-1, they are
// written to LDS, phase p + DEPTH is requested into the same registers, a
// barrier publishes the keys, and each wave computes its tile.  Splits are
// 32-token multiples, so a tile can end after its first key group (the
// second is then masked).  The bf16 residual window runs on splits of its
// own.  Caches whose Sq is a multiple of 64 use kivi_decode_kernel, which
// measured faster on them (the tiles' compute, not HBM, bounds both kernels
// at two waves per SIMD).
constexpr int kKsWaves = 8;
constexpr int kKsPhase = kKsWaves * 64;        // tokens per phase
constexpr int kKsGroups = kKsPhase / 32;       // key groups per phase

// The decode uses this kernel for caches with an odd number of 32-token key
// groups (Sq = 32 mod 64), whose key rows are only 8-byte aligned (2-bit) and
// whose rows of key scales/zeros start on odd halfwords: key codes are read
// in KPB-byte pieces (8 for 2-bit keys, 16 for 4-bit) and key scales/zeros
// one halfword at a time, and splits are 32-token multiples.
template <int D, int BITS, int KPB>
struct KsCfg {
  static constexpr int DEPTH = 2;                            // phases in flight
  static constexpr int NT = kKsWaves * 64;
  static constexpr int PPC = kKsPhase * BITS / 8 / KPB;      // key pieces per channel per phase
  static constexpr int KROW = kKsPhase * BITS / 8 + 16;      // LDS bytes per channel row (+16: bank spread)
  static constexpr int NKP = D * PPC;                        // key pieces per phase
  static constexpr int KP = (NKP + NT - 1) / NT;             // key pieces per thread per phase
  // threads past the phase's pieces load a valid piece again and store it
  // past the channel rows
  static constexpr int KBYTES = D * KROW + (KP * NT - NKP) * KPB;
  static constexpr int NKM = 2 * D * kKsGroups;             // key scale/zero halfwords per phase
  static constexpr int KMPT = (NKM + NT - 1) / NT;
  static constexpr int KMP = D + 8;                          // fp16 per staged (scale|zero, group) row
  static constexpr int KMBYTES = 2 * kKsGroups * KMP * 2;
  static constexpr int VROW = D * BITS / 8;                  // bytes of one token's value codes
  static constexpr int VBYTES = 64 * VROW;                   // value codes of one wave's tile
  static constexpr int VDMA = VBYTES / 1024;                 // 16-byte value pieces per lane
  static constexpr int NGV = D / 32;
  static constexpr int VMBYTES = 2 * 64 * NGV * 2;           // value scales + zeros of one tile
  static constexpr int WAVE = VBYTES + VMBYTES + kKiviOnes;
  static constexpr int kQuant = KBYTES + KMBYTES + kKsWaves * WAVE;
  static constexpr int kDense = 4 * DenseCfg<D>::WAVE;       // residual tiles of waves 0-3 (residual splits)
  static constexpr int kEpi = splitk_smem_floats<D, kKsWaves>() * 4;
  static constexpr int kSmem0 = kQuant > kDense ? kQuant : kDense;
  static constexpr int kSmem = kSmem0 > kEpi ? kSmem0 : kEpi;
  static_assert(kSmem <= 160 * 1024, "fits the LDS of one CU");
  static_assert(VBYTES >= 1024 && VBYTES % 1024 == 0, "whole 16-byte pieces per lane");
};

// One phase's requests of one thread.
template <int D, int BITS, int KPB>
struct KsRegs {
  using C = KsCfg<D, BITS, KPB>;
  using KPiece = typename std::conditional<KPB == 16, u32x4, u32x2>::type;
  KPiece k[C::KP];                             // key code pieces
  uint16_t km[C::KMPT];                        // key scales / zeros
  u32x4 v[C::VDMA];                            // this wave's value codes
  VMetaReg<D> vm;                              // value scales (lanes 0-31) or zeros (32-63) of two tokens
};

// One 64-token tile: scores from the staged key phase (kc: this tile's first
// byte of channel row 0, rows KROW bytes apart; kms: the scale row of its
// first key group, the second group's row KMP halfwords on, zeros kzo
// halfwords after the scales), online softmax, value accumulation from the
// wave's staged value tile.  Scales are folded into the other MFMA operand
// (see kivi_tile): codes enter the f16 MFMAs as exact integers.
template <int D, int BITS, int KROW, int KMP>
__device__ __forceinline__ void kivi_tile64(int lane, const f16x8 (&qh)[D / 32], const char* kc, const _Float16* kms,
                                            int kzo, const char* vst, const char* vml, bool second, float& m_run,
                                            f32x4& negm, f32x4 (&acc)[D / 16], f32x4& zv) {
  constexpr int KK = D / 32, NGV = D / 32, VROW = D * BITS / 8;
  const int l16 = lane & 15, lg = lane >> 4;
  // 2-bit: sc[sg*2 + p][i] is tile token 32sg + 8lg + 2i + p
  // 4-bit: sc[tb][i]       is tile token 16tb + 4lg + i
  f32x4 sc[4];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    const _Float16* ks_row = kms + sg * KMP;
    f16x8 qs[KK];
    f32x4 z = negm;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int off = lg * (D / 4) + kk * 8;
      const u32x4 ks = *reinterpret_cast<const u32x4*>(ks_row + off);
      const u32x4 kz = *reinterpret_cast<const u32x4*>(ks_row + kzo + off);
      qs[kk] = scale8(qh[kk], ks);
      z = mfma_f16(__builtin_bit_cast(f16x8, kz), qh[kk], z);
    }
    sc[sg * 2 + 0] = z;
    sc[sg * 2 + 1] = z;
#pragma unroll
    for (int bb = 0; bb < (BITS == 2 ? 1 : 2); ++bb) {
      const int blk = BITS == 2 ? sg : sg * 2 + bb;
#pragma unroll
      for (int rd = 0; rd < KK / 2; ++rd) {
        const int ch = lg * (D / 4) + rd * 16 + l16;
        const u32x2 x = tr4(kc + ch * KROW + blk * 8);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int kk = rd * 2 + half;
          if (BITS == 2) {
            const uint32_t e = x[half] & 0x33333333u, od = (x[half] >> 2) & 0x33333333u;
            sc[sg * 2 + 0] = mfma_f16(codes_fp4(e), qs[kk], sc[sg * 2 + 0]);
            sc[sg * 2 + 1] = mfma_f16(codes_fp4(od), qs[kk], sc[sg * 2 + 1]);
          } else {
            const uint32_t lo = x[half] & 0x0F0F0F0Fu, hi = (x[half] >> 4) & 0x0F0F0F0Fu;
            sc[blk] = mfma_f16(codes_fp8(lo, hi), qs[kk], sc[blk]);
          }
        }
      }
    }
  }

  // a tile that ends its split after its first key group: the second
  // group's tokens (past the split) take no part
  if (!second) {
    sc[2] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    sc[3] = sc[2];
  }
  float p[16];
  kivi_softmax<D>(sc, m_run, negm, acc, zv, p);
  f16x8 pb[2];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int idx = BITS == 2 ? (sg * 2 + (jj & 1)) * 4 + (jj >> 1) : (2 * sg + (jj >> 2)) * 4 + (jj & 3);
      pb[sg][jj] = (_Float16)p[idx];
    }

#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    f16x8 pg[NGV];
#pragma unroll
    for (int g = 0; g < NGV; ++g)
      pg[g] = scale8(pb[sg], *reinterpret_cast<const u32x4*>(vml + vmeta_slot<D, BITS>(0, g, sg * 32) * 2 + lg * 16));
    {
      const u32x4 vz = *reinterpret_cast<const u32x4*>(vml + vmeta_slot<D, BITS>(1, min(l16, NGV), sg * 32) * 2 + lg * 16);
      zv = mfma_f16(__builtin_bit_cast(f16x8, vz), pb[sg], zv);
    }
    if (BITS == 2) {
#pragma unroll
      for (int rd = 0; rd < D / 64; ++rd) {
        const int r = l16 & 7, cbr = 2 * rd + (l16 >> 3);
        const int tok = 32 * sg + 8 * lg + r;
        const u32x2 x = tr4(vst + tok * VROW + cbr * 8);
        const int ca = 2 * rd, cbb = 2 * rd + 1;
        const uint32_t e0 = x[0] & 0x33333333u, e1 = x[1] & 0x33333333u;
        const uint32_t o0 = (x[0] >> 2) & 0x33333333u, o1 = (x[1] >> 2) & 0x33333333u;
        acc[ca * 2 + 0] = mfma_f16(codes_fp4(e0), pg[ca], acc[ca * 2 + 0]);
        acc[cbb * 2 + 0] = mfma_f16(codes_fp4(e1), pg[cbb], acc[cbb * 2 + 0]);
        acc[ca * 2 + 1] = mfma_f16(codes_fp4(o0), pg[ca], acc[ca * 2 + 1]);
        acc[cbb * 2 + 1] = mfma_f16(codes_fp4(o1), pg[cbb], acc[cbb * 2 + 1]);
      }
    } else {
#pragma unroll
      for (int rd = 0; rd < D / 32; ++rd) {
        const int r = l16 & 7, cbr = 2 * rd + (l16 >> 3);
        const int tok = (r & 1) ? 32 * sg + 16 + 4 * lg + (r >> 1) : 32 * sg + 4 * lg + (r >> 1);
        const u32x2 x = tr4(vst + tok * VROW + cbr * 8);
        const uint32_t lo0 = x[0] & 0x0F0F0F0Fu, hi0 = (x[0] >> 4) & 0x0F0F0F0Fu;
        const uint32_t lo1 = x[1] & 0x0F0F0F0Fu, hi1 = (x[1] >> 4) & 0x0F0F0F0Fu;
        acc[2 * rd] = mfma_f16(codes_fp8(lo0, hi0), pg[rd], acc[2 * rd]);
        acc[2 * rd + 1] = mfma_f16(codes_fp8(lo1, hi1), pg[rd], acc[2 * rd + 1]);
      }
    }
  }
}

template <int D, int BITS, int KPB>
__global__ __launch_bounds__(kKsWaves * 64, 1) void kivi_stream_kernel(KiviArgs a) {
  using C = KsCfg<D, BITS, KPB>;
  using Regs = KsRegs<D, BITS, KPB>;
  constexpr int NT = C::NT;
  constexpr int DEPTH = C::DEPTH;
  PREFETCH_ARGS(a);
  __shared__ __attribute__((aligned(16))) char smem_raw[C::kSmem];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const UnitLoc loc = splitk_locate(a.o);
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk, hb = loc.hb;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);
  const uint16_t* qrow0 = a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh;
  const bool qlive = l16 < nh;

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int Sq = a.Sq;
  const bool quant = split < a.nsq;                // else a split of the residual window
  const int t_begin = quant ? split * a.chunk : 0;
  const int t_end = quant ? min(t_begin + a.chunk, Sq) : 0;
  const int ntok = t_end - t_begin;                // a multiple of 32
  const int r_begin = quant ? 0 : (split - a.nsq) * kResidPerSplit;
  const int r_end = quant ? 0 : min(r_begin + kResidPerSplit, a.R);
  const int rt = r_begin + w * kTile;
  const bool rtile = !quant && w < 4 && rt < r_end;

  if (quant) {
    const int nph = (ntok + kKsPhase - 1) / kKsPhase;
    const int64_t bh = (int64_t)b * a.Hk + hk;
    const int ngk = Sq >> 5;
    const int64_t wk = Sq * BITS / 32;             // int32 words per key channel row
    // zeros are addressed from the scales plus a uniform distance: a per-lane
    // choice between two argument fields otherwise becomes a vector load of
    // the argument block, waited on before the first request
    const int64_t kz_off = a.km - a.ks, vz_off = a.vm - a.vs;

    // Q as the fp16 B operand (scaled by scale*log2e), lane: Q[h = l16][ch = lg*(D/4) + kk*8 + kslot_ch(jj)]
    u32x4 qraw[D / 32];
    {
      const uint16_t* qp = qrow0 + (int64_t)(qlive ? l16 : 0) * a.q_sh + lg * (D / 4);
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) qraw[kk] = ld16(qp + kk * 8);
    }

    // Requests of phase ph (clamped into the split: phases and groups past its
    // end re-read its last valid bytes, which nothing uses).
    auto issue = [&](int ph, Regs& r) {
      const int p0 = t_begin + min(ph, nph - 1) * kKsPhase;            // phase's first token
      const int nvt = min(kKsPhase, t_end - p0);                        // valid tokens of the phase
      const int npc = max(nvt * BITS / 8 / KPB, 1);                     // valid key pieces per channel
      const int ngv = max(nvt >> 5, 1);                                 // valid key groups
      const uint32_t* kqb = a.kq + (bh * D) * wk + p0 * BITS / 32;
#pragma unroll
      for (int i = 0; i < C::KP; ++i) {
        const int pc = min((int)threadIdx.x + NT * i, C::NKP - 1);
        const int ch = pc / C::PPC, q = pc - (pc / C::PPC) * C::PPC;
        r.k[i] = *reinterpret_cast<const typename Regs::KPiece*>(kqb + ch * wk + min(q, npc - 1) * (KPB / 4));
      }
      const int g0 = p0 >> 5;
#pragma unroll
      for (int i = 0; i < C::KMPT; ++i) {
        const int e = min((int)threadIdx.x + NT * i, C::NKM - 1);
        const int g = e % kKsGroups, row = e / kKsGroups;               // row = sm * D + ch
        const int sm = row / D, ch = row - sm * D;
        const _Float16* src = a.ks + (sm ? kz_off : 0) + (bh * D + ch) * ngk + g0 + min(g, ngv - 1);
        r.km[i] = *reinterpret_cast<const uint16_t*>(src);
      }
      // this wave's tile (waves past the phase's tokens re-read its last
      // tile); reads stay inside its tv valid tokens (32 or 64)
      const int wt = p0 + min(w * 64, (nvt - 1) & ~63);
      const int tv = min(64, t_end - wt);
      const char* vsrc = reinterpret_cast<const char*>(a.vq + bh * (int64_t)Sq * (D * BITS / 32)) +
                         (int64_t)wt * C::VROW;
#pragma unroll
      for (int i = 0; i < C::VDMA; ++i) r.v[i] = ld16_nt(vsrc + min((lane + 64 * i) * 16, tv * C::VROW - 16));
      const _Float16* mp =
          a.vs + (lane < 32 ? 0 : vz_off) + (bh * Sq + wt + min(2 * (lane & 31), tv - 2)) * C::NGV;
      r.vm = *reinterpret_cast<const VMetaReg<D>*>(mp);
    };
    auto stage = [&](const Regs& r) {
      char* kbuf = smem_raw;
      _Float16* kml = reinterpret_cast<_Float16*>(smem_raw + C::KBYTES);
      char* vst = smem_raw + C::KBYTES + C::KMBYTES + w * C::WAVE;
      char* vml = vst + C::VBYTES;
#pragma unroll
      for (int i = 0; i < C::KP; ++i) {
        const int pc = threadIdx.x + NT * i;
        const int ch = pc / C::PPC, q = pc - (pc / C::PPC) * C::PPC;
        const int off = pc < C::NKP ? ch * C::KROW + q * KPB : D * C::KROW + (pc - C::NKP) * KPB;
        *reinterpret_cast<typename Regs::KPiece*>(kbuf + off) = r.k[i];
      }
#pragma unroll
      for (int i = 0; i < C::KMPT; ++i) {
        const int e = threadIdx.x + NT * i;
        if (C::KMPT * NT > C::NKM && e >= C::NKM) continue;
        const int g = e % kKsGroups, row = e / kKsGroups;
        const int sm = row / D, ch = row - sm * D;
        kml[(sm * kKsGroups + g) * C::KMP + kslot_pos<BITS>(ch)] = __builtin_bit_cast(_Float16, r.km[i]);
      }
#pragma unroll
      for (int i = 0; i < C::VDMA; ++i) *reinterpret_cast<u32x4*>(vst + (lane + 64 * i) * 16) = r.v[i];
      const _Float16* hv = reinterpret_cast<const _Float16*>(&r.vm);
      _Float16* dst = reinterpret_cast<_Float16*>(vml);
      const int sm = lane >> 5, tau0 = 2 * (lane & 31);
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int g = 0; g < C::NGV; ++g) dst[vmeta_slot<D, BITS>(sm, g, tau0 + u)] = hv[u * C::NGV + g];
    };

    Regs rg[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      issue(d, rg[d]);
      __builtin_amdgcn_sched_barrier(0);
    }

    f16x8 qh[D / 32];
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) {
      const bf16x8 qv = __builtin_bit_cast(bf16x8, qraw[kk]);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) qh[kk][jj] = (_Float16)((float)qv[kslot_ch<BITS>(jj)] * a.scale_log2);
    }
    f32x4 zv = {0.f, 0.f, 0.f, 0.f}, negm = {0.f, 0.f, 0.f, 0.f};
    // this wave's ones rows (read by the value zero-term MFMA), published by
    // the first phase's barrier
    reinterpret_cast<uint16_t*>(smem_raw + C::KBYTES + C::KMBYTES + w * C::WAVE + C::VBYTES + C::VMBYTES)[lane] =
        0x3C00u;
    // Phases run in groups of DEPTH (the last group padded with empty phases,
    // whose requests re-read the split's last bytes).  Every group but the
    // last requests the next group's phases, one per staged phase, with no
    // condition, so the waits before each staging count exactly the
    // requests that came after its own.  One LDS buffer: the barrier before
    // the staging waits for every wave to finish the previous phase.
    // Phase p + DEPTH is requested before phase p is computed, except for
    // 4-bit keys at D = 128, where it is requested after (its registers would
    // otherwise not fit beside the tile's).
    constexpr bool kEarly = !(BITS == 4 && D == 128);
    auto run_phase = [&](int ph, int d, bool more) {
      if (ph > 0) __syncthreads();
      stage(rg[d]);
      if (more && kEarly) issue(ph + DEPTH, rg[d]);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      const int left = ntok - (ph * kKsPhase + w * 64);                 // tokens of this wave's tile
      if (left > 0) {
        const _Float16* kms = reinterpret_cast<const _Float16*>(smem_raw + C::KBYTES) + 2 * w * C::KMP;
        const char* vst = smem_raw + C::KBYTES + C::KMBYTES + w * C::WAVE;
        kivi_tile64<D, BITS, C::KROW, C::KMP>(lane, qh, smem_raw + w * 64 * BITS / 8, kms, kKsGroups * C::KMP, vst,
                                              vst + C::VBYTES, left > 32, m_run, negm, acc, zv);
      }
      if (more && !kEarly) {
        __builtin_amdgcn_sched_barrier(0);
        issue(ph + DEPTH, rg[d]);
      }
    };
    const int ngroups = (nph + DEPTH - 1) / DEPTH;
    int p0 = 0;
    for (int gi = 0; gi + 1 < ngroups; ++gi, p0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) run_phase(p0 + d, d, true);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (p0 + d < nph) run_phase(p0 + d, d, false);
    }
    kivi_finish<D>(lane, zv, acc, l_run);
  } else if (rtile) {
    // A split of the bf16 residual window: one 32-token dense tile per wave of
    // waves 0-3.  Its K and V rows go straight from HBM to the wave's LDS tile
    // buffers (global_load_lds) in the buffers' swizzled layout: LDS chunk c
    // of row r holds column chunk c ^ swz(r).
    using DC = DenseCfg<D>;
    const uint16_t* rkbase = a.kr + (int64_t)b * a.kr_sb + (int64_t)hk * a.kr_sh;
    const uint16_t* rvbase = a.vr + (int64_t)b * a.vr_sb + (int64_t)hk * a.vr_sh;
    char* kst = smem_raw + w * DC::WAVE;
    char* rvst = kst + DC::VT;
#pragma unroll
    for (int i = 0; i < DC::VT / 1024; ++i) {
      const int p = lane + 64 * i;
      const int rr = p / DC::CPR, cc = p - rr * DC::CPR;
      const int row = min(rt + rr, a.R - 1);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(rkbase + (int64_t)row * a.kr_ss + kswz<D>(rr, cc) * 8),
          (__attribute__((address_space(3))) void*)(kst + i * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(rvbase + (int64_t)row * a.vr_ss + vswz<D>(rr, cc) * 8),
          (__attribute__((address_space(3))) void*)(rvst + i * 1024), 16, 0, 0);
    }
    bf16x8 qb[D / 32];
    load_q_bf16<D>(qrow0, a.q_sh, nh, lane, qb);
    // the compiler does not track LDS written by global_load_lds: wait for
    // every request (the tile's and Q's) before the tile is read
    __builtin_amdgcn_s_waitcnt(0);
    wave_lds_sync();
    dense_compute<D>(range_mask(rt, r_end), a.scale_log2, lane, qb, kst, rvst, m_run, l_run, acc);
  }
  splitk_epilogue<D, kKsWaves>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b, hq0, nh,
                               (BITS == 2 && quant) ? kDmapKivi2 : kDmapDense);
}

template <int D, int BITS, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void kivi_decode_kernel(KiviArgs a) {
  using C = KiviCfg<D, BITS, NW>;
  PREFETCH_ARGS(a);
  __shared__ __attribute__((aligned(16))) char smem_raw[C::kSmem];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int l16 = lane & 15, lg = lane >> 4;
  const UnitLoc loc = splitk_locate(a.o);
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk, hb = loc.hb;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);
  const uint16_t* qrow0 = a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh;

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The bf16 residual window [0, R) runs as dense 32-token tiles, at most one
  // per wave of waves 0-3 (the host keeps every split's share at or below 128
  // tokens), either on splits of its own (a.rsplit > 0: splits nsq.., 128
  // tokens each, when the extra workgroups still fit on the device at once)
  // or in pieces of a.rchunk tokens on the last splits (piece i on split
  // nsplit-1-i), after their quantized tiles: the residual rows are requested
  // once the second half is staged and arrive during the last tiles; (2-bit)
  // the accumulator then moves to the dense layout for the residual tile.
  const bool resid_only = a.rsplit > 0 && split >= a.nsq;
  const int rpiece = a.o.nsplit - 1 - split;
  const int r_begin = resid_only ? (split - a.nsq) * kResidPerSplit : rpiece * a.rchunk;
  const int r_end = min(r_begin + (resid_only ? kResidPerSplit : a.rchunk), a.R);
  const bool resid_first = a.rsplit == 0 && a.R > 0 && r_begin < r_end;
  const bool resid = resid_only || resid_first;
  static_assert(kResidPerSplit == 4 * kTile && NW >= 4, "one residual tile per wave of waves 0-3");
  const int rt = r_begin + w * kTile;
  // Lanes of head columns past nh load head hq0's query instead of zeros:
  // their scores and accumulators are computed and never stored, and no
  // select on a loaded value has to wait for the load at the end of the
  // conditional blocks that issue it.
  DenseRegs<D> rr;
  u32x4 qbraw[D / 32];
  const bool qlive = l16 < nh;
  const bool rtile = resid && rt < r_end;         // this wave has a residual tile
  // residual rows (the bases are computed where the residual is used)
  auto resid_k = [&]() { return a.kr + (int64_t)b * a.kr_sb + (int64_t)hk * a.kr_sh; };
  auto resid_v = [&]() { return a.vr + (int64_t)b * a.vr_sb + (int64_t)hk * a.vr_sh; };
  auto issue_resid = [&]() {
    dense_issue<D>(resid_k(), resid_v(), a.kr_ss, a.vr_ss, a.R, rt, r_end, lane, rr);
    const uint16_t* qp = qrow0 + (int64_t)(qlive ? l16 : 0) * a.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) qbraw[kk] = ld16(qp + kk * 32);
  };

  const int Sq = a.Sq;
  const int t_begin = split * a.chunk;
  const int t_end = resid_only ? t_begin : min(t_begin + a.chunk, Sq);
  const bool quant = t_begin < t_end;
  const int g_lo = t_begin >> 5;
  const int ngs = (t_end - t_begin) >> 5;        // even: splits are multiples of 64 tokens
  const uint32_t bh = (uint32_t)(b * a.Hk + hk);
  const int ngk = Sq >> 5;

  char* kchunk = smem_raw;
  char* kmeta = smem_raw + C::KCBYTES;
  char* vst = kmeta + C::KMETA + w * C::WAVE_BYTES;   // value codes of the wave's tile in half ph: + ph * VBYTES
  char* vml = vst + 2 * C::VBYTES;

  // The first half's scale/zero requests are issued on every path, so that
  // each wait the compiler counts sees the same requests whatever the path
  // (the counts of a wait after paths that issued different requests are
  // those of the shortest).  A split without quantized tokens (a residual-only
  // split, or Sq == 0 with no quantized cache at all) requests them through
  // zero-sized resources and reads zeros, and requests no codes (their LDS-DMA
  // would land in the residual tiles' buffers).
  const uint32_t wkb = (uint32_t)Sq * BITS / 8;    // bytes per key channel row
  const uint32_t mrb = (uint32_t)ngk * 2;          // bytes per key scale/zero row
  // a unit's part of each tensor: unit bytes (32-bit) times the unit index
  auto at = [&](const void* p, uint32_t unit_bytes) {
    return static_cast<const char*>(p) + (uint64_t)bh * unit_bytes;
  };
  const uint32_t kq_u = D * wkb, km_u = D * mrb, vq_u = (uint32_t)Sq * C::VROW, vm_u = (uint32_t)Sq * C::NGV * 2;
  KiviRsrc rs;
  rs.kq = buf_rsrc(at(a.kq, kq_u), quant ? kq_u : 0u);
  rs.ks = buf_rsrc(at(a.ks, km_u), quant ? km_u : 0u);
  rs.kz = buf_rsrc(at(a.km, km_u), quant ? km_u : 0u);
  rs.vq = buf_rsrc(at(a.vq, vq_u), quant ? vq_u : 0u);
  rs.vs = quant ? at(a.vs, vm_u) : reinterpret_cast<const char*>(qrow0);
  rs.vz = quant ? at(a.vm, vm_u) : reinterpret_cast<const char*>(qrow0);
  // the code resources again, in scalar registers for the LDS-DMA requests
  const __amdgpu_buffer_rsrc_t rkq = buf_rsrc_uniform(at(a.kq, kq_u), quant ? kq_u : 0u);
  const __amdgpu_buffer_rsrc_t rvq = buf_rsrc_uniform(at(a.vq, vq_u), quant ? vq_u : 0u);

  // Q as the fp16 B operand (scaled by scale*log2e):
  //   lane holds Q[h = l16][ch = lg*(D/4) + kk*8 + kslot_ch(jj)],
  // read from the workgroup's staged copy: thread t < 16 * D/8 loads chunk
  // t % (D/8) of head column t / (D/8) (columns past nh take head hq0's row;
  // their results are never stored).
  constexpr int QT = 16 * (D / 8);
  const int qt = min((int)threadIdx.x, QT - 1);
  const int qh_col = qt / (D / 8), qc = qt % (D / 8);
  u32x4 qraw1;

  // The chunk is staged in two halves of C::CHUNK/2 tokens, each the
  // first (ph = 0) or second (ph = 1) tile of every wave.  Key codes and
  // value codes go HBM -> LDS by LDS-DMA (no VGPRs: loads returning into
  // VGPRs while the waves compute the first half measured ~1.5x slower
  // tiles); key scales/zeros, two groups per 4-byte word, and value
  // scales/zeros go through VGPRs into their transposed layouts.
  constexpr int STEP = NW * kKiviTile;
  constexpr int NTW = C::CHUNK / STEP;
  static_assert(NTW == 2, "two halves, one tile per wave each");
  constexpr int NT = NW * 64;
  constexpr int NPC = C::NPC;
  constexpr int WRH = C::KMG / 4;                  // meta words per (scale|zero, channel) per half
  constexpr int PERMH = 2 * D * WRH / NT;
  static_assert(NT / WRH == 64 && D % 64 == 0, "row blocks of the staging loops");
  const int nwr = quant ? ngs >> 1 : 1;
  // per-thread parts of the offsets: key LDS-DMA request j of wave w covers
  // rows blk * KROWS_DMA + lane / NPC (blk = w * KDMA + j), slot lane % NPC
  // <- the piece kslot_swz maps there; thread t takes word t % WRH of meta
  // row t / WRH (+ 64 rows per step, scales then zeros)
  const int tid = threadIdx.x;
  const uint32_t mrow = (uint32_t)(tid / WRH) * mrb, mwd = tid % WRH;
  const uint32_t msplit = (uint32_t)g_lo * 2;
  const int tw = t_begin + w * kKiviTile;
  uint32_t mv[NTW][PERMH];
  VMetaReg<D> vm[NTW];
  // A half's requests: the wave's value codes and its share of the key codes
  // (LDS-DMA), then the key and value scales/zeros (VGPRs).  Every offset of
  // a code request is in the VGPR offset, which the range check covers.
  auto issue = [&](auto phc) {
    constexpr int ph = decltype(phc)::value;
    const int t = tw + ph * STEP;
    const int tv = t < t_end ? t : t_begin;
    if (quant) {
#pragma unroll
      for (int i = 0; i < C::VDMA; ++i)
        lds_dma16<true>(rvq, vst + ph * C::VBYTES + i * 1024, (uint32_t)(tv * C::VROW + i * 1024 + lane * 16));
      // non-temporal when a half's pieces of a channel row fill whole 128-byte
      // lines (else the other half of each line is fetched again later)
      constexpr bool KNT = C::KROW >= 128;
      const uint32_t kh = (uint32_t)(t_begin + ph * STEP) * BITS / 8;
#pragma unroll
      for (int j = 0; j < C::KDMA; ++j) {
        const int blk = w * C::KDMA + j;
        const int row = blk * C::KROWS_DMA + lane / NPC;
        const uint32_t off = (uint32_t)row * wkb + (uint32_t)(kslot_swz<NPC>(lane % NPC, row) << 4) + kh;
        lds_dma16<KNT>(rkq, kchunk + ph * C::KHALF + blk * 1024, off);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    vm[ph] = kivi_load_vmeta<D>(rs, quant, tv, lane);
    const int mo = mrow + min(ph * WRH + (int)mwd, nwr - 1) * 4;
#pragma unroll
    for (int i = 0; i < PERMH; ++i) {
      const int r0 = (i * 64) % D;                 // first channel of this step's rows
      const uint32_t so = msplit + (uint32_t)r0 * mrb;
      mv[ph][i] = (i * 64) / D ? __builtin_amdgcn_raw_buffer_load_b32(rs.kz, mo, (int)so, 0)
                               : __builtin_amdgcn_raw_buffer_load_b32(rs.ks, mo, (int)so, 0);
    }
    // keep the compiler from moving requests across this point
    __builtin_amdgcn_sched_barrier(0);
  };
  auto issue_first = [&]() {
    qraw1 = ld16(qrow0 + (int64_t)(qh_col < nh ? qh_col : 0) * a.q_sh + qc * 8);
    issue(std::integral_constant<int, 0>());
  };
  issue_first();
  if (!quant && rtile) issue_resid();             // residual-only split


  if (quant) {
    char* qlds = smem_raw + C::QOFF;
    {
      const bf16x8 qv = __builtin_bit_cast(bf16x8, qraw1);
      f16x8 qo;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) qo[jj] = (_Float16)((float)qv[kslot_ch<BITS>(jj)] * a.scale_log2);
      if ((int)threadIdx.x < QT) *reinterpret_cast<f16x8*>(qlds + qh_col * C::QP + qc * 16) = qo;
    }
    f16x8 qh[D / 32];

    _Float16* km_lds = reinterpret_cast<_Float16*>(kmeta);
    // value zero term: row g = value group, column = head; rows >= NGV: the
    // denominators
    f32x4 zv = {0.f, 0.f, 0.f, 0.f}, negm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ph = 0; ph < NTW; ++ph) {
      // every request of this half (and, at ph 0, Q) done: the LDS-DMA data
      // is in LDS once its request has counted down
      __builtin_amdgcn_s_waitcnt(0x0F70);         // vmcnt(0)
      // this half's key scales/zeros into LDS, stored unconditionally (groups
      // past the chunk end hold clamped copies no tile reads): a store under
      // a lane mask lets the compiler sink the load feeding it down to the
      // store, behind waits for every earlier load
#pragma unroll
      for (int i = 0; i < PERMH; ++i) {
        const int pc = threadIdx.x + NT * i;
        const int row = pc / WRH, wi = ph * WRH + (pc - (pc / WRH) * WRH);
        const int sm = row / D, ch = row - sm * D;
        _Float16* dst = km_lds + (sm * C::KMG + 2 * wi) * C::KMP + kslot_pos<BITS>(ch);
        dst[0] = __builtin_bit_cast(_Float16, (uint16_t)(mv[ph][i] & 0xFFFFu));
        dst[C::KMP] = __builtin_bit_cast(_Float16, (uint16_t)(mv[ph][i] >> 16));
      }
      // The second half is requested only once the first has arrived: first
      // halves then reach the head of the memory queues before second
      // halves, and the second half streams in while the first tiles run.
      // One workgroup per CU (NW = 8): once the whole workgroup's first half
      // has arrived (measured faster there); several rounds of 4-wave
      // workgroups: by each wave once its own share has arrived (the wait
      // above; the barrier then orders LDS only, so those requests stay in
      // flight), which keeps more bytes in flight.
      constexpr bool kWaveIssue = NW == 4;
      if (kWaveIssue && ph == 0) issue(std::integral_constant<int, 1>());
      if (kWaveIssue) lds_barrier();
      else __syncthreads();
      if (ph == 0) {
#pragma unroll
        for (int kk = 0; kk < D / 32; ++kk)
          qh[kk] = *reinterpret_cast<const f16x8*>(qlds + l16 * C::QP + (lg * (D / 32) + kk) * 16);
      }
      if (!kWaveIssue && ph == 0) issue(std::integral_constant<int, 1>());
      const int t = tw + ph * STEP;
      wave_lds_sync();
      kivi_stage_vmeta<D, BITS>(lane, vm[ph], vml);
      if (ph == 1 && rtile) issue_resid();        // arrives during the last tiles
      wave_lds_sync();
      if (t < t_end) {
        // the wave's tile is piece w (2-bit) or pieces 2w, 2w + 1 (4-bit) of
        // each key channel row of the half
        const char* krow0 = kchunk + ph * C::KHALF + l16 * C::KROW;
        const char* const kb[2] = {
            BITS == 2 ? krow0 + (kslot_swz<NPC>(w, l16) << 4) : krow0 + (kslot_swz<NPC>(2 * w, l16) << 4),
            BITS == 2 ? krow0 + (kslot_swz<NPC>(w, l16) << 4) + 8 : krow0 + (kslot_swz<NPC>(2 * w + 1, l16) << 4)};
        kivi_tile_at<D, BITS, C::KROW, C::KMP>(lane, qh, kb, kmeta, C::KMG * C::KMP * 2, (t >> 5) - g_lo,
                                               vst + ph * C::VBYTES, vml, m_run, negm, acc, zv);
      }
    }
    kivi_finish<D>(lane, zv, acc, l_run);
  }

  if (resid) {
    // Wave w's residual tile uses LDS bytes [w, w+1) * DenseCfg<D>::WAVE.  With
    // quantized tiles, waves below RES_EARLY find those bytes in the first
    // half's key block, which no wave reads once the second half is staged:
    // when the split's residual tiles all fit there they run right after the
    // wave's own tiles, while other waves still work on theirs.  Otherwise every
    // wave first finishes with the chunk.  Without quantized tiles the LDS is
    // not otherwise in use before the epilogue.
    const int ntiles = (r_end - r_begin + kTile - 1) / kTile;
    if (quant && ntiles > C::RES_EARLY) __syncthreads();
    if (rtile) {
      char* wbuf = smem_raw + w * DenseCfg<D>::WAVE;
      char* kst = wbuf;
      char* rvst = wbuf + DenseCfg<D>::VT;
      if (BITS == 2 && quant) {
        // 2-bit value layout -> dense layout, through the wave's buffer
        static_assert(D * 16 * 4 <= DenseCfg<D>::WAVE, "relayout buffer fits the wave's tile buffers");
        float* buf = reinterpret_cast<float*>(wbuf);
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) buf[acc_d(kDmapKivi2, db, lg, i) * 16 + l16] = acc[db][i];
        wave_lds_sync();
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[db][i] = buf[(db * 16 + lg * 4 + i) * 16 + l16];
      }
      // Q as the bf16 B operand of the dense tile: lane holds Q[h = l16][d = kk*32 + lg*8 + j]
      bf16x8 qb[D / 32];
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) qb[kk] = __builtin_bit_cast(bf16x8, qbraw[kk]);
      wave_lds_sync();
      dense_stage<D>(lane, rr, kst, rvst);
      wave_lds_sync();
      dense_compute<D>(range_mask(rt, r_end), a.scale_log2, lane, qb, kst, rvst, m_run, l_run, acc);
    }
  }
  splitk_epilogue<D, NW>(m_run, l_run, acc, reinterpret_cast<float*>(smem_raw), a.o, unit, split, b, hq0,
                                 nh, (BITS == 2 && quant && !rtile) ? kDmapKivi2 : kDmapDense);
}

// ============================================================================
// Pipelined decode for long caches: 4-wave workgroups (three per CU for
// 2-bit caches, two for 4-bit), each walking a long run of 256-token granules
// through a two-stage LDS ring
// ============================================================================
// A split is a run of granules of one unit.  Granule i's key codes and value
// codes go HBM -> LDS untouched (buffer loads with the LDS bit, no VGPRs),
// its key scales/zeros and value scales/zeros through VGPRs (their staged
// layouts are transposes of the stored ones).  While the waves compute
// granule i from one stage (wave w: tile w, the granule's tokens
// [64w, 64w + 64)), granule i + 1 streams into the other; one barrier per
// granule publishes a stage.  The two stages are separate LDS arrays and
// every read of a stage follows an explicit wait for the loads into it, so
// the loads into the other stage stay in flight across the reads (the
// compiler cannot tell the LDS-DMA destinations apart within one array and
// would wait for all of them).  A 2-bit workgroup's ~50 KB of LDS and at
// most 168 VGPRs let three share a CU, a 4-bit one's 80 KB two, so one
// workgroup's barrier or loads overlap the tiles of the others.  The bf16
// residual window runs on splits of its own (waves 0 and 1, two dense
// 32-token tiles each, in the stages' space).
constexpr int kPipeWaves = 4;
constexpr int kPipeGran = kPipeWaves * kKiviTile;      // tokens per granule
template <int BITS>
constexpr int pipe_wg_per_cu() { return BITS == 2 ? 3 : 2; }

template <int D, int BITS>
struct PipeCfg {
  static_assert(D == 128 && (BITS == 2 || BITS == 4), "pipelined decode: D = 128, 2- or 4-bit caches");
  static constexpr int KK = D / 32;
  static constexpr int KPR = kPipeGran * BITS / 8;      // bytes of a key channel row per granule (64 | 128)
  static constexpr int NPC = KPR / 16;                   // 16-byte key pieces per row and granule
  static constexpr int KC = D * KPR;                     // key codes of a granule
  static constexpr int KROWS_DMA = 1024 / KPR;           // key rows per 1 KB LDS-DMA instruction
  static constexpr int KDMA = KC / (kPipeWaves * 1024);  // key LDS-DMA instructions per wave per granule
  static constexpr int NGG = kPipeGran / 32;             // key groups per granule
  // halfwords per staged (scale|zero, group) row: for 2-bit caches the
  // 8-halfword pad puts the staging stores of a wave's four group rows in
  // distinct banks; 4-bit stages go without it to fit two workgroups per CU
  static constexpr int KMP = BITS == 2 ? D + 8 : D;
  static constexpr int KM = 2 * NGG * KMP * 2;
  static constexpr int VROW = D * BITS / 8;              // bytes of one token's value codes
  static constexpr int VB = kKiviTile * VROW;            // one wave's value codes
  static constexpr int VDMA = VB / 1024;
  static constexpr int NGV = D / 32;
  static constexpr int VMB = 2 * kKiviTile * NGV * 2;   // one wave's value scales + zeros
  static constexpr int OFF_KM = KC;
  static constexpr int OFF_V = OFF_KM + KM;
  static constexpr int OFF_VM = OFF_V + kPipeWaves * VB;
  static constexpr int STAGE = OFF_VM + kPipeWaves * VMB;
  static constexpr int WG_PER_CU = pipe_wg_per_cu<BITS>();
  static_assert(NPC == 4 * BITS / 2 && KROWS_DMA * NPC == 64, "one key row per NPC lanes of an LDS-DMA instruction");
  static_assert(KDMA * kPipeWaves * 1024 == KC && VDMA * 1024 == VB, "whole LDS-DMA instructions");
  static_assert(kPipeWaves * 64 * 4 == 2 * D * NGG / 2, "four 4-byte key scale/zero words per thread and granule");
  // residual tiles (waves 0 and 1, one dense tile buffer in each stage) and
  // the split-K epilogue (waves 0-1 rows in stage 0, waves 2-3 in stage 1)
  static_assert(DenseCfg<D>::WAVE <= STAGE, "a dense tile's K and V fit a stage");
  static_assert((kPipeWaves * 16 * 2 + kPipeWaves / 2 * 16 * acc_pitch<D>()) * 4 <= STAGE, "epilogue rows fit");
  static_assert(2 * STAGE <= 160 * 1024 / WG_PER_CU, "WG_PER_CU workgroups per CU");
};

// Wave w's tile of the granule staged in `stage` (pipelined kernel): key
// channel row r holds the granule's NPC 16-byte pieces (piece p = tokens
// [256p/NPC, 256(p+1)/NPC)) in slots kslot_swz<NPC>(p, r); the tile's tokens are
// piece w (2-bit) or pieces 2w, 2w + 1 (4-bit), and for the rows a lane reads
// (l16 + 16k) the slot depends on l16 only.  Every read stays in `stage`.
template <int D, int BITS>
__device__ __forceinline__ void kivi_pipe_tile(int w, int lane, const f16x8 (&qh)[D / 32], const char* stage,
                                               float& m_run, f32x4& negm, f32x4 (&acc)[D / 16], f32x4& zv) {
  using C = PipeCfg<D, BITS>;
  const int l16 = lane & 15;
  const char* row = stage + l16 * C::KPR;
  const char* const kb[2] = {
      BITS == 2 ? row + (kslot_swz<C::NPC>(w, l16) << 4) : row + (kslot_swz<C::NPC>(2 * w, l16) << 4),
      BITS == 2 ? row + (kslot_swz<C::NPC>(w, l16) << 4) + 8 : row + (kslot_swz<C::NPC>(2 * w + 1, l16) << 4)};
  kivi_tile_at<D, BITS, C::KPR, C::KMP>(lane, qh, kb, stage + C::OFF_KM, C::NGG * C::KMP * 2, 2 * w,
                                        stage + C::OFF_V + w * C::VB, stage + C::OFF_VM + w * C::VMB, m_run, negm,
                                        acc, zv);
}

// A granule's loads: key codes and the wave's value codes into `stage` by
// LDS-DMA, key and value scales/zeros into registers.  A granule reads 64
// (2-bit) or 128 (4-bit) bytes of each key row, not aligned to its lines, and
// 16 of each 128-byte key scale/zero line, the rest of the lines belonging to
// the split's neighbouring granules: those loads keep their lines in L2 (no
// non-temporal hint); value codes and value scales/zeros are whole lines read
// once.
template <int D, int BITS>
struct PipeMeta {
  uint32_t km[4];        // word t % 4 (groups 2(t%4), +1 of the granule) of (scale|zero, channel) row 64i + t / 4
  u32x4 vm;              // value scales (lanes 0-31) / zeros (32-63) of tokens 2(l % 32), +1 of the wave's tile
};

template <int D, int BITS>
__global__ __launch_bounds__(kPipeWaves * 64, pipe_wg_per_cu<BITS>()) void kivi_pipe_kernel(KiviArgs a) {
  using C = PipeCfg<D, BITS>;
  PREFETCH_ARGS(a);
  __shared__ __attribute__((aligned(16))) char st0[C::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[C::STAGE];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const UnitLoc loc = splitk_locate(a.o);
  const int unit = loc.unit, split = loc.split, b = loc.b, hk = loc.hk, hb = loc.hb;
  const int hq0 = hk * a.G + hb * 16;
  const int nh = min(16, a.G - hb * 16);
  const uint16_t* qrow0 = a.q + (int64_t)b * a.q_sb + (int64_t)hq0 * a.q_sh;

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool resid_only = split >= a.nsq;
  if (resid_only) {
    // residual tokens [r_begin, r_end): waves 0 and 1 take 32-token tiles
    // w and w + 2; wave 0 stages in st0, wave 1 in st1
    const int r_begin = (split - a.nsq) * kResidPerSplit;
    const int r_end = min(r_begin + kResidPerSplit, a.R);
    if (w < 2) {
      bf16x8 qb[D / 32];
      load_q_bf16<D>(qrow0, a.q_sh, nh, lane, qb);
      const uint16_t* kb = a.kr + (int64_t)b * a.kr_sb + (int64_t)hk * a.kr_sh;
      const uint16_t* vb = a.vr + (int64_t)b * a.vr_sb + (int64_t)hk * a.vr_sh;
      char* kst = w == 0 ? st0 : st1;
      char* vst = kst + DenseCfg<D>::VT;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int rt = r_begin + (w + 2 * j) * kTile;
        if (rt < r_end) {
          DenseRegs<D> rr;
          dense_issue<D>(kb, vb, a.kr_ss, a.vr_ss, a.R, rt, r_end, lane, rr);
          wave_lds_sync();
          dense_stage<D>(lane, rr, kst, vst);
          wave_lds_sync();
          dense_compute<D>(range_mask(rt, r_end), a.scale_log2, lane, qb, kst, vst, m_run, l_run, acc);
        }
      }
    }
    splitk_epilogue<D, kPipeWaves>(m_run, l_run, acc, reinterpret_cast<float*>(st0), a.o, unit, split, b, hq0, nh,
                                   kDmapDense, reinterpret_cast<float*>(st1));
    return;
  }

  // ---- quantized split: granules [g_begin, g_end) of the unit ----
  const int Sq = a.Sq;
  const int t_begin = split * a.chunk;
  const int t_end = min(t_begin + a.chunk, Sq);
  const int ngr = (t_end - t_begin + kPipeGran - 1) / kPipeGran;
  const uint32_t bh = (uint32_t)(b * a.Hk + hk);
  const int ngk = Sq >> 5;
  const uint32_t wkb = (uint32_t)Sq * BITS / 8;      // bytes per key channel row
  const uint32_t kq_u = D * wkb, vq_u = (uint32_t)Sq * C::VROW;
  const __amdgpu_buffer_rsrc_t rkq = buf_rsrc(reinterpret_cast<const char*>(a.kq) + (uint64_t)bh * kq_u, kq_u);
  const __amdgpu_buffer_rsrc_t rvq = buf_rsrc(reinterpret_cast<const char*>(a.vq) + (uint64_t)bh * vq_u, vq_u);
  // key LDS-DMA: instruction blk covers key rows blk*KROWS_DMA + lane/NPC,
  // slot lane % NPC <- the piece kslot_swz maps there (an involution), which
  // depends on blk only through its parity (4-bit caches)
  uint32_t kvoff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int row = par * C::KROWS_DMA + lane / C::NPC;
    kvoff[par] = (uint32_t)(lane / C::NPC) * wkb + (uint32_t)(kslot_swz<C::NPC>(lane % C::NPC, row) << 4);
  }
  // key scales/zeros: rows 0..D-1 scales, D..2D-1 zeros of channels 0..D-1;
  // thread t reads word t % 4 of the granule's 16 bytes of rows 64i + t / 4,
  // four threads to a row (a request touches 16 lines per wave)
  const int mwd = threadIdx.x & 3, mr0 = threadIdx.x >> 2;
  static_assert(kPipeWaves * 64 / 4 == D / 2, "64 rows per step: steps 0-1 scales, 2-3 zeros");
  const _Float16* mrow = a.ks + ((size_t)bh * D + mr0) * ngk + 2 * mwd;
  const _Float16* zrow = a.km + ((size_t)bh * D + mr0) * ngk + 2 * mwd;
  // value scales/zeros of two tokens per lane
  const _Float16* vmb = (lane < 32 ? a.vs : a.vm) + (size_t)bh * Sq * C::NGV + 2 * (lane & 31) * C::NGV;

  // Every offset is in the VGPR offset, which the buffer range check covers:
  // pieces of a last, partial granule past the unit's cache read zeros.
  auto issue = [&](int gi, char* stage, PipeMeta<D, BITS>& m) {
    const int tg = t_begin + gi * kPipeGran;
#pragma unroll
    for (int j = 0; j < C::KDMA; ++j) {
      const int blk = w * C::KDMA + j;
      lds_dma16<false>(rkq, stage + blk * 1024, kvoff[blk & 1] + (uint32_t)blk * C::KROWS_DMA * wkb + (uint32_t)tg * BITS / 8);
    }
    const int tt = tg + w * kKiviTile;
#pragma unroll
    for (int j = 0; j < C::VDMA; ++j)
      lds_dma16<true>(rvq, stage + C::OFF_V + w * C::VB + j * 1024, (uint32_t)tt * C::VROW + j * 1024 + lane * 16);
    // scales/zeros of groups and tokens past the cache end: clamped copies no tile reads
    const int g0 = tg >> 5;
    const int go = min(g0 + 2 * mwd, ngk - 2) - 2 * mwd;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m.km[i] = *reinterpret_cast<const uint32_t*>((i < 2 ? mrow : zrow) + (size_t)((i & 1) * 64) * ngk + go);
    m.vm = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vmb + (size_t)min(tt, Sq - kKiviTile) * C::NGV));
  };
  auto stage_meta = [&](char* stage, const PipeMeta<D, BITS>& m) {
    _Float16* kd = reinterpret_cast<_Float16*>(stage + C::OFF_KM) + 2 * mwd * C::KMP;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int o = (i >> 1) * C::NGG * C::KMP + kslot_pos<BITS>((i & 1) * 64 + mr0);
      kd[o] = __builtin_bit_cast(_Float16, (uint16_t)(m.km[i] & 0xFFFFu));
      kd[o + C::KMP] = __builtin_bit_cast(_Float16, (uint16_t)(m.km[i] >> 16));
    }
    _Float16* vd = reinterpret_cast<_Float16*>(stage + C::OFF_VM + w * C::VMB);
    const _Float16* hv = reinterpret_cast<const _Float16*>(&m.vm);
    const int sm = lane >> 5, tau0 = 2 * (lane & 31);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int g = 0; g < C::NGV; ++g) vd[vmeta_slot<D, BITS>(sm, g, tau0 + u)] = hv[u * C::NGV + g];
  };

  PipeMeta<D, BITS> meta;
  issue(0, st0, meta);

  // Q as the fp16 B operand scaled by scale*log2(e): lane holds
  // Q[h = l16][ch = lg*(D/4) + kk*8 + kslot_ch(jj)] (head columns past nh take head hq0)
  f16x8 qh[D / 32];
  {
    const uint16_t* qp = qrow0 + (int64_t)(l16 < nh ? l16 : 0) * a.q_sh + lg * (D / 4);
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) {
      const bf16x8 qv = __builtin_bit_cast(bf16x8, ld16(qp + kk * 8));
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) qh[kk][jj] = (_Float16)((float)qv[kslot_ch<BITS>(jj)] * a.scale_log2);
    }
  }

  f32x4 zv = {0.f, 0.f, 0.f, 0.f}, negm = {0.f, 0.f, 0.f, 0.f};
  // One granule: wait for its loads (the only ones in flight), stage its
  // meta, publish the stage, request the next granule into the other stage,
  // compute this wave's tile.
  auto step = [&](int gi, char* cur, char* nxt) {
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0)
    stage_meta(cur, meta);
    lds_barrier();
    if (gi + 1 < ngr) issue(gi + 1, nxt, meta);
    if (t_begin + gi * kPipeGran + w * kKiviTile < t_end)
      kivi_pipe_tile<D, BITS>(w, lane, qh, cur, m_run, negm, acc, zv);
  };
  for (int gi = 0; gi < ngr; gi += 2) {
    step(gi, st0, st1);
    if (gi + 1 < ngr) step(gi + 1, st1, st0);
  }
  kivi_finish<D>(lane, zv, acc, l_run);
  splitk_epilogue<D, kPipeWaves>(m_run, l_run, acc, reinterpret_cast<float*>(st0), a.o, unit, split, b, hq0, nh,
                                 BITS == 2 ? kDmapKivi2 : kDmapDense, reinterpret_cast<float*>(st1));
}

// nw: 8-wave workgroups with 1024-token chunks (one per CU) when that grid
// fills between half and all of the CUs in one go; else 4-wave workgroups with
// chunks of up to 512 tokens (two per CU), whose pairs overlap one
// workgroup's loads with the other's tiles across successive workgroups.
// rsplit: the residual gets splits of its own (128 tokens each) when that keeps
// the whole grid resident, when the grid is past that already, or when four
// pieces of at most 128 tokens cannot hold it; otherwise it rides, in up to
// four pieces (rchunk tokens each), on the last splits.
static void kivi_plan(int Sq, int R, long units, int chunk_req, int* nw, int* chunk, int* nsq, int* rsplit,
                      int* rchunk) {
  const long cus = device_cu_count();
  *nw = 4;
  if (chunk_req <= 0 && Sq > 0) {
    const long n8 = (long)((Sq + 1023) / 1024) * units;
    if (2 * n8 >= cus && n8 <= cus) *nw = 8;
  }
  const int step = *nw * kKiviTile, cmax = *nw * 2 * kKiviTile;
  const long resident = (8 / *nw) * cus;
  int c;
  if (chunk_req > 0) {
    c = (chunk_req + step - 1) / step * step;
  } else {
    const long per = ((long)Sq * units + resident - 1) / resident;
    c = (int)((per + step - 1) / step * step);
  }
  if (c < step) c = step;
  if (c > cmax) c = cmax;
  *chunk = c;
  *nsq = Sq > 0 ? (Sq + c - 1) / c : 0;
  const int nr = (R + kResidPerSplit - 1) / kResidPerSplit;    // residual splits if on its own
  const int pieces = R > 0 ? (*nsq < 4 ? *nsq : 4) : 0;
  const bool own = R > 0 && (*nsq == 0 || (long)(*nsq + nr) * units <= resident || (long)*nsq * units > resident ||
                             (long)pieces * kResidPerSplit < R);
  *rsplit = own ? nr : 0;
  // pieces on the last splits: whole 32-token tiles, at most kResidPerSplit each
  int rc = 0;
  if (R > 0 && !own) {
    const int per = (R + pieces - 1) / pieces;
    rc = (per + kTile - 1) / kTile * kTile;
  }
  *rchunk = rc;
}

// Plan of the streaming kernel: one eight-wave workgroup per CU at a time.
// The bf16 residual window gets splits of its own (128 tokens, one 32-token
// tile per wave of waves 0-3), and the quantized tokens of each unit are cut
// into the splits left on the CUs (about CUs/units - residual splits), in
// `gran`-token multiples (64 for 2-bit keys read in 16-byte pieces, else 32).
static void kivi_stream_plan(int Sq, int R, long units, int chunk_req, int gran, int* chunk, int* nsq, int* rsplit,
                             int* rchunk) {
  const long cus = device_cu_count();
  const int nr = (R + kResidPerSplit - 1) / kResidPerSplit;
  int c;
  if (chunk_req > 0) {
    c = chunk_req;
  } else {
    long ns = cus / units - nr;
    if (ns < 1) ns = 1;
    c = (int)((Sq + ns - 1) / ns);
  }
  c = (c + gran - 1) / gran * gran;
  if (c < gran) c = gran;
  int n = Sq > 0 ? (Sq + c - 1) / c : 0;
  if (n + nr > 1024) {                            // the merge takes up to 1024 splits
    c = ((Sq + 1023 - nr) / (1024 - nr) + gran - 1) / gran * gran;
    n = (Sq + c - 1) / c;
  }
  *chunk = c;
  *nsq = n;
  *rsplit = nr;
  *rchunk = 0;
}

// Granules per split of the pipelined kernel chosen by the library: the
// fewest that keep the grid within two workgroups per CU (one pass of the
// grid, measured best at L = 24K-128K, B4 H_k4, for both bit widths: e.g. 2-bit
// L32K 22.0 us at four granules against 27.0 at eight, L64K 31.0 at eight
// against 33.2 at six and 32.5 at ten).
static int kivi_pipe_gps(int Sq, long units) {
  const long ng = (Sq + kPipeGran - 1) / kPipeGran;
  const long slots = 2L * device_cu_count();
  return (int)((ng * units + slots - 1) / slots);
}

// The pipelined kernel serves D = 128 caches (2- or 4-bit) of whole 64-token
// tiles and at least four granules: always when the caller asks for it
// (chunk_req < 0), never when the caller sets a split length for the other
// kernels (chunk_req > 0), and otherwise when its splits are at least three
// granules long (B4 H_k4 from L = 24K; shorter caches finish sooner on the
// two-half kernel, whose splits are shorter).
static bool kivi_use_pipe(int D, int bits, int Sq, long units, int chunk_req) {
  if (D != 128 || Sq % kKiviTile != 0 || Sq < 4 * kPipeGran) return false;
  if (chunk_req != 0) return chunk_req < 0;
  return kivi_pipe_gps(Sq, units) >= 3;
}

// Plan of the pipelined kernel: the residual window on splits of its own
// (128 tokens each), the quantized tokens of each unit cut into runs of
// kivi_pipe_gps granules (-chunk_req when the caller sets it).
static void kivi_pipe_plan(int Sq, int R, long units, int chunk_req, int* chunk, int* nsq, int* rsplit, int* rchunk) {
  const int nr = (R + kResidPerSplit - 1) / kResidPerSplit;
  const int ng = (Sq + kPipeGran - 1) / kPipeGran;
  int gps = chunk_req < 0 ? -chunk_req : kivi_pipe_gps(Sq, units);
  if (gps < 1) gps = 1;
  int n = (ng + gps - 1) / gps;
  if (n + nr > 1024) {                            // the merge takes up to 1024 splits
    gps = (ng + 1023 - nr) / (1024 - nr);
    n = (ng + gps - 1) / gps;
  }
  *chunk = gps * kPipeGran;
  *nsq = n;
  *rsplit = nr;
  *rchunk = 0;
}

// Key piece width (bytes) and split granularity (tokens) of the streaming kernel.
static void kivi_stream_shape(int bits, int* kpb, int* gran) {
  *kpb = bits == 2 ? 8 : 16;
  *gran = 32;
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_kivi_quantize_pack(const void* x, int x_dtype, int64_t rows, int T, int64_t x_row_stride, int group_size,
                             int bits, void* code, void* scale, void* mn, void* stream) {
  if (!x || !code || !scale || !mn || rows < 0 || T <= 0) return (int)hipErrorInvalidValue;
  if ((bits != 2 && bits != 4) || group_size <= 0 || T % group_size != 0 || group_size % (32 / bits) != 0)
    return (int)hipErrorInvalidValue;
  if (x_dtype < 0 || x_dtype > 2) return (int)hipErrorInvalidValue;
  const int64_t n = rows * (T / group_size);
  if (n == 0) return 0;
  const int th = 256;
  hipLaunchKernelGGL(kivi_pack_kernel, dim3((unsigned)((n + th - 1) / th)), dim3(th), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, rows, T, x_row_stride, group_size, bits,
                     static_cast<uint32_t*>(code), static_cast<_Float16*>(scale), static_cast<_Float16*>(mn));
  return (int)hipGetLastError();
}

int bytes_kivi_dequant(const void* code, const void* scale, const void* mn, int64_t rows, int T, int group_size,
                       int bits, int fp16_math, void* out, int out_dtype, void* stream) {
  if (!code || !scale || !mn || !out || rows < 0 || T <= 0) return (int)hipErrorInvalidValue;
  if ((bits != 2 && bits != 4) || group_size <= 0 || T % group_size != 0 || T % (32 / bits) != 0)
    return (int)hipErrorInvalidValue;
  if (out_dtype < 0 || out_dtype > 2) return (int)hipErrorInvalidValue;
  const int64_t n = rows * T;
  if (n == 0) return 0;
  const int th = 256;
  hipLaunchKernelGGL(kivi_dequant_kernel, dim3((unsigned)((n + th - 1) / th)), dim3(th), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(code),
                     static_cast<const _Float16*>(scale), static_cast<const _Float16*>(mn), rows, T, group_size,
                     bits, fp16_math, out, out_dtype);
  return (int)hipGetLastError();
}

int bytes_kivi_decode_workspace_size(int B, int Hq, int Hk, int Sq, int R, int D, int bits, int chunk_req,
                                     size_t* bytes) {
  if (!bytes || B <= 0 || Hk <= 0 || Hq % Hk != 0 || Sq < 0 || R < 0 || Sq + R <= 0) return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || (bits != 2 && bits != 4)) return (int)hipErrorInvalidValue;
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  int chunk, nsq, rsplit, rchunk;
  if (kivi_use_pipe(D, bits, Sq, units, chunk_req)) {
    kivi_pipe_plan(Sq, R, units, chunk_req, &chunk, &nsq, &rsplit, &rchunk);
  } else if (Sq % kKiviTile == 0) {
    int nw;
    kivi_plan(Sq, R, units, chunk_req, &nw, &chunk, &nsq, &rsplit, &rchunk);
  } else {
    int kpb, gran;
    kivi_stream_shape(bits, &kpb, &gran);
    kivi_stream_plan(Sq, R, units, chunk_req, gran, &chunk, &nsq, &rsplit, &rchunk);
  }
  *bytes = splitk_workspace_bytes(units, nsq + rsplit, D);
  return 0;
}

// Kq/K_scale/K_mn/Vq/V_scale/V_mn contiguous in the layouts above; Sq % 32 == 0
// (Sq == 0 allowed); group size 32.
int bytes_kivi_decode_attn(const void* q, const void* kq, const void* k_scale, const void* k_mn, const void* k_res,
                           const void* vq, const void* v_scale, const void* v_mn, const void* v_res, void* out,
                           int B, int Hq, int Hk, int Sq, int R, int D, int bits, int64_t q_sb, int64_t q_sh,
                           int64_t kr_sb, int64_t kr_sh, int64_t kr_ss, int64_t vr_sb, int64_t vr_sh,
                           int64_t vr_ss, int64_t o_sb, int64_t o_sh, float scale, int chunk_req, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!q || !out || B <= 0 || Hk <= 0 || Hq % Hk != 0 || Sq < 0 || R < 0 || Sq + R <= 0)
    return (int)hipErrorInvalidValue;
  if ((D != 64 && D != 128) || (bits != 2 && bits != 4)) return (int)hipErrorInvalidValue;
  if (Sq > 0 && (!kq || !k_scale || !k_mn || !vq || !v_scale || !v_mn)) return (int)hipErrorInvalidValue;
  if (R > 0 && (!k_res || !v_res)) return (int)hipErrorInvalidValue;
  if (Sq % 32 != 0) return (int)hipErrorInvalidValue;     // key groups of 32 tokens
  const int G = Hq / Hk, HB = (G + 15) / 16;
  const long units = (long)B * Hk * HB;
  if (units > 65535) return (int)hipErrorInvalidConfiguration;
  KiviArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.kq = static_cast<const uint32_t*>(kq);
  a.ks = static_cast<const _Float16*>(k_scale);
  a.km = static_cast<const _Float16*>(k_mn);
  a.vq = static_cast<const uint32_t*>(vq);
  a.vs = static_cast<const _Float16*>(v_scale);
  a.vm = static_cast<const _Float16*>(v_mn);
  a.kr = static_cast<const uint16_t*>(k_res);
  a.vr = static_cast<const uint16_t*>(v_res);
  a.kr_sb = kr_sb; a.kr_sh = kr_sh; a.kr_ss = kr_ss;
  a.vr_sb = vr_sb; a.vr_sh = vr_sh; a.vr_ss = vr_ss;
  a.Hk = Hk; a.G = G; a.HB = HB; a.Sq = Sq; a.R = R;
  a.scale_log2 = scale * kLog2e;
  // Sq a multiple of 64: the two-half kernel; else (an odd number of 32-token
  // key groups) the streaming kernel, whose loads and tiles take 32-token
  // granularity
  const bool pipe = kivi_use_pipe(D, bits, Sq, units, chunk_req);
  const bool halves = !pipe && Sq % kKiviTile == 0;
  int nw = 8, kpb = 16, gran = 32;
  if (pipe) {
    kivi_pipe_plan(Sq, R, units, chunk_req, &a.chunk, &a.nsq, &a.rsplit, &a.rchunk);
  } else if (halves) {
    kivi_plan(Sq, R, units, chunk_req, &nw, &a.chunk, &a.nsq, &a.rsplit, &a.rchunk);
  } else {
    kivi_stream_shape(bits, &kpb, &gran);
    kivi_stream_plan(Sq, R, units, chunk_req, gran, &a.chunk, &a.nsq, &a.rsplit, &a.rchunk);
  }
  const int ns = a.nsq + a.rsplit;                       // quantized chunks, then the residual's own splits
  if (!workspace || workspace_bytes < splitk_workspace_bytes(units, ns, D)) return (int)hipErrorInvalidValue;
  if (ns > 1024) return (int)hipErrorInvalidConfiguration;
  a.o.out = out;
  a.o.out_dtype = kOutBF16;
  a.o.o_sb = o_sb; a.o.o_sh = o_sh;
  a.o.Hk = Hk; a.o.HB = HB; a.o.G = G;
  splitk_carve(workspace, units, ns, a.o);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(ns * units));
  if (pipe) {
    if (bits == 2) BYTES_LAUNCH(kProfKivi, (kivi_pipe_kernel<128, 2>), grid, dim3(kPipeWaves * 64), 0, st, a);
    else BYTES_LAUNCH(kProfKivi, (kivi_pipe_kernel<128, 4>), grid, dim3(kPipeWaves * 64), 0, st, a);
    int rc = (int)hipGetLastError();
    if (rc) return rc;
    return splitk_combine(a.o, units, D, st);
  }
  if (halves) {
    const dim3 block(nw * 64);
#define KIVI_HALVES(DD, BB)                                                                         \
  if (nw == 8) BYTES_LAUNCH(kProfKivi, (kivi_decode_kernel<DD, BB, 8>), grid, block, 0, st, a);     \
  else BYTES_LAUNCH(kProfKivi, (kivi_decode_kernel<DD, BB, 4>), grid, block, 0, st, a);
    if (D == 128 && bits == 2) {
      KIVI_HALVES(128, 2)
    } else if (D == 128 && bits == 4) {
      KIVI_HALVES(128, 4)
    } else if (D == 64 && bits == 2) {
      KIVI_HALVES(64, 2)
    } else {
      KIVI_HALVES(64, 4)
    }
#undef KIVI_HALVES
    int rc = (int)hipGetLastError();
    if (rc) return rc;
    return splitk_combine(a.o, units, D, st);
  }
  const dim3 block(kKsWaves * 64);
#define KIVI_LAUNCH(DD, BB, KP) BYTES_LAUNCH(kProfKivi, (kivi_stream_kernel<DD, BB, KP>), grid, block, 0, st, a)
  if (D == 128 && bits == 2) {
    KIVI_LAUNCH(128, 2, 8);
  } else if (D == 128 && bits == 4) {
    KIVI_LAUNCH(128, 4, 16);
  } else if (D == 64 && bits == 2) {
    KIVI_LAUNCH(64, 2, 8);
  } else {
    KIVI_LAUNCH(64, 4, 16);
  }
#undef KIVI_LAUNCH
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  return splitk_combine(a.o, units, D, st);
}

}  // extern "C"
