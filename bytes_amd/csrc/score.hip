// Token scoring: fp32 q.k scores of every cached key.
//
// Replaces src/attention_kernels.py:1077-1133 (`sparse_score_scalar`,
// scores[b, h, t] = (q[b, h] . k[b, h // G, t]) * scaling for bf16 keys) and
// adds the group-summed score of the token top-k pipeline,
// s[b, hk, t] = sum_{g < G} scores[b, hk*G + g, t] (g ascending), the
// selection score of one KV head shared by its query group.
//
// The query heads of a GQA group are scored together: one
// v_mfma_f32_16x16x32_bf16 computes S[h][t] for 16 heads x 16 tokens with
// A = Q (heads as rows) and B = K^T (tokens as columns).  Both operands use
// the same permutation of the contraction index: at k-step kk, lane l holds
// dims (kk*4 + l/16)*8 .. +8 of its row, so a lane's four k-steps cover 64
// contiguous bytes of one key row.  Key rows arrive whole-line (non-temporal
// loads) and are staged in the wave's LDS block, from which the B operands are
// read.  The output tile lands with head (l/16)*4 + i and token l%16 in lane
// l, so the group sum of up to four heads is a sum inside one lane.
//
// Group sums (and the per-head scores of fp8 keys and of D = 64 rows) are
// collected in an LDS score buffer over the workgroup's whole token range
// and leave in one burst of 16-byte stores after its last key load: a store
// issued between two batches of key loads would hold up every later wait
// for key rows until it is acknowledged.  The host sizes each workgroup's
// range to fit the buffer.
//
// fp8 (OCP e4m3fn) keys (`score_bits=8`, :1113) load 8 bytes per operand and
// are widened to bf16 exactly in registers.
//
// Packed 4/2-bit keys (`sparse_score_packed`, :1136-1222, layout of
// `quantize_and_pack_score_keys`, :1225-1249: codes along head_dim, element c
// at bits bits*(c % (8/bits)) of byte c // (8/bits), one bf16 scale/min per
// 32 dims) use a different row map: MFMA row m stands for the pair
// (group m / R, head m % R) with R = 16 / (D/32), and the A operand is q with
// every entry outside row m's group set to zero.  One MFMA chain then yields
// the per-group dot products (q . code)_g of R heads in separate rows, and
// each lane applies its own group's scale and min:
//   score = sum_g scale_g * (q . code)_g + min_g * (sum of q over group g).
// A lane's codes are one contiguous run of its row (D*bits/32 bytes, one
// load), all in one group.  Codes become bf16 operands by byte permutes
// against the constant 0x43: bf16 0x43cc is 128 + cc exactly, so the MFMA
// yields (q . code)_g + 128 * (sum of q)_g and the min term absorbs the
// offset as (min_g - 128 * scale_g).  The permute order of the codes inside
// an operand is applied to q as well.
#include "dense_tile.h"
#include "splitk.h"

namespace bytes_amd {

enum KeyMode : int { kKeyBf16 = 0, kKeyFp8 = 1, kKeyP4 = 2, kKeyP2 = 3 };

struct ScoreArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const void* k;             // bf16, fp8 e4m3fn or packed codes (strides in storage elements)
  int64_t k_sb, k_sh, k_ss;
  const uint16_t* ksc;       // packed keys: bf16 scale / min [B, Hk, S, D/32]
  const uint16_t* kmn;
  int64_t m_sb, m_sh, m_ss;
  float* out;                // [B, Hq, S] (per head) or [B, Hk, S] (group sum); unit stride along S
  int64_t o_sb, o_sh;
  uint32_t* hist;            // group sum only, optional: [B*Hk][2048] counts of the top 11 key bits
  int Hk, G, HPU, HB, S, tok_per_wg, parts, group_sum;   // HPU heads per unit, HB units per KV head
  float scaling;
};

constexpr int kScoreWaves = 4;
constexpr int kStoreBatch = 4;   // wave iterations whose group sums are emitted together
constexpr int kWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): every vector memory request done

// Per-head scores stored straight from the tile (packed keys, and dense keys
// with 256-byte rows) go through a buffer resource over the unit's output
// rows [row0, row0 + rows); a lane that must not store gets an offset past
// the resource (the store is dropped), so the store instruction is issued on
// every path.  (An LDS score buffer for packed keys took their workgroups
// from six to three per CU: int2 keys 75 -> 84 us at B32 H_q64 S16K.)
__device__ __forceinline__ void score_store(const ScoreArgs& a, int b, int row0, int rows, int r, int tok, bool ok,
                                            float v) {
  float* base = a.out + (int64_t)b * a.o_sb + (int64_t)row0 * a.o_sh;
  const uint32_t span = (uint32_t)(((int64_t)(rows - 1) * a.o_sh + a.S) * 4);
  const uint32_t off = ok ? (uint32_t)(((int64_t)r * a.o_sh + tok) * 4) : 0x80000000u;
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), buf_rsrc(base, span), (int)off, 0, kNonTemporal);
}

// Group-summed scores of 64 consecutive tokens, one per lane (lane l holds
// token tok = t + l), into the workgroup's LDS score buffer (which starts at
// token tb) and its histogram.
__device__ __forceinline__ void score_emit_sum64(const ScoreArgs& a, float tot, int tok, int tb, float* sbuf,
                                                 uint32_t* hlds) {
  if (tok < a.S) {
    sbuf[tok - tb] = tot;
    if (hlds) atomicAdd(&hlds[score_order_key(tot) >> 21], 1u);
  }
}

// Tokens of group sums one workgroup's LDS score buffer holds: what is left of
// a CU's 160 KB beside the key-row reservation and the 2048-bin histogram, in
// whole 256-token steps, at most 8192 (the host's largest workgroup range).
constexpr int score_sum_buf_tokens(int reserve) {
  const int t = (160 * 1024 - reserve - 2048 * 4) / 4 / 256 * 256;
  return t < 8192 ? t : 8192;
}

// LDS floats of the score buffer of a per-head policy: what is left of the
// workgroup's LDS budget beside its other LDS (the host keeps nh rows of a
// workgroup's token range within it).
constexpr int score_head_buf_floats(int budget, int other) { return (budget - other) / 4; }

// The workgroup's scores leave the LDS score buffer in one burst of
// non-temporal stores, 16 bytes per lane where a row is 16-byte aligned: rows
// row0 .. row0+rows-1 of the unit's output (the KV head's group-sum row, or
// the query heads' rows), buffer row r holding tokens tb .. tb+n-1 at
// sbuf[r * pitch ..].  Scores go to LDS during the loop and to memory only
// here because a store issued between two batches of key loads holds up
// every later wait for key rows until it is acknowledged (the memory counter
// completes in order): stored from the loop, even four iterations' group
// sums together, they cost 3.4% of the C5 score pass (339 against 327 us).
__device__ __forceinline__ void score_flush(const ScoreArgs& a, int b, int row0, int rows, int tb, int n, int pitch,
                                            const float* sbuf, int nthreads) {
  const int per_row = (n + 3) / 4;                 // 4-token pieces per row
  for (int e = threadIdx.x; e < rows * per_row; e += nthreads) {
    const int r = e / per_row, i = (e - r * per_row) * 4;
    float* row = a.out + (int64_t)b * a.o_sb + (int64_t)(row0 + r) * a.o_sh;
    const auto rs = buf_rsrc(row, (uint32_t)a.S * 4u);
    const float* src = sbuf + r * pitch + i;
    if (i + 4 <= n && ((reinterpret_cast<uintptr_t>(row + tb) | reinterpret_cast<uintptr_t>(src)) & 15) == 0) {
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4*>(src), rs, (tb + i) * 4, 0, kNonTemporal);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (i + q < n) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(src[q]), rs, (tb + i + q) * 4, 0, kNonTemporal);
    }
  }
}

// ---- bf16 / fp8 keys ------------------------------------------------------

template <int D, bool FP8, bool GS>
struct DenseKeys {
  static constexpr int CT = 4;                 // 16-token column tiles per wave iteration
  static constexpr int ES = FP8 ? 1 : 2;       // bytes per key element
  static constexpr int CPR = D * ES / 16;      // 16-byte chunks per key row
  // One iteration's 64 key rows are read whole-line (consecutive lanes,
  // consecutive 16-byte chunks of a row; non-temporal) and staged in the
  // wave's LDS block, chunk c of row r at slot c ^ (r % CPR), where the MFMA
  // B operands are read from: the 16 rows one operand read touches sit in
  // distinct slots.  (Reading the operands straight from memory splits each
  // row's 128-byte lines over several instructions, which the non-temporal
  // hint turns into refetches.)
  static constexpr int kWaveLds = 64 * D * ES;
  static constexpr int kLds = kScoreWaves * kWaveLds;
  // LDS reserved per workgroup.  With 256-byte rows two resident workgroups
  // would keep 256 KB of key rows in flight per CU; one (128 KB) streams
  // faster (C5: 336 against 347 us per score pass), so the reservation
  // leaves room for only one.  Narrower rows keep two (128 KB in flight).
  static constexpr bool kOneWg = D * ES >= 256;
  static constexpr int kLdsReserve = kOneWg ? 2 * kLds : kLds;
  static_assert(kLdsReserve + 2048 * 4 <= 160 * 1024, "the reservation and the histogram fit a CU's LDS");
  // Per-head scores of narrower rows (fp8, or D = 64) go through an LDS score
  // buffer too, a row per head, filling the two workgroups' share of LDS:
  // B32 H_q64 fp8 keys 138 -> 133 us at S16K, 42 -> 36 us at S4K.  With
  // 256-byte rows (one workgroup per CU) the end-of-range flush cost more than
  // it saved at S4K (bf16 67 -> 71 us), so those store from the tile.
  static constexpr bool kHeadBuf = !GS && !kOneWg;
  // LDS score buffer, in floats: group sums, one row of the workgroup's
  // tokens; per-head scores, a row per head (the host keeps a workgroup's
  // range within it)
  static constexpr int kSumBuf = GS ? score_sum_buf_tokens(kLdsReserve)
                                    : (kHeadBuf ? score_head_buf_floats(80 * 1024, kLdsReserve) : 4);
  static_assert(!GS || kSumBuf >= 1024, "room for a useful workgroup range");
  static_assert(!kHeadBuf || kSumBuf >= 8 * 1024, "room for sixteen heads of a 512-token range");
  float* hbuf;                 // per-head scores: the LDS score buffer, rows of hpitch tokens from htb
  int hpitch, htb;
  struct Regs {
    u32x4 k[CPR];            // chunk lane + 64 i: row (lane + 64 i) / CPR, chunk (lane + 64 i) % CPR
  };
  const uint8_t* kbase;         // the unit's key rows
  uint32_t row_bytes;          // bytes per token row
  char* kst;                   // this wave's LDS block
  bf16x8 qa[D / 32];

  __device__ __forceinline__ void init(const ScoreArgs& a, int b, int hk, int hq0, int nh, int lane) {
    const int l16 = lane & 15, lg = lane >> 4;
    row_bytes = (uint32_t)(a.k_ss * ES);
    kbase = static_cast<const uint8_t*>(a.k) + ((int64_t)b * a.k_sb + (int64_t)hk * a.k_sh) * ES;
    // Q as the A operand: lane holds Q[h = l16][dims (kk*4 + lg)*8 .. +8]
    const bool live = l16 < nh;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hq0 + (live ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk)
      qa[kk] = __builtin_bit_cast(bf16x8, ld16_live(qp + kk * 32, live));
  }

  // K rows t .. t+63 of one iteration, whole rows per load instruction,
  // through a buffer resource that starts at row t (wave-uniform) and ends at
  // row lim (<= S), so rows at or past lim read zero without a memory access
  // and the per-lane offsets are the same in every iteration.
  __device__ __forceinline__ void issue(const ScoreArgs& a, int t, int lim, int lane, Regs& r) const {
    const auto rk = buf_rsrc(kbase + (uint64_t)(uint32_t)t * row_bytes,
                             (uint32_t)(t < lim ? lim - t : 0) * row_bytes);
#pragma unroll
    for (int i = 0; i < CPR; ++i) {
      const int p = lane + 64 * i;
      const uint32_t off = (uint32_t)(p / CPR) * row_bytes + (uint32_t)(p % CPR) * 16;
      r.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)off, 0, kNonTemporal));
    }
  }

  static __device__ __forceinline__ bf16x8 operand(const u32x4& w) { return __builtin_bit_cast(bf16x8, w); }
  static __device__ __forceinline__ bf16x8 operand(const u32x2& w) {
    const u32x4 b = {fp8x2_to_bf16x2<false>(w[0]), fp8x2_to_bf16x2<true>(w[0]), fp8x2_to_bf16x2<false>(w[1]),
                     fp8x2_to_bf16x2<true>(w[1])};
    return __builtin_bit_cast(bf16x8, b);
  }

  // Group sums are returned (token t + lane per lane) for the driver to
  // store; per-head scores are stored here.
  static constexpr bool kDeferStore = GS;

  __device__ __forceinline__ float tile(const ScoreArgs& a, const Regs& r, int t, int lane, int b, int hk, int hq0,
                                        int nh, uint32_t* hlds) const {
    const int l16 = lane & 15, lg = lane >> 4;
    wave_lds_sync();                             // the previous iteration's operand reads are done
#pragma unroll
    for (int i = 0; i < CPR; ++i) {
      const int p = lane + 64 * i;
      const int row = p / CPR, ch = p % CPR;
      *reinterpret_cast<u32x4*>(kst + (row * CPR + (ch ^ (row % CPR))) * 16) = r.k[i];
    }
    wave_lds_sync();
    float keep = 0.f;                            // group sum: lane group lg keeps column tile lg's
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = c * 16 + l16;
      const char* rp = kst + row * CPR * 16;
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        if constexpr (FP8) {
          // dims (kk*4 + lg)*8 .. +8: 8 bytes, half lg & 1 of chunk kk*2 + lg/2
          const int ch = kk * 2 + (lg >> 1);
          const u32x2 w = *reinterpret_cast<const u32x2*>(rp + (ch ^ (row % CPR)) * 16 + (lg & 1) * 8);
          s = mfma_bf16(qa[kk], operand(w), s);
        } else {
          const int ch = kk * 4 + lg;
          const u32x4 w = *reinterpret_cast<const u32x4*>(rp + (ch ^ (row % CPR)) * 16);
          s = mfma_bf16(qa[kk], operand(w), s);
        }
      }
      const int tok = t + c * 16 + l16;
      if constexpr (GS) {
        // heads lg*4 + i summed in head order per lane, then the four lane
        // groups of the column folded by row swaps
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (lg * 4 + i < nh) part += s[i] * a.scaling;
        const float tot = col_sum4(part);
        keep = lg == c ? tot : keep;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = lg * 4 + i;
          if constexpr (kHeadBuf) {
            if (h < nh && tok < a.S) hbuf[h * hpitch + (tok - htb)] = s[i] * a.scaling;
          } else {
            score_store(a, b, hq0, nh, h, tok, h < nh && tok < a.S, s[i] * a.scaling);
          }
        }
      }
    }
    return keep;
  }
};

// ---- packed 4/2-bit keys --------------------------------------------------

// Position, inside its run of 8 codes, of the code that lands in operand
// element j after the byte permutes below (applied to q the same way).
__device__ __forceinline__ int packed_perm(int bits, int j) {
  return bits == 4 ? ((j & 3) * 2 + (j >> 2)) : ((j >> 1) + (j & 1) * 4);
}

constexpr uint32_t kBf16Hi128 = 0x43434343u;   // high byte of bf16 128 + cc (cc < 128)
constexpr uint32_t kSelLo = 0x04010400u;       // [x.b0, 0x43, x.b1, 0x43]
constexpr uint32_t kSelHi = 0x04030402u;       // [x.b2, 0x43, x.b3, 0x43]

template <int D, int BITS, int NB, bool GS>
struct PackedKeys {
  static constexpr int NG = D / 32;            // groups per row = MFMA k-steps
  static constexpr int R = 16 / NG;            // MFMA rows per group
  static constexpr int LB = D * BITS / 32;     // bytes of one row per lane (D/4 codes)
  static constexpr int NW = LB / 4;            // 32-bit words per lane
  static constexpr int CT = 4;                 // 16-token column tiles per wave iteration (64 tokens)
  typedef typename std::conditional<NW == 4, u32x4, typename std::conditional<NW == 2, u32x2, uint32_t>::type>::type T;
  typedef typename std::conditional<NG == 4, u32x2, uint32_t>::type SR;
  struct Regs {
    T k[CT];                                   // [column tile]
    SR srow, mrow;                             // scale / min row (NG bf16) of token t + lane
  };
  static constexpr int kLds = 16;              // operands come straight from registers
  static constexpr int kLdsReserve = kLds;
  // group sums are returned by tile() (token t + lane per lane) and collected
  // by the driver; per-head scores are stored by tile()
  static constexpr bool kDeferStore = GS;
  // LDS score buffer of group sums (as for dense keys); per-head scores are
  // stored by tile().  2-bit keys keep it at 4096 tokens, so more
  // workgroups fit a CU (C5 int2 score pass 95 -> 88 us; 4-bit keys ran
  // 1% slower with it, and both slower at 2048).
  static constexpr int kSumBuf =
      GS ? (BITS == 2 ? 4096 : score_sum_buf_tokens(kLdsReserve + kScoreWaves * 64 * NG * 4)) : 4;
  static constexpr bool kHeadBuf = false;
  char* kst;
  // One KV head's codes and scale/min rows, addressed through buffer
  // resources: every load is a 32-bit lane offset plus a uniform row offset,
  // and rows at or past S read as zero (their scores are not stored); an
  // issue at or past its range limit reads nothing.
  const uint8_t* kb;
  const uint16_t *scb, *mnb;
  uint32_t kspan, mspan;
  uint32_t koff;                               // lane part of the code offsets (bytes)
  uint32_t k_row, m_row;                       // row strides (bytes)
  bf16x8 qa[NB][NG];                           // [row block][k-step]
  f32x4 qsum[NB];                              // sum of q over the lane's group, rows lg*4 + i

  // 8 bf16 values (raw bits) reordered into operand order
  static __device__ __forceinline__ bf16x8 permute_q(const uint16_t (&e)[8]) {
    uint16_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = e[packed_perm(BITS, j)];
    const u32x4 w = {o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16), o[4] | ((uint32_t)o[5] << 16),
                     o[6] | ((uint32_t)o[7] << 16)};
    return __builtin_bit_cast(bf16x8, w);
  }

  __device__ __forceinline__ void init(const ScoreArgs& a, int b, int hk, int hq0, int nh, int lane) {
    const int l16 = lane & 15, lg = lane >> 4;
    const int grp = lg * NG / 4;
    k_row = (uint32_t)a.k_ss;
    m_row = (uint32_t)a.m_ss * 2;
    kspan = (uint32_t)((a.S - 1) * a.k_ss + LB * 4);
    mspan = (uint32_t)(((a.S - 1) * a.m_ss + NG) * 2);
    kb = static_cast<const uint8_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
    scb = a.ksc + (int64_t)b * a.m_sb + (int64_t)hk * a.m_sh;
    mnb = a.kmn + (int64_t)b * a.m_sb + (int64_t)hk * a.m_sh;
    koff = (uint32_t)l16 * k_row + lg * LB;
    const bool in_group = (l16 / R) == grp;
    const uint16_t* qrow = a.q + (int64_t)b * a.q_sb + lg * (D / 4);
    if constexpr (GS) {
      // group sum: rows (group, 0) and (group, 1) hold the bf16 high and low
      // parts of sum_h q_h; the other rows are zero
      const int slot = l16 % R;
#pragma unroll
      for (int kk = 0; kk < NG; ++kk) {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int h = 0; h < nh; ++h) {
          const u32x4 raw = ld16(qrow + (int64_t)(hq0 + h) * a.q_sh + kk * 8);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[2 * j] += __uint_as_float(raw[j] << 16);
            acc[2 * j + 1] += __uint_as_float(raw[j] & 0xFFFF0000u);
          }
        }
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint16_t hi = f32_to_bf16_bits(acc[j]);
          const uint16_t lo = f32_to_bf16_bits(acc[j] - bf16_bits_to_f32(hi));
          e[j] = !in_group ? (uint16_t)0 : (slot == 0 ? hi : (slot == 1 ? lo : (uint16_t)0));
        }
        qa[0][kk] = permute_q(e);
      }
    } else {
      // per head: row m = (group m / R, head m % R) of block nb
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int h = nb * R + l16 % R;
        const bool live = in_group && h < nh;
        const uint16_t* qp = qrow + (int64_t)(hq0 + (live ? h : 0)) * a.q_sh;
#pragma unroll
        for (int kk = 0; kk < NG; ++kk) {
          const u32x4 raw = ld16_live(qp + kk * 8, live);
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            e[2 * j] = (uint16_t)(raw[j] & 0xFFFFu);
            e[2 * j + 1] = (uint16_t)(raw[j] >> 16);
          }
          qa[nb][kk] = permute_q(e);
        }
      }
    }
    const u32x4 one = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0 x 8
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NG; ++kk) s = mfma_bf16(qa[nb][kk], __builtin_bit_cast(bf16x8, one), s);
      qsum[nb] = s;
    }
  }

  // rows t .. t+63; t and lim are wave-uniform, and t >= lim reads nothing
  __device__ __forceinline__ void issue(const ScoreArgs& a, int t, int lim, int lane, Regs& r) const {
    const bool live = t < lim;
    const auto rk = buf_rsrc(kb, live ? kspan : 0u);
    const auto rsc = buf_rsrc(scb, live ? mspan : 0u);
    const auto rmn = buf_rsrc(mnb, live ? mspan : 0u);
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const uint32_t row = (uint32_t)(t + c * 16);                  // wave-uniform
      const uint32_t ko = koff + row * k_row;
      if constexpr (NW == 4)
        r.k[c] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0);
      else if constexpr (NW == 2)
        r.k[c] = __builtin_amdgcn_raw_buffer_load_b64(rk, ko, 0, 0);
      else
        r.k[c] = __builtin_amdgcn_raw_buffer_load_b32(rk, ko, 0, 0);
    }
    // scale and min rows of the iteration's 64 tokens, one row per lane; the
    // tile hands each lane its (token, group) entry through LDS
    const uint32_t so = ((uint32_t)t + lane) * m_row;
    if constexpr (NG == 4) {
      r.srow = __builtin_amdgcn_raw_buffer_load_b64(rsc, so, 0, 0);
      r.mrow = __builtin_amdgcn_raw_buffer_load_b64(rmn, so, 0, 0);
    } else {
      r.srow = __builtin_amdgcn_raw_buffer_load_b32(rsc, so, 0, 0);
      r.mrow = __builtin_amdgcn_raw_buffer_load_b32(rmn, so, 0, 0);
    }
  }

  static __device__ __forceinline__ uint32_t word(const T& v, int i) {
    if constexpr (NW == 1)
      return v;
    else
      return v[i];
  }

  // the lane's D/4 codes as NG operands of 8 bf16 values 128 + code
  static __device__ __forceinline__ void operands(const T& v, bf16x8 (&op)[NG]) {
    if constexpr (BITS == 4) {
#pragma unroll
      for (int kk = 0; kk < NG; ++kk) {
        const uint32_t w = word(v, kk);
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        const u32x4 o = {__builtin_amdgcn_perm(kBf16Hi128, lo, kSelLo), __builtin_amdgcn_perm(kBf16Hi128, lo, kSelHi),
                         __builtin_amdgcn_perm(kBf16Hi128, hi, kSelLo), __builtin_amdgcn_perm(kBf16Hi128, hi, kSelHi)};
        op[kk] = __builtin_bit_cast(bf16x8, o);
      }
    } else {
#pragma unroll
      for (int wi = 0; wi < NG / 2; ++wi) {
        const uint32_t w = word(v, wi);
        const uint32_t x0 = w & 0x03030303u, x1 = (w >> 2) & 0x03030303u;
        const uint32_t x2 = (w >> 4) & 0x03030303u, x3 = (w >> 6) & 0x03030303u;
        const u32x4 lo = {__builtin_amdgcn_perm(kBf16Hi128, x0, kSelLo), __builtin_amdgcn_perm(kBf16Hi128, x1, kSelLo),
                          __builtin_amdgcn_perm(kBf16Hi128, x2, kSelLo), __builtin_amdgcn_perm(kBf16Hi128, x3, kSelLo)};
        const u32x4 hi = {__builtin_amdgcn_perm(kBf16Hi128, x0, kSelHi), __builtin_amdgcn_perm(kBf16Hi128, x1, kSelHi),
                          __builtin_amdgcn_perm(kBf16Hi128, x2, kSelHi), __builtin_amdgcn_perm(kBf16Hi128, x3, kSelHi)};
        op[2 * wi] = __builtin_bit_cast(bf16x8, lo);
        op[2 * wi + 1] = __builtin_bit_cast(bf16x8, hi);
      }
    }
  }

  __device__ __forceinline__ float tile(const ScoreArgs& a, const Regs& r, int t, int lane, int b, int hk, int hq0,
                                        int nh, uint32_t* hlds) const {
    const int l16 = lane & 15, lg = lane >> 4;
    float keep = 0.f;                          // group sum: lane group lg keeps column tile lg's
    // per wave: [token][group] words (bf16 scale low, bf16 min high)
    __shared__ uint32_t sm_lds[kScoreWaves][64 * NG];
    uint32_t* my = sm_lds[threadIdx.x >> 6];
    {
      uint32_t wv[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        uint32_t sw, mw;
        if constexpr (NG == 4) {
          sw = r.srow[g >> 1];
          mw = r.mrow[g >> 1];
        } else {
          sw = r.srow;
          mw = r.mrow;
        }
        wv[g] = (g & 1) ? __builtin_amdgcn_perm(mw, sw, 0x07060302u) : __builtin_amdgcn_perm(mw, sw, 0x05040100u);
      }
      wave_lds_sync();                         // the previous iteration's reads are done
      if constexpr (NG == 4)
        *reinterpret_cast<u32x4*>(my + lane * 4) = u32x4{wv[0], wv[1], wv[2], wv[3]};
      else
        *reinterpret_cast<u32x2*>(my + lane * 2) = u32x2{wv[0], wv[1]};
      wave_lds_sync();
    }
    const int grp = lg * NG / 4;
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      bf16x8 op[NG];
      operands(r.k[c], op);
      const uint32_t smc = my[(c * 16 + l16) * NG + grp];
      const float sc = __uint_as_float(smc << 16);
      const float mn = __uint_as_float(smc & 0xFFFF0000u);
      const float mn128 = fmaf(-128.f, sc, mn);
      const int tok = t + c * 16 + l16;
      if constexpr (GS) {
        f32x4 g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NG; ++kk) g = mfma_bf16(qa[0][kk], op[kk], g);
        // rows (group, 0/1) carry the high/low parts of the summed query; others are zero
        float v = fmaf(sc, g[0] + g[1], mn128 * (qsum[0][0] + qsum[0][1]));
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        keep = lg == c ? v * a.scaling : keep;
      } else {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < NG; ++kk) g = mfma_bf16(qa[nb][kk], op[kk], g);
          float p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = fmaf(sc, g[i], mn128 * qsum[nb][i]);
          if constexpr (NG == 4) {
            // lane group lg holds group lg of heads 0..3; reduce-scatter so that it ends with head lg
            const bool up = lg >= 2;
            const float k0 = up ? p[2] : p[0], k1 = up ? p[3] : p[1];
            const float s0 = up ? p[0] : p[2], s1 = up ? p[1] : p[3];
            const float a0 = k0 + __shfl_xor(s0, 32, 64), a1 = k1 + __shfl_xor(s1, 32, 64);
            const bool odd = lg & 1;
            const float tot = (odd ? a1 : a0) + __shfl_xor(odd ? a0 : a1, 16, 64);
            const int h = nb * R + lg;
            score_store(a, b, hq0, nh, h, tok, h < nh && tok < a.S, tot * a.scaling);
          } else {
            // lane groups lg and lg^2 hold groups 0 and 1 of heads (lg&1)*4 + i
            float tot[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) tot[i] = p[i] + __shfl_xor(p[i], 32, 64);
            const int i0 = (lg >> 1) * 2;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int h = nb * R + (lg & 1) * 4 + i0 + u;
              const float val = i0 ? tot[2 + u] : tot[u];
              score_store(a, b, hq0, nh, h, tok, h < nh && tok < a.S, val * a.scaling);
            }
          }
        }
      }
    }
    return keep;
  }
};

// ---- driver ---------------------------------------------------------------

// The register budget is that of two workgroups per CU; policies whose LDS
// reservation holds a CU to one workgroup make the compiler report the
// missed occupancy target, which is intended there.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <class P>
__global__ __launch_bounds__(kScoreWaves * 64, 2) void score_kernel(ScoreArgs a) {
  PREFETCH_ARGS(a);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int unit = blockIdx.x / a.parts, part = blockIdx.x - unit * a.parts;
  const int b = unit / (a.Hk * a.HB);
  const int rem = unit - b * a.Hk * a.HB;
  const int hk = rem / a.HB, hb = rem - (rem / a.HB) * a.HB;
  const int hq0 = hk * a.G + hb * a.HPU;
  const int nh = min(a.HPU, a.G - hb * a.HPU);
  P pol;
  pol.init(a, b, hk, hq0, nh, lane);
  __shared__ __attribute__((aligned(16))) char kst_mem[P::kLdsReserve];
  pol.kst = kst_mem + w * (P::kLds / kScoreWaves);

  const int t_begin = part * a.tok_per_wg;
  const int t_end = min(t_begin + a.tok_per_wg, a.S);
  constexpr int STEP = kScoreWaves * 16 * P::CT;
  __shared__ uint32_t hlds_mem[P::kDeferStore ? 2048 : 1];   // histogram: group sums only
  __shared__ __attribute__((aligned(16))) float sbuf[P::kSumBuf];
  if constexpr (P::kHeadBuf) {
    pol.hbuf = sbuf;
    pol.hpitch = a.tok_per_wg;
    pol.htb = t_begin;
  }
  uint32_t* hlds = nullptr;
  if constexpr (P::kDeferStore) {
    if (a.hist) {
      for (int i = threadIdx.x; i < 2048; i += kScoreWaves * 64) hlds_mem[i] = 0u;
      __syncthreads();
      hlds = hlds_mem;
    }
  }
  constexpr int ITER = 16 * P::CT;
  // wave-uniform (the compiler cannot see it from threadIdx), so the loop runs
  // on scalar branches rather than an exec-mask loop
  int t = __builtin_amdgcn_readfirstlane(t_begin + w * ITER);
  if (t < t_end) {
    // two register sets: the next iteration's rows are in flight while one is
    // scored.  The scheduling barriers keep each request batch ahead of the
    // tile that follows it (left alone, the compiler moves the requests below
    // the tile's first use of the current rows, so only one batch is ever in
    // flight).
    typename P::Regs r0, r1;
    pol.issue(a, t, t_end, lane, r0);
    if constexpr (P::kDeferStore) {
      // Group sums go to the LDS score buffer, kStoreBatch iterations' worth
      // together, and to memory after the loop (score_flush).
      static_assert(kStoreBatch % 2 == 0, "the register sets alternate within a batch");
      // one iteration: the next rows are requested (past the range the
      // resource has zero length, so the last step's requests read nothing
      // and return at once), the current rows scored; false at the range end
      auto step = [&](float& sc, typename P::Regs& cur, typename P::Regs& nxt) {
        const bool more = t + STEP < t_end;
        pol.issue(a, t + STEP, t_end, lane, nxt);
        __builtin_amdgcn_sched_barrier(0);
        sc = pol.tile(a, cur, t, lane, b, hk, hq0, nh, hlds);
        // finished here: left alone, the compiler sinks each tile's group sums
        // down to the emits, past the next batch's loads, and then needs
        // registers that those loads are still filling
        asm volatile("" : "+v"(sc));
        t += STEP;
        return more;
      };
      // Each exit waits for its last (empty) requests in a block of its own,
      // so no path reaches the emits with requests of the next batch still
      // counted.
      while (true) {
        float sc[kStoreBatch];
        const int t0 = t;
        int n = 0;
#pragma unroll
        for (int j = 0; j < kStoreBatch; j += 2) {
          if (!step(sc[j], r0, r1)) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            n = j + 1;
            break;
          }
          if (!step(sc[j + 1], r1, r0)) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            n = j + 2;
            break;
          }
        }
        if (n == 0) {
#pragma unroll
          for (int j = 0; j < kStoreBatch; ++j) score_emit_sum64(a, sc[j], t0 + j * STEP + lane, t_begin, sbuf, hlds);
          continue;
        }
#pragma unroll
        for (int j = 0; j < kStoreBatch; ++j)
          if (j < n) score_emit_sum64(a, sc[j], t0 + j * STEP + lane, t_begin, sbuf, hlds);
        break;
      }
    } else while (true) {
      const bool more1 = t + STEP < t_end;
      pol.issue(a, more1 ? t + STEP : t, a.S, lane, r1);
      __builtin_amdgcn_sched_barrier(0);
      pol.tile(a, r0, t, lane, b, hk, hq0, nh, hlds);
      t += STEP;
      if (!more1) break;
      const bool more0 = t + STEP < t_end;
      pol.issue(a, more0 ? t + STEP : t, a.S, lane, r0);
      __builtin_amdgcn_sched_barrier(0);
      pol.tile(a, r1, t, lane, b, hk, hq0, nh, hlds);
      t += STEP;
      if (!more0) break;
    }
  }
  if constexpr (P::kDeferStore) {
    __syncthreads();
    score_flush(a, b, hk, 1, t_begin, t_end - t_begin, 0, sbuf, kScoreWaves * 64);
  } else if constexpr (P::kHeadBuf) {
    __syncthreads();
    score_flush(a, b, hq0, nh, t_begin, t_end - t_begin, a.tok_per_wg, sbuf, kScoreWaves * 64);
  }
  if constexpr (P::kDeferStore) {
    if (a.hist) {
      __syncthreads();
      uint32_t* hr = a.hist + ((int64_t)b * a.Hk + hk) * 2048;
      for (int i = threadIdx.x; i < 2048; i += kScoreWaves * 64)
        if (hlds_mem[i]) atomicAdd(hr + i, hlds_mem[i]);
    }
  }
}

#pragma clang diagnostic pop

template <int D, bool FP8>
static void launch_dense(const dim3& g, const dim3& blk, hipStream_t st, const ScoreArgs& a) {
  if (a.group_sum)
    BYTES_LAUNCH(kProfScore, (score_kernel<DenseKeys<D, FP8, true>>), g, blk, 0, st, a);
  else
    BYTES_LAUNCH(kProfScore, (score_kernel<DenseKeys<D, FP8, false>>), g, blk, 0, st, a);
}

template <int D, int BITS>
static void launch_packed(const dim3& g, const dim3& blk, hipStream_t st, const ScoreArgs& a, int nb) {
  if (a.group_sum) {
    BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<D, BITS, 1, true>>), g, blk, 0, st, a);
  } else if constexpr (D == 128) {
    if (nb == 1) BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<128, BITS, 1, false>>), g, blk, 0, st, a);
    else if (nb == 2) BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<128, BITS, 2, false>>), g, blk, 0, st, a);
    else BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<128, BITS, 4, false>>), g, blk, 0, st, a);
  } else {
    if (nb == 1) BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<64, BITS, 1, false>>), g, blk, 0, st, a);
    else BYTES_LAUNCH(kProfScore, (score_kernel<PackedKeys<64, BITS, 2, false>>), g, blk, 0, st, a);
  }
}

}  // namespace bytes_amd

using namespace bytes_amd;

extern "C" {

int bytes_sparse_score(const void* q, const void* k, int k_mode, const void* k_scale, const void* k_min, void* out,
                       int B, int Hq, int Hk, int S, int D, int group_sum, int64_t q_sb, int64_t q_sh, int64_t k_sb,
                       int64_t k_sh, int64_t k_ss, int64_t m_sb, int64_t m_sh, int64_t m_ss, int64_t o_sb,
                       int64_t o_sh, float scaling, void* hist, void* stream) {
  if (!q || !k || !out || B <= 0 || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || S <= 0) return (int)hipErrorInvalidValue;
  if (D != 64 && D != 128) return (int)hipErrorInvalidValue;
  if (k_mode < kKeyBf16 || k_mode > kKeyP2) return (int)hipErrorInvalidValue;
  const bool packed = k_mode >= kKeyP4;
  if (packed && (!k_scale || !k_min)) return (int)hipErrorInvalidValue;
  ScoreArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.ksc = static_cast<const uint16_t*>(k_scale);
  a.kmn = static_cast<const uint16_t*>(k_min);
  a.m_sb = m_sb; a.m_sh = m_sh; a.m_ss = m_ss;
  a.out = static_cast<float*>(out);
  a.o_sb = o_sb; a.o_sh = o_sh;
  a.hist = static_cast<uint32_t*>(hist);
  a.Hk = Hk; a.G = Hq / Hk; a.S = S;
  // packed keys: heads per row block R = 16 / (D/32); 1, 2 or 4 blocks per unit share the code widening
  int nb = 1;
  if (packed && !group_sum) {
    const int R = 16 / (D / 32), nbmax = 16 / R;
    nb = (a.G + R - 1) / R;
    nb = nb <= 1 ? 1 : (nb <= 2 ? 2 : 4);
    if (nb > nbmax) nb = nbmax;
    a.HPU = R * nb;
  } else {
    a.HPU = 16;                  // bf16/fp8 keys; packed group sums fold every head of the group into q
  }
  if (packed) {
    // one KV head's codes and scale/min rows are addressed with 32-bit offsets
    const int64_t kspan = (int64_t)(S - 1) * k_ss + D * (k_mode == kKeyP4 ? 4 : 2) / 8;
    const int64_t mspan = ((int64_t)(S - 1) * m_ss + D / 32) * 2;
    // (a wave's last iteration reads up to 63 rows past S - 1)
    if (k_ss <= 0 || m_ss <= 0 || kspan + 64L * k_ss >= (1LL << 32) || mspan + 128L * m_ss >= (1LL << 32))
      return (int)hipErrorNotSupported;
  }
  a.HB = (a.G + a.HPU - 1) / a.HPU;
  a.group_sum = group_sum ? 1 : 0;
  if (a.group_sum && a.G > 16) return (int)hipErrorNotSupported;
  if (a.hist && !a.group_sum) return (int)hipErrorInvalidValue;
  // each unit's output rows must fit one buffer resource with room for the
  // out-of-range offset of dropped stores, and (dense keys) the unit's key
  // rows plus one iteration of 64 rows must stay below 2^32 bytes of offset
  if (((int64_t)((a.group_sum ? 1 : a.HPU) - 1) * o_sh + S) * 4 >= ((int64_t)1 << 31))
    return (int)hipErrorNotSupported;
  if ((k_mode == kKeyBf16 || k_mode == kKeyFp8) &&
      ((int64_t)S + 64) * k_ss * (k_mode == kKeyBf16 ? 2 : 1) >= ((int64_t)1 << 32))
    return (int)hipErrorNotSupported;
  a.scaling = scaling;
  const long units = (long)B * Hk * a.HB;
  // about 8 workgroups per CU in total (eight rounds of one resident with
  // 256-byte key rows, four of two otherwise), each a multiple of one
  // iteration of all waves: fine enough that the last round's uneven finish
  // costs little
  const long target = 8L * device_cu_count();
  const int step = kScoreWaves * 64;
  long per = ((long)S * units + target - 1) / target;
  per = (per + step - 1) / step * step;
  if (per < step) per = step;
  // a workgroup's range fits its LDS score buffer: one row of group sums, or
  // a row per query head of the unit
  static_assert(PackedKeys<64, 2, 1, true>::kSumBuf == PackedKeys<128, 2, 1, true>::kSumBuf &&
                    PackedKeys<64, 4, 1, true>::kSumBuf >= PackedKeys<128, 4, 1, true>::kSumBuf,
                "packed group-sum buffers of D = 64 hold at least the D = 128 ones");
  static_assert(!DenseKeys<128, false, false>::kHeadBuf && DenseKeys<128, true, false>::kHeadBuf &&
                    DenseKeys<64, false, false>::kHeadBuf && DenseKeys<64, true, false>::kHeadBuf,
                "which per-head policies buffer their scores");
  long buf;
  const bool bf = k_mode == kKeyBf16;
  if (packed)
    buf = k_mode == kKeyP2 ? PackedKeys<128, 2, 1, true>::kSumBuf    // group sums (per-head
                           : PackedKeys<128, 4, 1, true>::kSumBuf;   // scores are stored directly)
  else if (a.group_sum)
    buf = D == 128 ? (bf ? DenseKeys<128, false, true>::kSumBuf : DenseKeys<128, true, true>::kSumBuf)
                   : (bf ? DenseKeys<64, false, true>::kSumBuf : DenseKeys<64, true, true>::kSumBuf);
  else if (D == 128 && bf)
    buf = 8192;                              // per-head scores are stored directly
  else
    buf = (D == 128 ? DenseKeys<128, true, false>::kSumBuf
                    : (bf ? DenseKeys<64, false, false>::kSumBuf : DenseKeys<64, true, false>::kSumBuf)) /
          (a.HPU < a.G ? a.HPU : a.G);       // a row per head of the unit
  long cap = buf / step * step;
  if (cap > 8192) cap = 8192;
  if (per > cap) per = cap;
  a.tok_per_wg = (int)per;
  a.parts = (int)((S + per - 1) / per);
  const long grid = units * a.parts;
  if (grid > 0x7FFFFFFFL) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)grid), blk(kScoreWaves * 64);
  if (D == 128) {
    switch (k_mode) {
      case kKeyBf16: launch_dense<128, false>(g, blk, st, a); break;
      case kKeyFp8: launch_dense<128, true>(g, blk, st, a); break;
      case kKeyP4: launch_packed<128, 4>(g, blk, st, a, nb); break;
      default: launch_packed<128, 2>(g, blk, st, a, nb); break;
    }
  } else {
    switch (k_mode) {
      case kKeyBf16: launch_dense<64, false>(g, blk, st, a); break;
      case kKeyFp8: launch_dense<64, true>(g, blk, st, a); break;
      case kKeyP4: launch_packed<64, 4>(g, blk, st, a, nb); break;
      default: launch_packed<64, 2>(g, blk, st, a, nb); break;
    }
  }
  return (int)hipGetLastError();
}

// Quantize and pack score keys along head_dim (src/attention_kernels.py:1225-1249):
// per row and group of 32, scale = max(hi - lo, 1e-8) / (2^bits - 1) and
// code = clamp(rint((x - lo) / scale)) in fp32; scale and lo stored in x's
// dtype (round to nearest even).
__device__ __forceinline__ void store_as(void* p, int64_t i, int dtype, float v) {
  if (dtype == 0)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else if (dtype == 1)
    static_cast<_Float16*>(p)[i] = (_Float16)v;
  else
    static_cast<float*>(p)[i] = v;
}

__global__ void score_pack_kernel(const void* x, int x_dtype, int64_t rows, int D, int64_t x_rs, int bits,
                                  uint8_t* packed, void* scale, void* mn) {
  const int ng = D / 32;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * ng) return;
  const int64_t row = gid / ng;
  const int g = (int)(gid - row * ng);
  const int64_t base = row * x_rs + g * 32;
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    v[i] = x_dtype == 0 ? bf16_bits_to_f32(static_cast<const uint16_t*>(x)[base + i])
                        : (x_dtype == 1 ? (float)static_cast<const _Float16*>(x)[base + i]
                                        : static_cast<const float*>(x)[base + i]);
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
  const int levels = 1 << bits;
  const float s = fmaxf(hi - lo, 1e-8f) / (float)(levels - 1);
  const int per = 8 / bits;
  uint8_t* out = packed + row * (int64_t)(D * bits / 8) + g * (32 * bits / 8);
  for (int byte = 0; byte < 32 / per; ++byte) {
    uint32_t w = 0;
    for (int i = 0; i < per; ++i) {
      float c = rintf((v[byte * per + i] - lo) / s);
      c = fminf(fmaxf(c, 0.f), (float)(levels - 1));
      w |= (uint32_t)c << (i * bits);
    }
    out[byte] = (uint8_t)w;
  }
  store_as(scale, row * ng + g, x_dtype, s);
  store_as(mn, row * ng + g, x_dtype, lo);
}

int bytes_score_keys_pack(const void* x, int x_dtype, int64_t rows, int D, int64_t x_row_stride, int bits,
                          void* packed, void* scale, void* mn, void* stream) {
  if (!x || !packed || !scale || !mn || rows < 0 || D <= 0 || D % 32 != 0 || (bits != 4 && bits != 2) ||
      x_dtype < 0 || x_dtype > 2)
    return (int)hipErrorInvalidValue;
  const int64_t n = rows * (D / 32);
  if (n == 0) return 0;
  const int th = 256;
  hipLaunchKernelGGL(score_pack_kernel, dim3((unsigned)((n + th - 1) / th)), dim3(th), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, rows, D, x_row_stride, bits,
                     static_cast<uint8_t*>(packed), scale, mn);
  return (int)hipGetLastError();
}

}  // extern "C"
