/*
 * bytes_amd C ABI: the MI355X (gfx950) decode-attention hot path of the
 * saifmb0/bytes KV-cache study.
 *
 * Conventions (every entry point):
 *  - Tensor arguments are device pointers; shapes are ints; strides are int64
 *    ELEMENT strides; the innermost (head-dim / packed) axis has unit stride
 *    and every row starts on a 16-byte boundary.
 *  - `stream` is a hipStream_t (0 = legacy default stream).  Launches are
 *    asynchronous; nothing here synchronises, allocates or copies to host, so
 *    every call can be captured in a hipGraph.
 *  - `workspace` is caller-owned device memory of at least the size returned
 *    by the matching *_workspace_size query.  It must be zero-filled once
 *    before first use; the kernels leave their counters at zero on exit.
 *    Calls that share a workspace must be ordered on one stream.
 *  - Return value: 0 on success, otherwise a hipError_t value
 *    (bytes_error_string() gives its text).  No C++ exception crosses the ABI.
 */
#ifndef BYTES_AMD_H_
#define BYTES_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version of this ABI (bumped on incompatible changes). */
int bytes_abi_version(void);

/* Text of a status code returned by any entry point. */
const char* bytes_error_string(int code);

/* ---------------------------------------------------------------------------
 * Dense bf16 GQA decode attention.
 * Replaces src/attention_kernels.py:65-92 (`decode_attn_bf16`, kernel :8-63).
 *   q   [B, Hq, D] bf16 (strides q_sb, q_sh)
 *   k,v [B, Hk, S, D] bf16 (strides *_sb, *_sh, *_ss)
 *   out [B, Hq, D] bf16 (strides o_sb, o_sh)
 *   out[b,h] = softmax(scale * q[b,h] . k[b,h/G]^T) v[b,h/G],  G = Hq/Hk
 * D in {64, 128}.  chunk = split-K chunk in tokens (0 = automatic).
 * The reference applies no scale; pass scale = 1.0 for identical semantics.
 * ------------------------------------------------------------------------- */
int bytes_decode_attn_bf16_workspace_size(int B, int Hq, int Hk, int S, int D, int chunk,
                                          size_t* bytes);
int bytes_decode_attn_bf16(const void* q, const void* k, const void* v, void* out,
                           int B, int Hq, int Hk, int S, int D,
                           int64_t q_sb, int64_t q_sh,
                           int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           int64_t v_sb, int64_t v_sh, int64_t v_ss,
                           int64_t o_sb, int64_t o_sh,
                           float scale, int chunk, void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* BYTES_AMD_H_ */
