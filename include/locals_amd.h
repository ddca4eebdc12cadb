/* locals_amd: MI355X (gfx950) kernels for Locals' batched attention hot path.
 *
 * C ABI of liblocals_amd.so.  Every entry point is asynchronous on `stream`
 * (a hipStream_t passed as void*), allocates nothing, never synchronises, and
 * returns a status:
 *     0                 ok (the work is enqueued)
 *    -1  LCL_EINVAL     bad argument (null pointer, inconsistent shape, dtype)
 *    -2  LCL_EUNSUPPORTED  shape the kernels do not implement (e.g. head_dim != 128)
 *    -3  LCL_EWORKSPACE workspace missing or smaller than *_workspace_bytes()
 *    >0                 a hipError_t from the launch, passed through
 * All tensors are contiguous, row-major, in device memory owned by the caller.
 * dtype codes: 0 float16, 1 bfloat16, 2 float32.
 *
 * The reference interface each entry point replaces is cited beside it
 * (paths are in Generated-Computers/Locals).
 */
#ifndef LOCALS_AMD_H
#define LOCALS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LCL_F16 = 0, LCL_BF16 = 1, LCL_F32 = 2 };
enum { LCL_OK = 0, LCL_EINVAL = -1, LCL_EUNSUPPORTED = -2, LCL_EWORKSPACE = -3 };

/* Bytes of split-K workspace for R query rows of H heads over `extent` keys
 * (n for lcl_qkv_attend, cap for lcl_ragged_attention) with key chunk `block`
 * (0 = the library's choice; otherwise a multiple of 64). */
size_t lcl_decode_workspace_bytes(int R, int H, int extent, int block);

/* qkv.attend (locals/qkv.py:213-249): one query per row against 8-bit affine
 * K/V read in place.
 *   q      (B, H, 128) dtype qdt
 *   kw, vw (B, KVH, cap, 32) uint32 words (4 codes each, little endian)
 *   ks, kb, vs, vb (B, KVH, cap, 2) scales / biases, dtype sdt (f16 or bf16)
 *   start  (B,) int32: row b attends to keys [max(start[b], 0), n); may be NULL (0)
 *   sinks  (H,) float32 logits in the softmax denominator only; may be NULL
 *   out    (B, H, 128) dtype qdt
 * cap must be a multiple of 16 and n <= cap.  `block` plays the role of the
 * reference's BLOCK (locals/qkv.py:28): keys per pass-1 workgroup. */
int lcl_qkv_attend(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                   const void* vs, const void* vb, int sdt, const int32_t* start, const float* sinks, float scale,
                   int B, int H, int KVH, int head_dim, int cap, int n, int block, void* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* attention.ragged_attention (locals/attention.py:200-224): row r of a packed
 * batch reads KV slot slots[r] and its first nkeys[r] keys.
 *   q (R, H, 128) dtype qdt; keys, values (n_slots, Hkv, cap, 128) dtype kvdt
 *   (f16 or bf16); slots, nkeys (R,) int32; out (R, H, 128) dtype qdt.
 * scale_dev, when not NULL, is a (1,) float32 device scalar used instead of
 * `scale` (the reference passes the scale as a (1,) array).
 * A row with nkeys 0 gives 0.  A slot outside [0, n_slots) is clamped. */
int lcl_ragged_attention(const void* q, int qdt, const void* keys, const void* values, int kvdt, const int32_t* slots,
                         const int32_t* nkeys, float scale, const float* scale_dev, int R, int H, int n_slots, int Hkv, int head_dim, int cap,
                         int block, void* out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCALS_AMD_H */
