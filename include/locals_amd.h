/* locals_amd: MI355X (gfx950) kernels for Locals' batched attention hot path.
 *
 * C ABI of liblocals_amd.so.  Every entry point is asynchronous on `stream`
 * (a hipStream_t passed as void*), allocates nothing, never synchronises, and
 * returns a status:
 *     0                 ok (the work is enqueued)
 *    -1  LCL_EINVAL     bad argument (null pointer, inconsistent shape, dtype)
 *    -2  LCL_EUNSUPPORTED  shape the kernels do not implement (e.g. head_dim != 128)
 *    -3  LCL_EWORKSPACE workspace missing or smaller than *_workspace_bytes()
 *    -4  LCL_ESCRATCH   the call needs more than the fixed scratch of the
 *                       allocation-free entry point (LCL_NOALLOC_SCRATCH_BYTES)
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
enum { LCL_OK = 0, LCL_EINVAL = -1, LCL_EUNSUPPORTED = -2, LCL_EWORKSPACE = -3, LCL_ESCRATCH = -4 };

/* Size of the device-resident scratch array behind lcl_qkv_attend_noalloc (one per GPU, held until the process
 * ends): 32 MiB, room for the split-K parts of 16 rows x 32 heads at 64k keys (BASELINE config 2 needs 17 MB,
 * config 3 4 MB). */
#define LCL_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Bytes of split-K workspace for R query rows of H heads over `extent` keys
 * (n for lcl_qkv_attend, cap for lcl_ragged_attention) with key chunk `block`
 * (0 = the library's choice; otherwise a multiple of 64): m, l and o[128] in fp32 for
 * every part of every (row, head), then one int32 part count a (row, head). */
size_t lcl_decode_workspace_bytes(int R, int H, int extent, int block);

/* qkv.attend (locals/qkv.py:213-249): one query per row against 8-bit affine
 * K/V read in place.
 *   q      (B, H, 128) dtype qdt
 *   kw, vw (B, KVH, cap, 32) uint32 words (4 codes each, little endian)
 *   ks, kb, vs, vb (B, KVH, cap, 2) scales / biases, dtype sdt (f16 or bf16)
 *   start  (B,) int32: row b attends to keys [max(start[b], 0), n); may be NULL (0)
 *   sinks  (H,) float32 logits in the softmax denominator only; may be NULL
 *   out    (B, H, 128) dtype qdt
 * n <= cap (any capacity).  `block` plays the role of the
 * reference's BLOCK (locals/qkv.py:28): keys per pass-1 workgroup. */
int lcl_qkv_attend(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                   const void* vs, const void* vb, int sdt, const int32_t* start, const float* sinks, float scale,
                   int B, int H, int KVH, int head_dim, int cap, int n, int block, void* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Profiling form of lcl_qkv_attend: the same call, with the pass-1 kernel's
 * dispatch bracketed by two hipEvent_t (ev_start, ev_stop; either may be NULL)
 * recorded by the dispatch itself.  No counterpart in the reference (it is for
 * callers that time the dominant kernel, e.g. bench.py). */
int lcl_qkv_attend_ex(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                      const void* vs, const void* vb, int sdt, const int32_t* start, const float* sinks, float scale,
                      int B, int H, int KVH, int head_dim, int cap, int n, int block, void* out, void* workspace,
                      size_t workspace_bytes, void* stream, void* ev_start, void* ev_stop);

/* lcl_qkv_attend without a workspace argument: the same kernels, with the split-K parts in a fixed
 * LCL_NOALLOC_SCRATCH_BYTES device array of the library instead of the caller's workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Calls a workspace of more than LCL_NOALLOC_SCRATCH_BYTES would need
 * (lcl_decode_workspace_bytes(B, H, n, block)) return LCL_ESCRATCH.  It allocates nothing: the array's address is
 * looked up once per device.  All calls on one GPU share its array, so calls that overlap on one GPU (two streams
 * at once) race; calls ordered on one stream do not. */
int lcl_qkv_attend_noalloc(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb,
                           const uint32_t* vw, const void* vs, const void* vb, int sdt, const int32_t* start,
                           const float* sinks, float scale, int B, int H, int KVH, int head_dim, int cap, int n,
                           int block, void* out, void* stream);

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

/* Profiling form of lcl_ragged_attention: pass 1's dispatch bracketed by two
 * hipEvent_t.  No counterpart in the reference. */
int lcl_ragged_attention_ex(const void* q, int qdt, const void* keys, const void* values, int kvdt,
                            const int32_t* slots, const int32_t* nkeys, float scale, const float* scale_dev, int R,
                            int H, int n_slots, int Hkv, int head_dim, int cap, int block, void* out, void* workspace,
                            size_t workspace_bytes, void* stream, void* ev_start, void* ev_stop);

/* BatchQuantizedKVCache.update_and_fetch's store (locals/qkv.py:309-326): MLX
 * affine 8-bit quantization (mx.quantize, group 64, bits 8, called at
 * locals/qkv.py:322-323) of a step's new keys k and values v, each
 * (B, KVH, L, D) of dtype dt (f16 or bf16), written at positions
 * [prev, prev + L) of the cache triples (B, KVH, cap, D/4) words and
 * (B, KVH, cap, D/64) scales/biases of dtype dt.  v (and its triple) may be NULL.
 * round_mode: 0 = ties away from zero (MLX's Metal path), 1 = ties to even
 * (MLX's CPU path).  With cap == L and prev == 0 this is plain mx.quantize.
 * Bit-exact: IEEE fp32 with correctly rounded division, RNE casts. */
int lcl_quantize_append(const void* k, const void* v, int dt, uint32_t* kw, void* ks, void* kb, uint32_t* vw,
                        void* vs, void* vb, int B, int KVH, int L, int D, int cap, int prev, int round_mode,
                        void* stream);

/* The buffer moves of BatchQuantizedKVCache's row bookkeeping -- merge (locals/qkv.py:417-431), extend
 * (:382-406), filter (:370-380), extract (:408-415) and finalize's roll (:340-346, mlx-lm dynamic_roll) -- as one
 * gather into a new triple: words dw (rows, KVH, cap, D/4) uint32, scales ds and biases db (rows, KVH, cap, D/64)
 * 16-bit.  Destination row r reads the source triple (src_w[r], src_s[r], src_b[r]) -- pointers to that row's
 * (kv head 0, position 0), src_cap[r] positions a kv head -- at position t - shift[r]: wrap[r] == 0 copies it when
 * it lies in [0, len[r]) and writes 0 elsewhere; wrap[r] == 1 takes it modulo len[r] (the roll).  The row
 * arrays are host memory (len rows each); a row with len 0 is all zeros and its pointers may be NULL.  The copy
 * is exact.  D a multiple of 64. */
int lcl_kv_gather(uint32_t* dw, void* ds, void* db, int rows, int KVH, int cap, int D, const uint32_t* const* src_w,
                  const void* const* src_s, const void* const* src_b, const long long* src_cap, const int* shift,
                  const int* len, const int* wrap, void* stream);

/* qkv.dequantized (locals/qkv.py:252-253, mx.dequantize): rows of D values
 * scale * code + bias from (rows, D/4) words and (rows, D/64) scales/biases of
 * dtype sdt, written as dtype odt (f16, bf16 or f32). */
int lcl_dequantize(const uint32_t* words, const void* scales, const void* biases, int sdt, long long rows, int D,
                   void* out, int odt, void* stream);

/* Bytes of split-K workspace for lcl_sdpa (B rows, H heads, L queries, N keys, key chunk
 * `block`, 0 = the library's choice).  0 when the call needs none: with a single chunk,
 * pass 1 writes the output itself and the workspace pointer may be NULL. */
size_t lcl_sdpa_workspace_bytes(int B, int H, int L, int N, int block);

/* Bytes of workspace for lcl_sdpa given the K/V format and mask as well: the split-K
 * bytes above, plus -- when the library takes its dequantize-first route for this call --
 * room for K and V dequantized to 16 bits, 2 * B * KVH * cap * 128 * 2 bytes after the
 * split-K part (rounded up to 256).  That route is taken for 8-bit K/V, any mask but the
 * sliding window, at least 16 row blocks per (row, KV head) and cap - N <= 512: the reference's
 * own prompt path dequantizes the whole prefix first too (locals/qkv.py:270-272).  A smaller
 * workspace (lcl_sdpa_workspace_bytes) keeps the fused 8-bit kernel; both give the same
 * values.  No counterpart in the reference. */
size_t lcl_sdpa_workspace_bytes_kv(int B, int H, int KVH, int L, int N, int cap, int block, int kvfmt,
                                   int mask_kind);

/* MLX scaled_dot_product_attention(q, k, v, scale, mask, sinks) as the reference
 * routes its multi-query variants through it: the 8-bit prefill/span branch of
 * qkv.attention -> fuse.attend_few over dequantized K/V (locals/qkv.py:270-272,
 * locals/fuse.py:131-144), tree verification (locals/treedec.py:56-79,
 * locals/packed.py:107-116) and packed segments (locals/packed.py:137-143).
 *   q (B, H, L, 128) dtype qdt; out (B, H, L, 128) dtype qdt
 *   kvfmt 0: 8-bit triples kw/ks/kb, vw/vs/vb as in lcl_qkv_attend (scales dtype kvdt)
 *   kvfmt 1: 16-bit kf, vf (B, KVH, cap, 128) dtype kvdt
 *   the first N <= cap keys of each buffer row are attended; start (B,) or NULL
 *   masks keys before start[b] (left padding)
 *   mask_kind 0 none; 1 causal (query i sees key j iff j <= N - L + i);
 *   2 tree: key j < N - L visible to all, key N - L + d visible to query i iff
 *     bit d of tree[b * tree_bs + i] (L <= 64; tree_bs = L, or 0 for one shared mask);
 *   3 dense: uint8 dense[b*msb + h*msh + i*msq + j*msk] != 0 (strides may be 0);
 *   4 sliding window: query i sees key j iff N - L + i - window < j <= N - L + i
 *     (window >= 1; the banded prompt chunks of the sliding-window layers,
 *     locals/fuse.py:113-125, locals/models/flint_streamed.py:114-128); each
 *     workgroup reads only the keys its queries' windows reach
 *   window is read for mask_kind 4 only.
 *   sinks (H,) float32 or NULL.  A query with no visible key and no sink gives 0. */
int lcl_sdpa(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
             const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
             const int32_t* start, int mask_kind, int window, const unsigned long long* tree, long long tree_bs,
             const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
             float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
             void* workspace, size_t workspace_bytes, void* stream);

/* Profiling form of lcl_sdpa: pass 1's dispatch bracketed by two hipEvent_t.  No
 * counterpart in the reference. */
int lcl_sdpa_ex(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
                const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
                const int32_t* start, int mask_kind, int window, const unsigned long long* tree, long long tree_bs,
                const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
                float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
                void* workspace, size_t workspace_bytes, void* stream, void* ev_start, void* ev_stop);

/* qk_kernel.qk_norm_rope (locals/qk_kernel.py:24-109, metal_kernel source
 * :24-69, launch :85-109): per-head RMS norms of q and k, RoPE over halves, v
 * split out.
 *   qkv  (B, L, (H + 2 KV) * head_dim) dtype dt (f16 or bf16); head_dim a multiple of 128 up to 1024
 *   q_w, k_w (head_dim,) dtype dt: the q_norm / k_norm weights; eps the shared norm eps
 *   offsets int32 device array: (B,) if offsets_per_row else (1,); position of
 *     (b, l) is offsets[b or 0] + l
 *   rope 0: norms only (a layer without RoPE); log2_base = log2(rope base)
 *   q (B, H, L, head_dim), k and v (B, KV, L, head_dim), dtype dt
 * Rounding points as qk_kernel.py:56-62: T(w * T(x r)), then T of the rotation;
 * the angle in fp32 as qk_kernel.py:59; v is copied bit-exactly. */
int lcl_qk_norm_rope(const void* qkv, int dt, const void* q_w, const void* k_w, const int32_t* offsets,
                     int offsets_per_row, float eps, float log2_base, int rope, int B, int L, int H, int KV,
                     int head_dim, void* q, void* k, void* v, void* stream);

/* lcl_qk_norm_rope fused with the 8-bit cache store that follows it
 * (locals/fuse.py:80-83 -> BatchQuantizedKVCache.update_and_fetch,
 * locals/qkv.py:309-326): q as lcl_qk_norm_rope; the normed/rotated k and the
 * raw v are quantized (MLX affine 8 bits, group 64, as lcl_quantize_append, same
 * round_mode) into positions [prev, prev + L) of the cache triples
 * kw/vw (B, KV, cap, head_dim/4) uint32, ks/kb/vs/vb (B, KV, cap, head_dim/64)
 * dtype dt.  The result equals lcl_qk_norm_rope followed by
 * lcl_quantize_append of its k and v, bit for bit. */
int lcl_qk_norm_rope_append(const void* qkv, int dt, const void* q_w, const void* k_w, const int32_t* offsets,
                            int offsets_per_row, float eps, float log2_base, int rope, int B, int L, int H, int KV,
                            int head_dim, void* q, void* kw, void* ks, void* kb, void* vw, void* vs, void* vb,
                            int cap, int prev, int round_mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCALS_AMD_H */
