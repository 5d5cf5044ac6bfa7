/*
 * mpx_attn.h — C ABI of libmpx_attn.so, the MI355X (gfx950) attention hot path
 * behind the mlx-primitives Python API.
 *
 * Every entry point:
 *   - takes raw device pointers, element strides and sizes (no framework types);
 *   - never allocates or frees device memory (the caller passes the workspace);
 *   - launches asynchronously on the caller's HIP stream (`stream` is a
 *     hipStream_t; NULL means the legacy default stream) and never synchronises;
 *   - returns MPX_OK or a negative MPX_E* code, with a message readable through
 *     mpx_last_error() on the calling thread.
 *
 * dtype codes: MPX_F32 (float), MPX_F16 (IEEE half), MPX_BF16 (bfloat16).
 * Tensors are addressed through element strides in the logical order
 * (batch, head, seq); the head dimension must be contiguous (stride 1).
 */
#ifndef MPX_ATTN_H
#define MPX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MPX_OK 0
#define MPX_EINVAL (-1)       /* bad argument: the Python layer raises ValueError */
#define MPX_EUNSUPPORTED (-2) /* valid but not implemented (e.g. head_dim > 256) */
#define MPX_EHIP (-3)         /* a HIP launch/runtime call failed: RuntimeError */

#define MPX_F32 0
#define MPX_F16 1
#define MPX_BF16 2

/* Library version, (major << 16) | minor. */
int mpx_version(void);

/* Message describing the last failure on this thread ("" if none). */
const char* mpx_last_error(void);

/*
 * Exact softmax attention forward, O = softmax(scale * Q K^T + mask) V, with
 * the row sums normalised as O / (l + 1e-6) like the reference's tiled
 * online-softmax path.
 *
 * Replaces (one entry serves all four reference entry points):
 *   - flash_attention / FlashAttention  (mlx_primitives/attention/flash.py:52-254,
 *     tiled path 257-316, BHSD dense branch 172-192, Metal kernel 319-476);
 *   - sliding_window_attention / SlidingWindowAttention
 *     (mlx_primitives/attention/sliding_window.py:227-313, tiled 363-511);
 *   - chunked_cross_attention / ChunkedCrossAttention
 *     (mlx_primitives/attention/chunked.py:43-169);
 *   - the per-chunk kernel + merge (mlx_primitives/attention/_online_softmax.py:42-176).
 *
 * Shapes: Q (B, H, Sq, D), K and V (B, H, Sk, D), O (B, H, Sq, D) addressed by
 * the *_strides arrays = {batch, head, seq} element strides, so BSHD and BHSD
 * tensors are both passed without a transpose.
 *
 * Mask, with q and kv absolute positions (top-left aligned, kv <= q when causal):
 *   causal != 0        -> kv <= q  (window_right is then ignored)
 *   window_left  >= 0  -> kv >= q - window_left   (-1 = unbounded)
 *   window_right >= 0  -> kv <= q + window_right  (-1 = unbounded)
 * Sliding-window semantics of the reference (|q-kv| <= W, plus kv <= q when
 * causal) are window_left = W with causal = 1, or window_left = window_right = W.
 *
 * Supported: D <= 256 (kernels are built for D in {32, 64, 128, 256}; pass D
 * as one of those, zero-padded by the caller otherwise), dtype f32/f16/bf16,
 * 16-byte aligned base pointers and seq strides that are multiples of 8
 * elements (4 for f32).
 *
 * workspace: device memory of at least mpx_attn_fwd_workspace_bytes(...) bytes
 * for the same arguments (0 bytes means no workspace is needed, pass NULL).
 */
int mpx_attn_fwd(const void* q, const void* k, const void* v, void* o,
                 const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 int B, int H, int Sq, int Sk, int D, float scale, int causal,
                 int window_left, int window_right, int dtype,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Workspace needed by mpx_attn_fwd (split-KV partials for long KV / few q tiles). */
size_t mpx_attn_fwd_workspace_bytes(int B, int H, int Sq, int Sk, int D, int causal,
                                    int window_left, int window_right, int dtype);

/*
 * Paged-KV decode attention: one query token per sequence against the
 * sequence's cached tokens, gathered through a block table.
 *
 * Replaces paged_attention(q, k_pool, v_pool, block_tables, context_lens, ...)
 * with seq_q == 1 (mlx_primitives/cache/paged_attention.py:44-105 -> decode
 * path 108-208), including the optional ALiBi bias (163-178).
 *
 *   q             (B, H, D) via q_strides = {batch, head}, D contiguous
 *   k_pool/v_pool (num_blocks, block_size, H, D), contiguous
 *   block_tables  int32 (B, max_blocks), row-major, -1 = no page
 *   context_lens  int32 (B,)
 *   alibi_slopes  float32 (H,) or NULL; bias = slope_h * (kv_pos - context_len)
 *   o             (B, H, D) via o_strides
 *
 * D is the head dim of q, the pools and o: any multiple of 8 elements (16-bit
 * dtypes) or 4 (float32) up to 256, read in place (no padded copy of the
 * pools). Token t of sequence b is valid iff t < context_lens[b] and
 * 0 <= block_tables[b, t / block_size] < num_blocks; the softmax runs over
 * valid tokens only (exact, no epsilon). A sequence with no valid token gets
 * NaN, as the reference's softmax over an all -inf row does.
 */
int mpx_paged_decode(const void* q, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, const int32_t* context_lens,
                     const float* alibi_slopes, void* o,
                     const int64_t* q_strides, const int64_t* o_strides,
                     int B, int H, int D, int num_blocks, int block_size, int max_blocks,
                     float scale, int dtype, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Workspace needed by mpx_paged_decode (per-partition (o, m, l) partials). */
size_t mpx_paged_decode_workspace_bytes(int B, int H, int D, int block_size, int max_blocks);

/*
 * Paged-KV prefill attention: Sq query tokens per sequence against the
 * sequence's cached tokens, gathered through a block table inside the
 * attention kernel (no dense copy of the pages is made).
 *
 * Replaces paged_attention(...) with seq_q > 1
 * (mlx_primitives/cache/paged_attention.py:44-105 -> prefill path 211-320).
 *
 *   q             (B, H, Sq, D) via q_strides = {batch, head, seq}, D contiguous
 *   k_pool/v_pool (num_blocks, block_size, H, D), contiguous
 *   block_tables  int32 (B, max_blocks), row-major, -1 = no page
 *   context_lens  int32 (B,)
 *   alibi_slopes  float32 (H,) or NULL; bias = slope_h * (kv_pos - q_pos)
 *   o             (B, H, Sq, D) via o_strides
 *
 * Query i sits at position i (top-left alignment, as in the reference): with
 * causal != 0 it sees kv_pos <= i. Token t of sequence b is valid iff
 * t < context_lens[b] and 0 <= block_tables[b, t / block_size] < num_blocks.
 * Exact softmax over the valid, unmasked tokens; a query row with none gets
 * NaN (the reference's softmax over an all -inf row). D in {32, 64, 128, 256};
 * pools of any size (from 4 GiB - 256 bytes on, 16-bit pools are read through
 * 64-bit addresses).
 */
int mpx_paged_prefill(const void* q, const void* k_pool, const void* v_pool,
                      const int32_t* block_tables, const int32_t* context_lens,
                      const float* alibi_slopes, void* o,
                      const int64_t* q_strides, const int64_t* o_strides,
                      int B, int Sq, int H, int D, int num_blocks, int block_size,
                      int max_blocks, float scale, int causal, int dtype,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace needed by mpx_paged_prefill (split-KV partials when few query tiles). */
size_t mpx_paged_prefill_workspace_bytes(int B, int Sq, int H, int D, int block_size,
                                         int max_blocks, int causal, int dtype);

/*
 * KV-cache append: write T new key/value token rows per sequence into their
 * pages. Token t (< n_tokens[b]) of sequence b goes to position
 * pos = start_pos[b] + t, i.e. page block_tables[b, pos / block_size], slot
 * pos % block_size of both pools.
 *
 * Replaces KVCache._store_kv (mlx_primitives/cache/kv_cache.py:194-264) and the
 * BlockAllocator.set_block_data writes it issues
 * (mlx_primitives/cache/block_allocator.py:299-331), batched over sequences.
 *
 *   k, v          (B, T, H, D) via k_strides / v_strides = {batch, token, head}
 *   k_pool/v_pool (num_blocks, block_size, H, D), contiguous, updated in place
 *   block_tables  int32 (B, max_blocks); start_pos, n_tokens int32 (B,)
 *   errors        int32[3] device words, cleared to 0 by the caller; the kernel
 *                 sets [0] = 1 for a negative position, [1] = 1 for a block
 *                 index >= max_blocks, [2] = 1 for a page id outside
 *                 [0, num_blocks). Such tokens are skipped; all others are
 *                 written. Two tokens aimed at the same slot race.
 *
 * D * element size must be a multiple of 16 bytes; H * D * element size
 * below 2^34 bytes and B * T * ceil(H * D * element size / 4096) below 2^31
 * (MPX_EINVAL otherwise).
 */
int mpx_kv_append(const void* k, const void* v, void* k_pool, void* v_pool,
                  const int32_t* block_tables, const int32_t* start_pos,
                  const int32_t* n_tokens, const int64_t* k_strides, const int64_t* v_strides,
                  int B, int T, int H, int D, int num_blocks, int block_size, int max_blocks,
                  int dtype, int32_t* errors, void* stream);

/*
 * mpx_kv_append with each K row rotated to its position on the way into the
 * pool (half-split RoPE over the contiguous (n_pos, D/2) cos / sin tables of
 * cache_dtype, float32 arithmetic, one rounding: the same values as mpx_rope
 * followed by mpx_kv_append); V rows are copied. errors holds 4 words: the 3
 * of mpx_kv_append and [3] = 1 for a position at or past n_pos (token
 * skipped). D must be a multiple of 16, rows 16-byte aligned.
 *
 * Replaces the K side of the reference's fused kernel, which rotates K at
 * kv_offset + j every time it attends (mlx_primitives/kernels/
 * fused_rope_attention.py:766-800, 939-987): a cache written through this
 * entry point holds K already rotated, so the attention that reads it rotates
 * only Q (mpx_rope_at, or Q-on-load in mpx_attn_fwd_rope). Together with
 * KVCache._store_kv (mlx_primitives/cache/kv_cache.py:194-264) as in
 * mpx_kv_append.
 */
int mpx_kv_append_rope(const void* k, const void* v, void* k_pool, void* v_pool,
                       const int32_t* block_tables, const int32_t* start_pos,
                       const int32_t* n_tokens, const int64_t* k_strides,
                       const int64_t* v_strides, int B, int T, int H, int D, int num_blocks,
                       int block_size, int max_blocks, int dtype, const void* cos_cache,
                       const void* sin_cache, int n_pos, int cache_dtype, int32_t* errors,
                       void* stream);

/*
 * Grouped-query variants (no counterpart in the reference, whose flash_attention
 * rejects Hq != Hk at mlx_primitives/attention/flash.py:151-154 and whose paged
 * pools carry the query heads; an extension behind the Python flag enable_gqa):
 * the same entries with K/V carrying H_kv heads, H a multiple of H_kv, query head h
 * reading K/V head h / (H / H_kv). mpx_attn_fwd, mpx_paged_decode and
 * mpx_paged_prefill are these with H_kv = H. K/V strides (and the pools'
 * (num_blocks, block_size, H_kv, D) layout) describe the H_kv heads; workspace
 * sizes are those of the plain entries.
 */
int mpx_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o,
                     const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                     int window_left, int window_right, int dtype,
                     void* workspace, size_t workspace_bytes, void* stream);

int mpx_paged_decode_gqa(const void* q, const void* k_pool, const void* v_pool,
                         const int32_t* block_tables, const int32_t* context_lens,
                         const float* alibi_slopes, void* o,
                         const int64_t* q_strides, const int64_t* o_strides,
                         int B, int H, int H_kv, int D, int num_blocks, int block_size,
                         int max_blocks, float scale, int dtype, void* workspace,
                         size_t workspace_bytes, void* stream);

int mpx_paged_prefill_gqa(const void* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, const int32_t* context_lens,
                          const float* alibi_slopes, void* o,
                          const int64_t* q_strides, const int64_t* o_strides,
                          int B, int Sq, int H, int H_kv, int D, int num_blocks, int block_size,
                          int max_blocks, float scale, int causal, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Rotary position embedding, half-split form: for a row at position
 * p = offset + s and i < D/2, with c = cos_cache[p, i], s_ = sin_cache[p, i],
 *   out[i] = x[i] * c - x[i + D/2] * s_,   out[i + D/2] = x[i] * s_ + x[i + D/2] * c
 * in float32, rounded once to dtype.
 *
 * Replaces rope(x, cos_cache, sin_cache, offset) (mlx_primitives/kernels/rope.py:451-497)
 * as applied to Q and K by fast_fused_rope_attention / fused_rope_attention
 * (mlx_primitives/kernels/fused_rope_attention.py:711-714, 939-985).
 *
 *   x, out      (B, S, H, D) via {batch, seq, head} element strides, D contiguous,
 *               16-byte aligned rows; out may not alias x
 *   cos/sin     contiguous (n_pos, D/2) tables of cache_dtype; offset + S <= n_pos
 *
 * D must be a multiple of 16.
 */
int mpx_rope(const void* x, void* out, const void* cos_cache, const void* sin_cache,
             const int64_t* x_strides, const int64_t* out_strides, int B, int S, int H, int D,
             int offset, int n_pos, int dtype, int cache_dtype, void* stream);

/*
 * mpx_rope with a position per sequence: row s of batch b is rotated to
 * position positions[b] + s (positions: device int32 (B,)). Rows whose position
 * falls outside [0, n_pos) are left unwritten and set errors[0] = 1 (device
 * int32 word, cleared by the caller).
 *
 * Replaces rope(x, cos_cache, sin_cache, offset) (mlx_primitives/kernels/rope.py:451-497)
 * applied to each sequence of a decode batch at its own offset, as a serving
 * loop rotates every sequence's new query at the position it has reached
 * (mlx_primitives/kernels/fused_rope_attention.py:766-800: q_offset per call).
 */
int mpx_rope_at(const void* x, void* out, const void* cos_cache, const void* sin_cache,
                const int64_t* x_strides, const int64_t* out_strides, int B, int S, int H,
                int D, const int32_t* positions, int n_pos, int dtype, int cache_dtype,
                int32_t* errors, void* stream);

/*
 * mpx_attn_fwd_gqa with Q rotated on load: query row i is rotated to position
 * q_offset + i (half-split RoPE with the contiguous (n_pos, D/2) cos / sin
 * tables of cache_dtype, float32 arithmetic, one rounding to dtype; the same
 * values as mpx_rope applied to q first). K must already be rotated.
 *
 * Replaces the Q side of the reference's fused kernel, which rotates Q and K
 * while loading them (mlx_primitives/kernels/fused_rope_attention.py:766-800,
 * 939-985). 16-bit dtypes only (float32: MPX_EUNSUPPORTED); q_offset + Sq <=
 * n_pos; 16-byte aligned tables.
 */
int mpx_attn_fwd_rope(const void* q, const void* k, const void* v, void* o,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                      int window_left, int window_right, int dtype,
                      const void* cos_cache, const void* sin_cache, int q_offset, int n_pos,
                      int cache_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward pass of the flash attention forward.
 *
 * The reference differentiates flash_attention (and sliding_window_attention,
 * chunked_cross_attention) with mx.grad through its tiled online-softmax path
 * (mlx_primitives/attention/flash.py:257-316; tests/attention/test_flash.py:338-362,
 * tests/parity/pytorch/test_attention_parity.py:107-163). Here the forward
 * saves each row's log-sum-exp and the backward recomputes the probabilities.
 *
 * mpx_attn_fwd_lse is mpx_attn_fwd_gqa plus lse: a (B, H, Sq) contiguous
 * float32 array that receives m + log2(l + 1e-6) per query row (base-2 units
 * of the scaled scores, m the row max of scale * log2(e) * q.k), +inf for rows
 * that see no key; lse may be NULL.
 *
 * mpx_attn_bwd: given q, k, v, the forward output o, its lse, and dout
 * (= dL/do), writes dq, dk, dv (dk, dv carry H_kv heads; a K/V head's gradient
 * sums over its group of query heads). All tensors use {batch, head, seq}
 * element strides like mpx_attn_fwd, D contiguous; dq, dk, dv must not
 * overlap the inputs. Masks (causal, windows) are those of the forward call.
 * Scope: dtype float32 / float16 / bfloat16, D in {64, 128, 256}, scale > 0.
 * Workspace: mpx_attn_bwd_workspace_bytes(B, H, Sq) bytes, 16-byte aligned
 * (per-row rowsum(dout * o)). A workspace of at least
 * mpx_attn_bwd_ds_workspace_bytes(...) bytes (same problem arguments; 0 when
 * the problem has no such schedule: float32, or D other than 128) selects the
 * stored-dS schedule: the dK/dV kernel stores dS (16-bit, only the 32 x 32
 * blocks the mask leaves, about B * H * Sq * Sk bytes under a causal mask)
 * and dQ is computed from it instead of recomputing S and dP (and, with
 * dropout, the keep mask). On MI355X it is the faster schedule for
 * mpx_attn_bwd_dropout (6% over forward and backward at 4 x 32 x 4096 x 128)
 * and runs level with the other one for mpx_attn_bwd.
 */
int mpx_attn_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse,
                     const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                     int window_left, int window_right, int dtype,
                     void* workspace, size_t workspace_bytes, void* stream);

size_t mpx_attn_bwd_workspace_bytes(int B, int H, int Sq);

/* The workspace of mpx_attn_bwd's stored-dS schedule (no counterpart in the
 * reference, which differentiates through mx.grad; it is the same backward
 * with dQ taken from stored dS). */
size_t mpx_attn_bwd_ds_workspace_bytes(int B, int H, int Sq, int Sk, int D, int dtype,
                                       int causal, int window_left, int window_right);

int mpx_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                 const float* lse, void* dq, void* dk, void* dv,
                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                 const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                 const int64_t* dk_strides, const int64_t* dv_strides,
                 int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                 int window_left, int window_right, int dtype,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Attention with dropout on the weights, forward and backward.
 *
 * Replaces the reference's training path with dropout_p > 0
 * (mlx_primitives/attention/flash.py:202-205 -> _reference_flash_attention_with_dropout,
 * flash.py:528-578; sliding_window.py:280-282, 564-625; chunked.py:109-110, 206-255):
 * weights = softmax(scores) * keep / (1 - dropout_p), output = weights @ v, with
 * keep ~ Bernoulli(1 - dropout_p) per (batch, head, query, key).
 *
 * Here the keep mask is never stored: it is a hash of (seed, row, key), so the
 * backward regenerates the forward's mask from the same seed. Row r =
 * (b * H + h) * Sq + q (mod 2^32), key k, pair m = k / 2:
 *   bits = lowbias32((r * 0x9E3779B1 + seed_lo) ^ (m * 0x85EBCA77 + seed_hi))
 * (lowbias32: x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b;
 * x ^= x >> 16), seed_lo / seed_hi the low / high 32 bits of seed; key 2m reads
 * the low 16 bits of bits, key 2m + 1 the high 16, and a key is kept when its
 * 16 bits are >= round(dropout_p * 65536) (at most 65535): the keep
 * probability is 1 - dropout_p to within 2^-17.
 *
 * mpx_attn_fwd_dropout is mpx_attn_fwd_lse with dropout_p in [0, 1) and the
 * seed (lse may be NULL; its values, and so the backward's probabilities, are
 * those of the undropped softmax). dropout_p = 0 is the plain forward.
 * mpx_attn_bwd_dropout is mpx_attn_bwd of that forward: same arguments plus
 * the forward's dropout_p and seed. Scope: D in {64, 128, 256}, float32 /
 * float16 / bfloat16, every mask and K/V head grouping of the plain kernels.
 */
int mpx_attn_fwd_dropout(const void* q, const void* k, const void* v, void* o, float* lse,
                         const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides, const int64_t* o_strides,
                         int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                         int window_left, int window_right, int dtype, float dropout_p,
                         uint64_t seed, void* workspace, size_t workspace_bytes, void* stream);

int mpx_attn_bwd_dropout(const void* q, const void* k, const void* v, const void* o,
                         const void* dout, const float* lse, void* dq, void* dk, void* dv,
                         const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides, const int64_t* o_strides,
                         const int64_t* do_strides, const int64_t* dq_strides,
                         const int64_t* dk_strides, const int64_t* dv_strides,
                         int B, int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                         int window_left, int window_right, int dtype, float dropout_p,
                         uint64_t seed, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Paged-KV decode that allocates nothing: mpx_paged_decode_gqa without the
 * workspace arguments. It has no counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).
 *
 * The per-partition (o, m, l) partials go to a static device array of
 * MPX_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends. Calls needing more (B * H *
 * ceil(max_blocks * block_size / 512) * (kernel head dim + 2) * 4 bytes,
 * kernel head dim = 32, 64, 128 or 256 >= D) return MPX_EINVAL. Nothing in the
 * array has to start at zero: each call writes every partial it reads. All
 * calls on one GPU share that GPU's array, so two calls that overlap on one
 * GPU (different streams, or threads without ordering) race and corrupt each
 * other; calls on one stream are ordered and safe. `stream` must belong to the
 * calling thread's current device. Results are identical to mpx_paged_decode_gqa.
 */
#define MPX_NOALLOC_SCRATCH_BYTES (32u << 20)

int mpx_paged_decode_noalloc(const void* q, const void* k_pool, const void* v_pool,
                             const int32_t* block_tables, const int32_t* context_lens,
                             const float* alibi_slopes, void* o,
                             const int64_t* q_strides, const int64_t* o_strides,
                             int B, int H, int H_kv, int D, int num_blocks, int block_size,
                             int max_blocks, float scale, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MPX_ATTN_H */
