/*
 * fmkv -- MI355X quantized KV cache for Gemma-4 attention layers (C ABI).
 *
 * Drop-in boundary for flash-moe's KV-cache path. The reference keeps the
 * cache in Rust (`KVCache`, src/cache.rs:166-310) and computes with MLX
 * through mlx-rs; its one hand-written FFI is `mlx_array_from_mmap`
 * (src/ffi.rs:5-14). This header is the C surface that replaces the MLX calls
 * on that path: plain integers, sizes and device pointers, no exceptions, an
 * int status on every call and a thread-local error string.
 *
 * Conventions
 *  - Device buffers are HIP device pointers owned by the caller.
 *  - K/V input rows are bf16, contiguous [n_tokens][n_kv_heads][head_dim]
 *    (post-RoPE K and post-v_norm V, src/model/gemma4_attention.rs:62-81).
 *  - q is bf16 [n_q_heads][head_dim]; out is [n_q_heads][head_dim] in bf16
 *    or f32 (FMKV_DTYPE_*). q head h reads KV head h / (n_q_heads/n_kv_heads).
 *  - `stream` is a hipStream_t (NULL = default stream). Every call is
 *    stream-ordered and asynchronous unless stated; nothing synchronises.
 *  - A handle is used by one host thread at a time (no internal locks).
 *  - Descriptor validation runs before any HIP call, so invalid input is
 *    reported on machines without a GPU too.
 *  - Magnitude bound of the affine attention read: the softmax weight times
 *    a V group's scale travels as an f16 pair (high part + residual, at most
 *    about 1.3e5) with weights up to 2^8, so a V group's f16 scale must stay
 *    below 511 -- a rotated V group spanning less than 511 * (2^bits - 1),
 *    about 7.6e3 at 4 bits and 1.3e5 at 8 bits. v_norm'd V (unit RMS) is
 *    four orders of magnitude inside; raw V rows beyond it lose accuracy.
 */
#ifndef FMKV_H
#define FMKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define FMKV_OK 0
#define FMKV_ERR_INVALID_ARG 1 /* null pointer, negative size, bad dtype */
#define FMKV_ERR_UNSUPPORTED 2 /* head_dim / bits / group / mode not supported */
#define FMKV_ERR_OOM 3         /* device allocation failed */
#define FMKV_ERR_HIP 4         /* a HIP call or launch failed */
#define FMKV_ERR_CAPACITY 5    /* append would exceed a linear cache's capacity */

/* cache modes */
#define FMKV_MODE_AFFINE 0   /* rotated, group-64 affine 4/8-bit codes + f16 scale/bias */
#define FMKV_MODE_CODEBOOK 1 /* rotated TurboQuant Lloyd-Max 2/3/4-bit indices + f16 norm */
#define FMKV_MODE_PLAIN 2    /* unquantized bf16 rows (bits = 16): KVCacheInner::Plain,
                                src/cache.rs:174-178, :274-288; --no-kv-quant */

/* output dtypes */
#define FMKV_DTYPE_BF16 0
#define FMKV_DTYPE_F32 1

/* Cache descriptor. Mirrors the arguments of
 * KVCache::new_quantized_with_window(head_dim, bits, window)
 * (src/cache.rs:206-227) plus what a preallocated device arena needs. */
typedef struct fmkv_cache_desc {
  int32_t n_kv_heads; /* >= 1 */
  int32_t head_dim;   /* 128, 256 or 512 */
  int32_t bits;       /* affine: 4 or 8; codebook: 2, 3 or 4 (src/cache.rs:67-89); plain: 16 */
  int32_t group_size; /* 64 */
  int32_t mode;       /* FMKV_MODE_* */
  int32_t window;     /* 0: global layer, linear growth; W > 0: sliding window of the last W
                       * positions, kept in a ring of W rounded up to 16 slots (W <= 2^30) */
  int64_t capacity;   /* linear caches: max positions; ignored for rings */
  uint64_t sign_seed; /* seed of the RHT sign vector; the reference uses 42 (src/cache.rs:49) */
} fmkv_cache_desc;

typedef struct fmkv_cache fmkv_cache;

/* Message of the last failed call on this thread ("" if none). */
const char* fmkv_last_error(void);

/* Validate a descriptor without touching HIP (src/cache.rs:87 panics on bad
 * bits; here it is FMKV_ERR_UNSUPPORTED). */
int fmkv_validate_desc(const fmkv_cache_desc* desc);

/* Bytes of one 16-token head-block and of the whole arena for `desc`. */
int fmkv_layout_bytes(const fmkv_cache_desc* desc, int64_t* block_bytes, int64_t* arena_bytes);

/* Create / destroy. Replaces KVCache::new_quantized_with_window
 * (src/cache.rs:206-227) and its drop; Model::make_cache (src/model/mod.rs:375-396)
 * calls it once per layer. The handle owns all device storage. */
int fmkv_cache_create(const fmkv_cache_desc* desc, fmkv_cache** out);
int fmkv_cache_destroy(fmkv_cache* cache);

/* KVCache::offset (src/cache.rs:230-232): positions appended so far. */
int fmkv_cache_offset(const fmkv_cache* cache, int64_t* out);
/* KVCache::stored_len (src/cache.rs:236-242): positions currently visible
 * (min(offset, window) for rings, minus anything trimmed). */
int fmkv_cache_stored_len(const fmkv_cache* cache, int64_t* out);

/* The store half of KVCache::update_and_fetch (src/cache.rs:266-310):
 * rotate, quantize and write n_tokens new positions (offset .. offset+n-1);
 * rings overwrite slot pos % W, so afterwards exactly the last W positions
 * are stored (tail_along_time, src/cache.rs:140-148). Advances offset by n. */
int fmkv_cache_append(fmkv_cache* cache, const void* k_bf16, const void* v_bf16,
                      int64_t n_tokens, void* stream);

/* Hide all but the last `keep_last` stored positions (the explicit form of
 * tail_along_time, src/cache.rs:140-148). offset is unchanged. */
int fmkv_cache_trim(fmkv_cache* cache, int64_t keep_last);

/* Decode-step attention read over the cache, replacing
 * mlx_rs::fast::scaled_dot_product_attention(q, k_all, v_all, scale, None)
 * at src/model/gemma4_attention.rs:94-103 for L == 1 (Gemma-4: scale 1.0).
 * The current position attends to its own quantized K/V, as in the
 * reference where the round trip precedes the concat (src/cache.rs:295-298).
 * All modes: a codebook (TurboQuant) cache is read as stored --
 * centroid[idx] * norm / sqrt(D) in the rotated domain -- with no bf16 round
 * trip (src/cache.rs:94-129); a plain cache is the bf16 rows themselves.
 * sparse_v_tau > 0 is the reference's sparse-V decode
 * (src/model/gemma4_attention.rs:196-234): softmax weights below tau are
 * zeroed without renormalisation. It reads the keys twice (a statistics
 * pass, then the gated pass, which skips the blocks whose weights all fall
 * below tau); 0 is plain softmax attention. Every cache mode. Negative or
 * non-finite tau returns FMKV_ERR_INVALID_ARG. */
int fmkv_decode_attention(fmkv_cache* cache, const void* q_bf16, int32_t n_q_heads, float scale,
                          float sparse_v_tau, void* out, int32_t out_dtype, void* stream);

/* The layer's prologue before the cache store, fused into the append
 * (src/model/gemma4_attention.rs:52-81; no separate pass over K/V):
 *   K = RoPE(k_norm(k_proj)) -- fast::rms_norm with the layer's weight
 *       (norm.rs:5-14), rounded to bf16, then fast::rope (non-traditional,
 *       scale 1, at each token's position), rounded to bf16;
 *   V = v_norm(v_proj) -- RMSNormNoScale (norm.rs:16-29), f32 -- or, with
 *       v_from_k, v_norm of the raw K (K==V global layers, :54-59).
 * rope_dims = head_dim * partial_rotary_factor (config.rs:209-225), a power
 * of 2 in [2 * head_dim / 64, head_dim]. Every cache mode: affine and
 * codebook caches quantize the prologue's output (V in f32), a plain cache
 * stores it rounded to bf16. */
typedef struct fmkv_kv_prologue {
  const void* k_norm_weight; /* bf16 [head_dim], device */
  float eps;                 /* rms_norm_eps (k_norm and v_norm) */
  int32_t rope_dims;
  float rope_theta;
  int32_t v_from_k;          /* 1: V is taken from k_proj (v_proj ignored, may be NULL) */
} fmkv_kv_prologue;

/* fmkv_cache_append of raw projections through the prologue; RoPE positions
 * start at the cache offset (the reference's cache.offset(), :73). */
int fmkv_cache_append_projected(fmkv_cache* cache, const void* k_proj_bf16,
                                const void* v_proj_bf16, int64_t n_tokens,
                                const fmkv_kv_prologue* prologue, void* stream);

/* One decode step of an attention layer, as Gemma4Attention::forward runs it
 * (src/model/gemma4_attention.rs:84-103): cache.update_and_fetch(k, v) for
 * n_tokens new positions, then attention of q over every visible position --
 * fmkv_cache_append followed by fmkv_decode_attention. With one new token
 * and sparse_v_tau == 0 this is, in every mode, a single attention launch
 * (plus the split combine) whose new-token column also appends the token;
 * with sparse_v_tau > 0 the statistics pass's new-token column appends it
 * (then the gather, or the gated pass and the combine: see
 * fmkv_set_sparse_v_gather). Arguments and errors as those two
 * calls; nothing is launched or changed when validation fails. */
int fmkv_decode_step(fmkv_cache* cache, const void* k_bf16, const void* v_bf16, int64_t n_tokens,
                     const void* q_bf16, int32_t n_q_heads, float scale, float sparse_v_tau,
                     void* out, int32_t out_dtype, void* stream);

/* fmkv_decode_step of raw projections: the layer's prologue (see
 * fmkv_kv_prologue) on the n_tokens new rows at positions offset ..
 * offset + n_tokens - 1, their store, then the attention read -- the whole
 * of Gemma4Attention::forward after the q/k/v projections for L == n_tokens
 * (src/model/gemma4_attention.rs:50-104; q arrives normed and roped). With
 * one new token the prologue, quantization and store run inside the
 * attention launch's new-token column (one launch plus the split combine;
 * with sparse_v_tau > 0 inside the statistics pass's); otherwise
 * fmkv_cache_append_projected, then fmkv_decode_attention. Every cache mode;
 * errors as those calls. */
int fmkv_decode_step_projected(fmkv_cache* cache, const void* k_proj_bf16,
                               const void* v_proj_bf16, int64_t n_tokens,
                               const fmkv_kv_prologue* prologue, const void* q_bf16,
                               int32_t n_q_heads, float scale, float sparse_v_tau, void* out,
                               int32_t out_dtype, void* stream);

/* Bytes of device scratch behind fmkv_decode_step_noalloc (per GPU). */
#define FMKV_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

/* fmkv_decode_step with no device allocation: no counterpart in the
 * reference; for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The same
 * kernels run, with the split partials in a fixed per-GPU scratch of
 * FMKV_NOALLOC_SCRATCH_BYTES held until the process ends instead of the
 * handle's growable workspace: P = (splits + 1) * n_q_heads rows of split
 * partials take P * (head_dim + 2) * 4 bytes; with sparse_v_tau > 0 add
 * 12 * n_q_heads bytes of softmax statistics, P * 8 bytes of the statistics
 * pass's split (m, l), padding to 16 bytes, and 32 * n_kv_heads * blocks
 * bytes of per-block score maxima (blocks = visible 16-token blocks of the
 * call); sparse-V's gather (fmkv_set_sparse_v_gather) also takes
 * 512 * n_kv_heads * blocks bytes of block scores and 4 * n_q_heads bytes of
 * counters, and where those do not fit the call runs the gated pass instead.
 * A call needing more gets FMKV_ERR_CAPACITY and nothing is launched (a
 * 32K-token head_dim-512 layer with 16 q heads needs about 4 MiB dense,
 * 4.2 MiB with sparse-V, 6.3 MiB with its gather). All calls on one GPU
 * share that scratch: calls that overlap in time on one GPU (other streams,
 * other threads) race. */
int fmkv_decode_step_noalloc(fmkv_cache* cache, const void* k_bf16, const void* v_bf16,
                             int64_t n_tokens, const void* q_bf16, int32_t n_q_heads, float scale,
                             float sparse_v_tau, void* out, int32_t out_dtype, void* stream);

/* One prefill (chunked-prefill) pass of an attention layer, as
 * Gemma4Attention::forward runs it for L = n_tokens > 1
 * (src/model/gemma4_attention.rs:84-104): cache.update_and_fetch(k, v) of the
 * chunk, then attention of its n_tokens queries q [n_tokens][n_q_heads][D]
 * (bf16, post-RoPE) with the mask of create_attention_mask (global layers) or
 * create_sliding_mask (sliding layers, src/model/mod.rs:682-753): query
 * position p attends to the visible positions j <= p, and on a ring of W
 * slots also j > p - W. A ring attends before its slots are overwritten (the
 * chunk's rows are quantized into a handle-owned staging area first), so
 * every query sees its whole window. out: [n_tokens][n_q_heads][D] in
 * out_dtype. Every cache mode (codebook caches are read as stored, plain
 * caches as their bf16 rows); at most 8 query heads per KV head;
 * n_tokens >= 1. Nothing is launched or changed when validation fails. */
int fmkv_prefill_step(fmkv_cache* cache, const void* k_bf16, const void* v_bf16, int64_t n_tokens,
                      const void* q_bf16, int32_t n_q_heads, float scale, void* out,
                      int32_t out_dtype, void* stream);

/* The fetch half of update_and_fetch and KVCache::peek_kv (src/cache.rs:247-257):
 * dequantized, un-rotated K and V of the visible positions in chronological
 * order, [stored_len][n_kv_heads][head_dim] in out_dtype (plain caches: the
 * stored bf16 rows). */
int fmkv_cache_fetch(const fmkv_cache* cache, void* k_out, void* v_out, int32_t out_dtype,
                     void* stream);

/* Raw stored codes in a canonical layout, indexed by slot (slot = pos % W for
 * rings, pos for linear caches), for bit-exact checks:
 *   codes  uint32 [n_slots][2][n_kv_heads][words]   (K = 0, V = 1; LE bit stream)
 *   meta   uint16 [n_slots][2][n_kv_heads][n_meta]  (affine: scale g, bias g
 *          interleaved, n_meta = 2*head_dim/64; codebook: norm, n_meta = 1;
 *          plain: n_meta = 0 and meta may be NULL)
 * Plain caches: words = head_dim / 2, the bf16 row (dim 2w in the low half
 * of word w). n_slots = window for rings, capacity for linear caches. */
int fmkv_cache_read_codes(const fmkv_cache* cache, void* codes, void* meta, void* stream);

/* ---------------------------------------------------------------------- */
/* Paged pool for batched, ragged decode (block tables of 16-token blocks). */
/* The reference has no paged cache (one Vec<Cache> per request,            */
/* src/engine.rs:70); this is the batched form of the same append/read.     */
/* ---------------------------------------------------------------------- */

typedef struct fmkv_pool fmkv_pool;

/* Pool of n_blocks physical 16-token blocks, each holding all KV heads. */
int fmkv_pool_create(const fmkv_cache_desc* desc, int64_t n_blocks, fmkv_pool** out);
int fmkv_pool_destroy(fmkv_pool* pool);

/* Append n_new tokens to each of n_seqs sequences. k/v: bf16
 * [n_seqs][n_new][n_kv_heads][head_dim]. block_tables: int32 device
 * [n_seqs][max_blocks]; start_pos: int32 device [n_seqs], the position of
 * each sequence's first new token. */
int fmkv_paged_append(fmkv_pool* pool, const void* k_bf16, const void* v_bf16,
                      const int32_t* block_tables, int32_t max_blocks, const int32_t* start_pos,
                      int32_t n_seqs, int32_t n_new, void* stream);

/* fmkv_paged_append of raw projections through the prologue (see
 * fmkv_cache_append_projected); RoPE positions start at start_pos. */
int fmkv_paged_append_projected(fmkv_pool* pool, const void* k_proj_bf16, const void* v_proj_bf16,
                                const int32_t* block_tables, int32_t max_blocks,
                                const int32_t* start_pos, int32_t n_seqs, int32_t n_new,
                                const fmkv_kv_prologue* prologue, void* stream);

/* Decode attention for n_seqs sequences; seq_lens: int32 device [n_seqs]
 * (positions visible, current token included); max_seq_len bounds them.
 * q: bf16 [n_seqs][n_q_heads][head_dim]; out: [n_seqs][n_q_heads][head_dim].
 * scale and sparse_v_tau as in fmkv_decode_attention. */
int fmkv_paged_decode_attention(fmkv_pool* pool, const void* q_bf16, const int32_t* block_tables,
                                int32_t max_blocks, const int32_t* seq_lens, int32_t n_seqs,
                                int32_t max_seq_len, int32_t n_q_heads, float scale,
                                float sparse_v_tau, void* out, int32_t out_dtype, void* stream);

/* Batched decode step: fmkv_paged_append of n_new tokens per sequence at
 * start_pos, then fmkv_paged_decode_attention with seq_lens (which the
 * caller sets to start_pos + n_new) -- the per-layer sequence of
 * src/model/gemma4_attention.rs:84-103 for a batch of requests. With one new
 * token per sequence the attention launch appends the tokens itself (at
 * seq_lens - 1; with sparse_v_tau > 0 the statistics pass does). */
int fmkv_paged_decode_step(fmkv_pool* pool, const void* k_bf16, const void* v_bf16,
                           const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* start_pos, const int32_t* seq_lens, int32_t n_seqs,
                           int32_t n_new, int32_t max_seq_len, const void* q_bf16,
                           int32_t n_q_heads, float scale, float sparse_v_tau, void* out,
                           int32_t out_dtype, void* stream);

/* fmkv_paged_decode_step of raw projections through the layer's prologue
 * (see fmkv_decode_step_projected); RoPE positions start at start_pos. */
int fmkv_paged_decode_step_projected(fmkv_pool* pool, const void* k_proj_bf16,
                                     const void* v_proj_bf16, const int32_t* block_tables,
                                     int32_t max_blocks, const int32_t* start_pos,
                                     const int32_t* seq_lens, int32_t n_seqs, int32_t n_new,
                                     int32_t max_seq_len, const fmkv_kv_prologue* prologue,
                                     const void* q_bf16, int32_t n_q_heads, float scale,
                                     float sparse_v_tau, void* out, int32_t out_dtype,
                                     void* stream);

/* Batched chunked prefill: fmkv_paged_append of n_new tokens per sequence at
 * start_pos, then each sequence's causal attention of those n_new queries
 * over its positions [0, start_pos + i] (src/model/gemma4_attention.rs
 * :84-104 with L > 1, mask of create_attention_mask, src/model/mod.rs
 * :682-704) -- fmkv_prefill_step for a batch of requests. q: bf16
 * [n_seqs][n_new][n_q_heads][head_dim]; out: the same shape in out_dtype.
 * Every cache mode; at most 8 query heads per KV head. */
int fmkv_paged_prefill_step(fmkv_pool* pool, const void* k_bf16, const void* v_bf16,
                            const int32_t* block_tables, int32_t max_blocks,
                            const int32_t* start_pos, int32_t n_seqs, int32_t n_new,
                            const void* q_bf16, int32_t n_q_heads, float scale, void* out,
                            int32_t out_dtype, void* stream);

/* Canonical codes of every pool block, indexed by (physical block * 16 + t). */
int fmkv_pool_read_codes(const fmkv_pool* pool, void* codes, void* meta, void* stream);

/* ---------------------------------------------------------------------- */
/* Tuning and introspection                                                 */
/* ---------------------------------------------------------------------- */

/* Blocks per split-K work-group for decode attention (0 = automatic). In a
 * paged pool each sequence's first split takes 4 x that many blocks when the
 * grid holds at least four work-groups per CU. */
int fmkv_set_blocks_per_split(int32_t blocks_per_split);

/* Sparse-V (sparse_v_tau > 0) after its statistics pass: 1 (the default)
 * reads the V rows of the kept tokens only, in one launch that writes the
 * output; 0 runs the gated pass over the blocks that hold kept tokens and
 * the split merge. Both give the reference's result
 * (src/model/gemma4_attention.rs:196-234); the gather also falls back to the
 * gated pass beyond 262144 visible tokens per sequence, or when the
 * no-allocation scratch cannot hold its score rows. No reference
 * counterpart (a tuning and test switch). */
int fmkv_set_sparse_v_gather(int32_t on);

/* Kernel timing (profiling aid, no reference counterpart): while enabled,
 * each decode attention call records a pair of HIP events around its split-K
 * kernel on the caller's stream, up to max_records pairs (0 disables and
 * frees them). fmkv_profile_collect waits for the recorded pairs, returns the
 * summed kernel time in milliseconds and the number of launches timed, and
 * clears the records. */
int fmkv_profile_enable(int32_t max_records);
int fmkv_profile_collect(double* total_ms, int32_t* n_records);
/* As fmkv_profile_collect, but writes each recorded launch's kernel time in
 * milliseconds to ms_out[0 .. *n_records) (FMKV_ERR_CAPACITY when capacity
 * is smaller than the number of records). */
int fmkv_profile_collect_each(float* ms_out, int32_t capacity, int32_t* n_records);
/* Split columns per KV head that the next fmkv_decode_attention call on
 * `cache` will launch (for profiling; the decode step adds its new-token
 * column to these and plans around it). */
int fmkv_cache_decode_splits(const fmkv_cache* cache, int32_t* n_splits);

#ifdef __cplusplus
}
#endif
#endif /* FMKV_H */
