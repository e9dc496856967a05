/*
 * tinyllm_kv.h -- C ABI of libtinyllm_kv.so, the MI355X (gfx950) KV-cache
 * decode path of tiny-llm: per-step K/V append, block/slot gather and GQA
 * decode attention over the cache.
 *
 * Plain pointers and sizes only.  fp16 tensors are passed as `void *` device
 * pointers holding IEEE binary16 values; streams are `void *` holding a
 * hipStream_t (NULL = the default stream).  Every `int` result is TL_OK (0) or
 * a negative status; tl_last_error() returns the message of the last failing
 * call on the calling thread.  Every entry point is asynchronous with respect
 * to the host exactly where its reference counterpart is (stream-ordered
 * device work, synchronous host bookkeeping).
 *
 * Reference = AICL-Lab/tiny-llm v2.0.2.  Each declaration names the reference
 * interface it replaces (file:line).  The C++ mirror of the same API
 * (tiny_llm::KVCacheManager, tiny_llm::kernels::attention_decode) lives in
 * tiny-llm_amd/include/tiny_llm/ and is exported from the same library.
 */
#ifndef TINYLLM_KV_H
#define TINYLLM_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TL_OK 0
#define TL_ERR_INVALID (-1) /* host validation failed: Result::err(...) in the reference */
#define TL_ERR_HIP (-2)     /* HIP runtime failure: CudaException via CUDA_CHECK */

/* Message of the last failing call on this thread ("" if none). */
const char *tl_last_error(void);

/* Library version string, e.g. "tinyllm_kv 0.1.0 gfx950". */
const char *tl_version(void);

/* ------------------------------------------------------------------------
 * KVCacheManager (include/tiny_llm/kv_cache.h:24-111, src/kv_cache.cpp)
 * Same semantics and the same pool layout:
 *   pool = [slot][layer][K|V][max_seq_len][num_heads][head_dim] fp16.
 * ---------------------------------------------------------------------- */

/* KVCacheConfig (include/tiny_llm/types.h:122-128); num_heads = KV heads. */
typedef struct tl_kv_config {
    int num_layers;
    int num_heads;
    int head_dim;
    int max_seq_len;
    int max_batch_size;
} tl_kv_config;

typedef struct tl_kv_manager tl_kv_manager;

/* KVCacheManager::create (kv_cache.cpp:8-60): validates, hipMalloc + zero. */
int tl_kv_create(const tl_kv_config *cfg, tl_kv_manager **out);
/* ~KVCacheManager (kv_cache.cpp:62-67). NULL is accepted. */
void tl_kv_destroy(tl_kv_manager *mgr);
/* allocateSequence (kv_cache.cpp:91-119): lowest free slot, monotonically
 * increasing ids; error text contains "exhausted" when no slot is free. */
int tl_kv_allocate_sequence(tl_kv_manager *mgr, int max_len, int *seq_id);
/* releaseSequence (kv_cache.cpp:121-137): device bytes are not cleared. */
int tl_kv_release_sequence(tl_kv_manager *mgr, int seq_id);
/* getCacheChecked (kv_cache.cpp:139-157): device pointers of the (seq,
 * layer) K and V regions ([max_seq_len][num_heads][head_dim] each).  Fails
 * for paged pools (tl_kv_set_block_map), which have no contiguous region. */
int tl_kv_get_cache(tl_kv_manager *mgr, int seq_id, int layer, void **k_cache, void **v_cache);
/* appendKV (kv_cache.cpp:168-238): copies num_tokens tokens of
 * [num_tokens][num_heads][head_dim] fp16 K and V to the sequence tail
 * (current_len) on `stream`; does NOT advance the visible length. */
int tl_kv_append(tl_kv_manager *mgr, int seq_id, int layer, const void *new_k, const void *new_v,
                 int num_tokens, void *stream);
/* advanceSeqLen (kv_cache.cpp:240-259): clamps to the sequence's max_len. */
int tl_kv_advance(tl_kv_manager *mgr, int seq_id, int num_tokens);
/* getSeqLen (kv_cache.cpp:261-267): 0 for an unknown sequence. */
int tl_kv_seq_len(const tl_kv_manager *mgr, int seq_id);
/* hasSequence (kv_cache.cpp:269-271). */
int tl_kv_has_sequence(const tl_kv_manager *mgr, int seq_id);
/* getUsedMemory / getTotalMemory / getFreeMemory (kv_cache.cpp:273-286). */
size_t tl_kv_used_memory(const tl_kv_manager *mgr);
size_t tl_kv_total_memory(const tl_kv_manager *mgr);
size_t tl_kv_free_memory(const tl_kv_manager *mgr);
/* getActiveSequenceCount (kv_cache.cpp:288-295). */
int tl_kv_active_count(const tl_kv_manager *mgr);
/* getConfig (kv_cache.h:83). */
int tl_kv_get_config(const tl_kv_manager *mgr, tl_kv_config *out);
/* Device base of the pool and the per-slot byte size (slot_size_,
 * kv_cache.cpp:28); no reference accessor exists, these expose the private
 * memory_pool_ / slot_size_ for parity checks of the whole pool. */
void  *tl_kv_pool(const tl_kv_manager *mgr);
size_t tl_kv_slot_bytes(const tl_kv_manager *mgr);
/* Slot index of a live sequence (seq_to_slot_, kv_cache.h:104), -1 if absent. */
int tl_kv_slot_of(const tl_kv_manager *mgr, int seq_id);

/* Paged addressing over the same pool (build addition; the reference layout
 * is the identity map).  Logical block x = slot*(max_seq_len/block_tokens)+j
 * (token block j of that slot) is stored at physical block perm[x] of the
 * same geometry; every layer's K and V region uses the same map.  perm must
 * be a permutation of [0, max_batch_size*max_seq_len/block_tokens); it is
 * copied.  block_tokens must be a power of two dividing max_seq_len.
 * perm == NULL restores the reference layout. */
int tl_kv_set_block_map(tl_kv_manager *mgr, int block_tokens, const int32_t *perm, size_t n);

/* Block-granular pool (build addition; replaces the full-slot reservation
 * of allocateSequence, kv_cache.cpp:91-119).  The pool holds num_blocks
 * blocks of block_tokens tokens (a power of two >= 16), each with every
 * layer's K and V of those tokens, plus one spare block that unmapped table
 * entries point to:
 *   [layer][K|V][num_blocks + 1][block_tokens][num_heads][head_dim]  fp16.
 * max_batch_size bounds the live sequences.  tl_kv_append, tl_kv_advance and
 * tl_kv_batch_prepare map the blocks they need (all or nothing per call) and
 * fail with "KV cache exhausted" when too few are free; release returns a
 * sequence's blocks.  Used/total/free memory count blocks of
 * tl_kv_block_bytes.  tl_kv_get_cache fails (no contiguous region). */
int tl_kv_create_paged(const tl_kv_config *cfg, int block_tokens, int num_blocks,
                       tl_kv_manager **out);
/* Blocks in the pool / free now (0 for other pools). */
int    tl_kv_num_blocks(const tl_kv_manager *mgr);
int    tl_kv_free_blocks(const tl_kv_manager *mgr);
/* Bytes of one block (all layers, K and V); 0 for other pools. */
size_t tl_kv_block_bytes(const tl_kv_manager *mgr);
/* Physical blocks of a sequence in token order: writes min(*n, mapped) ids
 * to out and sets *n to the number mapped.  Block pools: ids of
 * tl_kv_create_paged's layout; a block map over the slot pool
 * (tl_kv_set_block_map): all max_seq_len/block_tokens ids of the sequence's
 * slot, counted in blocks of block_tokens tokens from a layer's K base. */
int tl_kv_block_table(const tl_kv_manager *mgr, int seq_id, int32_t *out, int *n);

/* ------------------------------------------------------------------------
 * Batched decode surface (build addition layered on the manager).  The
 * reference decodes one sequence per call: TransformerLayer::attention
 * (src/transformer.cpp:222-237) does getCache -> appendKV(n=1) ->
 * attention_decode(q, K*, V*, out, 1/sqrt(D), 1, Hq, getSeqLen+1, D) per
 * layer, and InferenceEngine::decodeStep commits with advanceSeqLen(seq, 1)
 * after all layers (src/inference_engine.cpp:287-291).  A batch snapshots
 * that state for n sequences once per step; every layer then appends and
 * attends through it.  Query head h reads KV head h / (num_q_heads/num_heads).
 * ---------------------------------------------------------------------- */
typedef struct tl_kv_batch tl_kv_batch;

/* A batch of at most max_seqs sequences with num_q_heads query heads. */
int tl_kv_batch_create(tl_kv_manager *mgr, int max_seqs, int num_q_heads, tl_kv_batch **out);
void tl_kv_batch_destroy(tl_kv_batch *batch);
/* Snapshot for a decode step: for each seq_ids[i] (distinct, live),
 * write position = getSeqLen (kv_cache.cpp:208), attended length = write
 * position + 1 (transformer.cpp:230-235).  Fails like appendKV(n=1) when a
 * sequence is full.  Uploads the step's metadata on `stream`. */
int tl_kv_batch_prepare(tl_kv_batch *batch, const int *seq_ids, int n, void *stream);
/* Like prepare, but with explicit attended lengths and no append slot:
 * attended[i] tokens of seq_ids[i] (1 <= attended[i] <= its max_len) are
 * read by attention/gather; append is rejected for such a batch. */
int tl_kv_batch_prepare_lengths(tl_kv_batch *batch, const int *seq_ids, const int *attended, int n,
                                void *stream);
/* Size, split-K chunk length (tokens per work item) and work-item count of
 * the last prepare; any pointer may be NULL.  No reference counterpart. */
int tl_kv_batch_info(const tl_kv_batch *batch, int *n, int *chunk_tokens, int *work_items);
/* Fused append of one token per (sequence, layer) for layers
 * [layer_begin, layer_begin + num_layers): new_k/new_v are
 * [num_layers][n][num_heads][head_dim] fp16.  Byte-identical to n*num_layers
 * appendKV(seq, layer, k_row, v_row, 1) calls (kv_cache.cpp:226-233). */
int tl_kv_batch_append(tl_kv_batch *batch, int layer_begin, int num_layers, const void *new_k,
                       const void *new_v, void *stream);
/* GQA decode attention of every batch entry at `layer`: q and out are
 * [n][num_q_heads][head_dim] fp16; replaces the per-sequence
 * attention_decode call of transformer.cpp:236-237 (math of
 * kernels/attention.cu:11-112). */
int tl_kv_batch_attention(tl_kv_batch *batch, int layer, const void *q, void *out, float scale,
                          void *stream);
/* The whole decode branch of TransformerLayer::attention for one layer
 * (transformer.cpp:222-237): append the new token, then attend over
 * attended = write position + 1, in one stream-ordered call. */
int tl_kv_batch_decode(tl_kv_batch *batch, int layer, const void *q, const void *new_k,
                       const void *new_v, void *out, float scale, void *stream);
/* Gather of the attended tokens into compact head-major layout (the K/V
 * layout attention_decode reads, kernels/attention.cuh:10-13):
 * k_out/v_out are [n][num_heads][s_max][head_dim]; tokens at or beyond a
 * sequence's attended length are written as +0.0.  Either output may be NULL. */
int tl_kv_batch_gather(tl_kv_batch *batch, int layer, void *k_out, void *v_out, int s_max,
                       void *stream);
/* DecodeBatch projection with the append fused into its epilogue
 * (transformer.cpp:214-226: w8a16_matmul of wk/wv into k_buf_/v_buf_, then
 * appendKV(n=1)): for every entry i of the last prepare,
 *   K_i = x_i @ dequant(wk, sk), V_i = x_i @ dequant(wv, sv)
 * (W8A16 arithmetic of kernels/w8a16_matmul.cu) are written straight into
 * the cache of `layer` at the entry's write position -- byte-identical to
 * tl_w8a16_matmul into a buffer followed by tl_kv_append(n=1).  x:
 * [n][hidden] fp16; wk/wv: [hidden][num_heads*head_dim] int8; sk/sv:
 * [ceil(hidden/group_size)][num_heads*head_dim] fp16.  Optionally (wq, sq,
 * q_out all non-NULL) q_out[n][num_q_heads*head_dim] = x @ dequant(wq, sq) in
 * the same launch.  packed != 0: all weights are in the layout of
 * tl_w8a16_pack (hidden % 32 == 0 and group_size in {32, 64, 128, 256,
 * 512}); the MFMA kernel reads both layouts into the same fragments and
 * sums in the same order, so the bytes equal the reference layout's.  Does
 * not advance lengths (commit does). */
int tl_kv_batch_project(tl_kv_batch *batch, int layer, const void *x, int hidden, int group_size,
                        const int8_t *wk, const void *sk, const int8_t *wv, const void *sv,
                        const int8_t *wq, const void *sq, void *q_out, int packed, void *stream);
/* The commit of InferenceEngine::decodeStep (src/inference_engine.cpp:291):
 * advanceSeqLen(seq_id, num_tokens) for every sequence of the last prepare,
 * in batch order; stops at (and reports) the first failing sequence. */
int tl_kv_batch_commit(tl_kv_batch *batch, int num_tokens);

/* ------------------------------------------------------------------------
 * Stateless kernels over an explicit cache view (no manager).
 * ---------------------------------------------------------------------- */

/* Element offset of (sequence b, kv head g, token t) relative to k_base or
 * v_base:  blk(b, t >> log2_blk) * blk_stride + (t & (2^log2_blk - 1)) *
 * tok_stride + g * head_stride, with blk(b, j) = block_table[b*bt_stride+j]
 * (device int32) or b when block_table is NULL.  Strides are in elements. */
typedef struct tl_kv_view {
    const void    *k_base;
    const void    *v_base;
    const int32_t *block_table;
    int            bt_stride;
    int            log2_blk;
    int64_t        blk_stride;
    int64_t        tok_stride;
    int64_t        head_stride;
} tl_kv_view;

/* GQA decode attention over a view.  seq_lens_host[b] (host memory) is the
 * attended length of entry b (0 gives a zero output row).  q/out:
 * [B][Hq][D] fp16 device.  head_dim in {32, 64, 128, 256}, Hq/Hkv in
 * {1, 2, 4, 8}.  Uses library-owned device workspace. */
int tl_attn_decode_gqa(const void *q, const tl_kv_view *kv, const int32_t *seq_lens_host, int B,
                       int Hq, int Hkv, int D, float scale, void *out, void *stream);

/* tl_attn_decode_gqa without any allocation: no hipMalloc, hipFree, pinned
 * host memory or host-to-device copy, so it can run under HIP graph capture
 * or where the caller forbids allocation.  No counterpart in the reference:
 * it exists for callers that cannot allocate.  Same arguments, launches and
 * results (bit for bit) as tl_attn_decode_gqa; the split-K partials and, for
 * plans too large for the kernel arguments, the plan metadata go to a static
 * device array of tl_attn_noalloc_scratch_bytes() bytes (16 MiB) that each GPU
 * holds until the process ends.  A call that would need more is rejected
 * with TL_ERR_INVALID: per split item Hq*(D+2)*4 bytes of partials, plus
 * 4*(2B+1+2*items) bytes of metadata when that exceeds 896 words.  All calls
 * on one GPU share its array (the last call's contents stay): calls that
 * overlap on one GPU race. */
int tl_attn_decode_gqa_noalloc(const void *q, const tl_kv_view *kv, const int32_t *seq_lens_host,
                               int B, int Hq, int Hkv, int D, float scale, void *out, void *stream);
/* Size in bytes of the static scratch array of tl_attn_decode_gqa_noalloc. */
size_t tl_attn_noalloc_scratch_bytes(void);

/* attention_decode (kernels/attention.cuh:15-18, attention.cu:114-128):
 * q [B][H][D], k/v [B][H][S][D], out [B][H][D] fp16 device pointers.
 * Silently returns on non-positive dimensions, like the reference. */
void tl_attention_decode(const void *q, const void *k, const void *v, void *out, float scale,
                         int batch, int num_heads, int seq_len, int head_dim, void *stream);

/* attention_prefill (kernels/attention.cuh:20-26, attention.cu:131-237):
 * q/k/v/out [B][H][S][D] fp16 device pointers, causal (query i attends to
 * keys 0..i), softmax with 1/(sum+1e-6), MFMA with fp32 accumulation.
 * Silently returns on non-positive dimensions; head_dim in {32,64,128,256}. */
void tl_attention_prefill(const void *q, const void *k, const void *v, void *out, float scale,
                          int batch, int num_heads, int seq_len, int head_dim, void *stream);
/* softmax (kernels/attention.cuh:28-30, attention.cu:288-354): rows of
 * seq_len fp16 values, [batch][seq_len] in and out. */
void tl_softmax(const void *input, void *output, int batch, int seq_len, void *stream);
/* get_attention_weights (kernels/attention.cuh:32-36, attention.cu:240-286):
 * weights [B][H][query_len][key_len] = fp16(scale * q.k), 0 above the
 * diagonal when causal != 0; no softmax. */
void tl_get_attention_weights(const void *q, const void *k, void *weights, float scale, int batch,
                              int num_heads, int query_len, int key_len, int head_dim, int causal,
                              void *stream);

/* ------------------------------------------------------------------------
 * Prefill into the cache (build addition).  The reference's prefill branch
 * (src/transformer.cpp:214-241, inference_engine.cpp:233-272) appends the
 * prompt's K/V with appendKV(n) and runs attention_prefill over k_buf_/v_buf_;
 * this batch appends the new tokens of several sequences and runs causal
 * GQA attention of each new token over its sequence's cache (positions
 * 0 .. getSeqLen + j), so a prompt can also continue chunk by chunk.
 *   prepare: seq_ids[i] brings num_tokens[i] >= 1 new tokens (same checks and
 *            error texts as appendKV; block pools map the blocks needed);
 *   append:  new_k/new_v [T][num_heads*head_dim], sequences back to back,
 *            T = sum of num_tokens (bytes identical to appendKV per sequence);
 *   attention: q/out [T][num_q_heads][head_dim];
 *   run:     append + attention in one launch (same bytes and outputs; q,
 *            out, new_k and new_v 16-byte aligned);
 *   commit:  advanceSeqLen(seq_ids[i], num_tokens[i]).
 * num_q_heads / num_heads in {1,2,4,8}; head_dim in {32,64,128,256}. */
typedef struct tl_kv_prefill tl_kv_prefill;
int  tl_kv_prefill_create(tl_kv_manager *mgr, int max_seqs, int num_q_heads, tl_kv_prefill **out);
void tl_kv_prefill_destroy(tl_kv_prefill *p);
int  tl_kv_prefill_prepare(tl_kv_prefill *p, const int *seq_ids, const int *num_tokens, int n,
                           void *stream);
int  tl_kv_prefill_info(const tl_kv_prefill *p, int *n, int *tokens);
int  tl_kv_prefill_append(tl_kv_prefill *p, int layer, const void *new_k, const void *new_v,
                          void *stream);
int  tl_kv_prefill_attention(tl_kv_prefill *p, int layer, const void *q, void *out, float scale,
                             void *stream);
int  tl_kv_prefill_run(tl_kv_prefill *p, int layer, const void *q, const void *new_k,
                       const void *new_v, void *out, float scale, void *stream);
int  tl_kv_prefill_commit(tl_kv_prefill *p);

/* Waves per prefill-attention workgroup, process-wide: 0 = auto, 4 or 8
 * (8: one 256-row workgroup per CU; 4: two 128-row workgroups per CU, one's
 * start-up under the other's tiles).  Auto takes 4 at head_dim 64 (three
 * workgroups per CU), 8 at head_dim 32, and at head_dim 128 4 when the
 * 8-wave tiling gives every CU at least 3 work items ((entry, query tile) x
 * kv heads) that attend at most 800 keys on average, else 8; head_dim 256 is
 * always 4.  Initial value from the environment variable TL_PREFILL_WAVES
 * ("4" / "8"), else 0.  A prefill batch keeps the waves of its prepare; the
 * compact tl_attention_prefill chooses per call.  Every setting gives the
 * same outputs within the 1e-3 gate.  No reference counterpart (tuning
 * knob). */
int tl_prefill_set_waves(int waves);
int tl_prefill_get_waves(void);
/* The waves per workgroup the prefill entry points choose under the current
 * setting for n sequences with prefix_lens[i] cached and num_tokens[i] new
 * tokens (num_tokens[i] >= 1), num_q_heads / num_kv_heads in {1,2,4,8},
 * head_dim in {32,64,128,256}, on num_cus CUs (0: the current device's). */
int tl_prefill_plan_waves(const int32_t *prefix_lens, const int32_t *num_tokens, int n,
                          int num_q_heads, int num_kv_heads, int head_dim, int num_cus, int *waves);

/* w8a16_matmul (kernels/w8a16_matmul.cuh:22-26, w8a16_matmul.cu:219-236):
 * output[M][N] = fp16(input[M][K] @ dequant(weight[K][N] int8,
 * scales[ceil(K/group_size)][N] fp16)), fp32 accumulation.  Returns TL_OK
 * without work on non-positive dimensions, like the reference's silent
 * return.  MFMA path for K % 32 == 0, group_size in {32, 64, 128, 256, 512}, N % 16 == 0 and
 * 16-byte aligned input/weight; otherwise the reference's per-element order. */
int tl_w8a16_matmul(const void *input, const int8_t *weight, const void *scales, void *output, int M,
                    int N, int K, int group_size, void *stream);
/* o_proj + residual of TransformerLayer::forward (transformer.cpp:149-151,
 * 246-247; add_inplace of kernels/elementwise.cu:7-14) in one launch:
 * hidden[M][N] = fp16(f(hidden) + f(fp16(input @ dequant(weight, scales)))).
 * packed != 0: weight is in the layout of tl_w8a16_pack. */
int tl_w8a16_matmul_residual(const void *input, const int8_t *weight, const void *scales,
                             void *hidden, int M, int N, int K, int group_size, int packed,
                             void *stream);
/* One-time repack of a W8A16 weight [K][N] int8 (K % 32 == 0, N % 16 == 0)
 * into the layout the packed entry points read (K*N bytes, device to device,
 * stream-ordered): the B fragments of v_mfma_f32_16x16x32_f16, so the kernel
 * streams weights straight into MFMA operands.  Lane l = 0..63 of the
 * fragment of column block nb = n/16 and k step ks = k/32 holds rows
 * 32ks + 8(l/16) .. +7 of column 16nb + l%16 as offset-binary bytes (w + 128,
 * the bits of w ^ 0x80, which convert to fp16 without a sign fix-up).  Column
 * block nb takes the K*16 bytes from nb*K*16; in them steps 2p and 2p+1 share
 * the 1024 bytes from 1024p, lane l's 16 bytes at 16l (step 2p first), and a
 * last unpaired step (K % 64 == 32) takes 8 bytes per lane.  No reference counterpart (weights are static; an engine packs
 * them once at load, like model_loader.cpp's quantised tensors). */
int tl_w8a16_pack(const int8_t *weight, int K, int N, int8_t *packed, void *stream);
/* W8A16 kernel selection, process-wide: 0 = normal (MFMA where the shape
 * allows), 1 = always the reference-order kernel.  No reference counterpart
 * (test knob). */
int tl_w8a16_set_path(int path);

/* Score (q.K^T) path of the decode attention kernels, process-wide:
 * 0 = VALU v_dot2 over the loaded K rows, 1 = MFMA v_mfma_f32_16x16x32_f16
 * over an LDS-transposed K tile (head_dim <= 128; VALU above), 2 = auto,
 * which resolves to VALU for every supported group (<= 8): both paths are
 * HBM-bound and MFMA was never faster on the measured decode workloads;
 * 3 = both contractions on MFMA (S^T = K Q^T and O^T = V^T P^T, K/V quarters
 * streamed into LDS by DMA; head_dim 64 and 128, other head_dims take 2).
 * Both give results within the 1e-3 gate of the same oracle.  Initial value
 * from the environment variable TL_ATTN_QK ("valu" / "mfma" / "auto"), else
 * 2.  No reference counterpart (tuning knob). */
int tl_attn_set_score_path(int path);
int tl_attn_get_score_path(void);

/* Waves per decode-attention workgroup, process-wide: 4, 8, or 0 = auto (8
 * when the launch gives every CU at most two workgroups in turn, else two
 * 4-wave workgroups per CU whose ramp-up and drain overlap).  Initial value
 * from the environment variable TL_ATTN_WAVES ("4" / "8" / "auto"), else 0.
 * Every setting gives results within the same 1e-3 gate.  No reference
 * counterpart (tuning knob). */
int tl_attn_set_waves(int waves);
int tl_attn_get_waves(void);

/* Head-fused decode plans, process-wide: 0 = auto, 1 = off, 2 / 4 / 8 =
 * that many kv heads per workgroup where a plan with it applies.  A
 * head-fused plan (head_dim 128, the VALU score path, waves not forced to 4,
 * lengths within 10% of the longest, kv heads a multiple of H, at most one
 * (sequence, H-head block) per CU) gives one 8-wave workgroup H kv heads of
 * a work item -- wave w head w % H, tile slice w / H -- so it reads H heads'
 * pieces of each token row at once, and a sequence's work items interleave
 * its 64-token tiles.  Auto takes the H in {8, 4, 2} with the fewest items
 * per sequence (one item: no merge launch), the larger H on a tie.  Other
 * lengths keep the chunk plan, with H = 2 over its items where per-head
 * workgroups would have 4 waves (forced: the forced H).  Initial
 * value from the environment variable TL_ATTN_HF ("0" = off, "2" / "4" /
 * "8", else auto).  Every setting gives results within the same 1e-3 gate.
 * No reference counterpart (tuning knob). */
int tl_attn_set_head_fuse(int mode);
int tl_attn_get_head_fuse(void);

/* Where a multi-chunk decode plan merges its chunks' partials, process-wide:
 * 0 = in a second launch (attn_merge_kernel; default), 1 = inside the
 * attention launch (the workgroup that completes a sequence's last chunk of
 * a kv-head block merges them, after device-scope fences; measured slower
 * than the second launch on every plan timed).  Both give the same bits.
 * Plans with an empty sequence, and tl_attn_decode_gqa_noalloc, always take
 * the second launch.  Initial value from the environment variable
 * TL_ATTN_MERGE ("fused" = 1).  No reference counterpart (the reference's
 * decode kernel is one workgroup per (sequence, head), attention.cu:114-128). */
int tl_attn_set_fused_merge(int on);
int tl_attn_get_fused_merge(void);

/* The launch plan of the decode attention entry points (tl_kv_batch_attention,
 * tl_kv_batch_decode, tl_attn_decode_gqa) for attended lengths
 * seq_lens[0..n) at head_dim (32, 64, 128 or 256) on a device of num_cus
 * compute units -- host only, no GPU needed.
 * head_fuse = TL_PLAN_HF_CURRENT: the plan those entry points make now, under
 * this process's settings (tl_attn_get_head_fuse, tl_attn_get_waves,
 * tl_attn_get_score_path, TL_ATTN_CHUNK); forced_chunk / waves_setting of 0
 * then mean "the process setting" too.
 * head_fuse = 0 (auto), 1 (off), 2 / 4 / 8 (that many kv heads per
 * workgroup): the codes of tl_attn_set_head_fuse, as if set, with the VALU
 * score path; forced_chunk: 0 or a multiple of 256 tokens, as TL_ATTN_CHUNK
 * would force; waves_setting: 0 (auto), 4 or 8, as tl_attn_set_waves.  A
 * head-fused plan exists only for head_dim 128 with waves not forced to 4.
 * with_rows != 0 counts the slot row per entry that DecodeBatch passes.
 * Optional outputs: part_base[n + 1] (first partial row of each entry) and
 * work[2 * work_items] ((entry, chunk) pairs in launch order, longest
 * first).  No reference counterpart (planner introspection for tests and
 * tuning; the reference launches one workgroup per (sequence, head),
 * kernels/attention.cu:121-125). */
#define TL_PLAN_HF_CURRENT (-1)
typedef struct tl_attn_plan_info {
    int chunk_tokens;  /* tokens per work item, a multiple of 256 */
    int work_items;    /* workgroups of the attention launch / Hkv */
    int waves;         /* waves per workgroup (4 or 8; 0 when no work) */
    int any_multi;     /* some sequence spans several chunks: merge launch */
    int any_empty;     /* some sequence attends to zero tokens */
    int max_len;       /* longest attended length */
    int inline_words;  /* metadata words in the kernel arguments, -1: device copy */
    int inline_compact;/* 1: the compact encoding (one chunk per sequence; 16-bit
                          lengths and slots: one word per sequence + 16 bits
                          per work item) */
    int head_fused;    /* kv heads per 8-wave workgroup of a head-fused plan (2, 4
                          or 8), 0: per-head plan */
    int fused_chunked; /* 1: head-fused over the chunk plan's items (ragged
                          lengths); 0 with head_fused: a sequence's work items
                          interleave its tiles, chunk_tokens is the longest
                          length rounded up, work is in chunk-major order */
} tl_attn_plan_info;
int tl_attn_plan(const int32_t *seq_lens, int n, int num_kv_heads, int head_dim, int num_cus,
                 int forced_chunk, int waves_setting, int head_fuse, int with_rows,
                 tl_attn_plan_info *info, int32_t *part_base, int32_t *work);

/* Seeded normal fp16 values for synthetic inputs: out[j] (device, j < n) =
 * element first + j of the stream splitmix64(seed) -> Box-Muller (double)
 * -> x stddev -> fp32 -> fp16 round-to-nearest-even, where element pair P
 * takes splitmix64 calls 2P + 1 and 2P + 2 (cosine, then sine).  Element for
 * element the oracle's generator (oracle/kv_oracle.c, orc_fill_normal_f16),
 * so any range of a stream can be drawn on its own, on any host.  No
 * reference counterpart: the input generator of the benchmarks and tests. */
int tl_fill_normal_f16(uint64_t seed, uint64_t first, float stddev, void *out, size_t n,
                       void *stream);

/* ------------------------------------------------------------------------
 * Kernel timing (the reference has only an unused CudaEvent wrapper,
 * include/tiny_llm/cuda_streams.h:67-99).  When enabled, every launch of the
 * named kernels is bracketed by hipEvents on its own stream.
 * Names: "attn_chunk", "attn_merge", "kv_append", "kv_gather", "w8a16"
 * (the W8A16 GEMM kernel), "w8a16_reduce" (its split-K reduction).
 * ---------------------------------------------------------------------- */
void tl_profile_enable(int on);
void tl_profile_reset(void);
/* Synchronises the recorded events; total device milliseconds and launch
 * count of `kernel`.  Returns TL_ERR_INVALID for an unknown name. */
int tl_profile_query(const char *kernel, double *total_ms, long long *launches);

#ifdef __cplusplus
}
#endif
#endif
