/*
 * kv_oracle.h -- CPU restatement of tiny-llm's KV-cache decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
 * (tiny-llm_amd/) is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never links it and
 * never falls back to it.
 *
 * What it restates (reference = AICL-Lab/tiny-llm v2.0.2):
 *   - KVCacheManager bookkeeping, layout and byte-copy append
 *       src/kv_cache.cpp:8-297, include/tiny_llm/kv_cache.h:15-111
 *   - attention_decode_kernel arithmetic
 *       kernels/attention.cu:11-112 (launcher :114-128)
 *   - the call-site contract of TransformerLayer::attention
 *       src/transformer.cpp:222-237 (scale = 1/sqrt(D), attended = len + 1)
 *
 * The GQA / cache-layout generalisation of the decode math (query head h reads
 * kv head h / (Hq/Hkv) straight out of the token-major cache, optionally through
 * a block table) is a decision of this build, not reference behaviour: the
 * reference kernel only knows the compact [B][H][S][D] layout.
 *
 * Pinning status of each function is listed at the top of kv_oracle.c.
 *
 * All fp16 values travel as raw IEEE-754 binary16 bit patterns (uint16_t).
 */
#ifndef TINYLLM_KV_ORACLE_H
#define TINYLLM_KV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE-754 binary16 <-> binary32 (round to nearest even) ------------- */
float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
void     orc_h2f_n(const uint16_t *src, float *dst, size_t n);
void     orc_f2h_n(const float *src, uint16_t *dst, size_t n);

/* ---- seeded normal generator: splitmix64 -> Box-Muller -> fp16 RNE ------ */
void orc_fill_normal_f16(uint64_t seed, float stddev, uint16_t *out, size_t n);

/* ---- KVCacheManager restatement (host pool) ----------------------------- */
typedef struct {
    int num_layers;     /* KVCacheConfig::num_layers   (types.h:123) */
    int num_heads;      /* KVCacheConfig::num_heads == num_kv_heads (types.h:124) */
    int head_dim;       /* KVCacheConfig::head_dim     (types.h:125) */
    int max_seq_len;    /* KVCacheConfig::max_seq_len  (types.h:126) */
    int max_batch_size; /* KVCacheConfig::max_batch_size (types.h:127) */
} orc_kv_config;

typedef struct orc_kv orc_kv;

/* Every function returning int: 0 on success, -1 on error with the
 * reference's error message copied into err (if err != NULL). */
int    orc_kv_create(const orc_kv_config *cfg, orc_kv **out, char *err, int errlen);
void   orc_kv_destroy(orc_kv *kv);
int    orc_kv_allocate(orc_kv *kv, int max_len, int *seq_id, char *err, int errlen);
int    orc_kv_release(orc_kv *kv, int seq_id, char *err, int errlen);
/* getCacheChecked: element offsets of the K and V regions inside the pool. */
int    orc_kv_get_cache(const orc_kv *kv, int seq_id, int layer, size_t *k_off, size_t *v_off,
                        char *err, int errlen);
/* appendKV: new_k/new_v are [num_tokens][num_heads][head_dim]. */
int    orc_kv_append(orc_kv *kv, int seq_id, int layer, const uint16_t *new_k,
                     const uint16_t *new_v, int num_tokens, char *err, int errlen);
int    orc_kv_advance(orc_kv *kv, int seq_id, int num_tokens, char *err, int errlen);
int    orc_kv_seq_len(const orc_kv *kv, int seq_id);
int    orc_kv_has(const orc_kv *kv, int seq_id);
int    orc_kv_slot_of(const orc_kv *kv, int seq_id); /* -1 if absent */
size_t orc_kv_used(const orc_kv *kv);
size_t orc_kv_total(const orc_kv *kv);
size_t orc_kv_free(const orc_kv *kv);
int    orc_kv_active(const orc_kv *kv);
size_t orc_kv_slot_bytes(const orc_kv *kv);
uint16_t       *orc_kv_pool(orc_kv *kv);
size_t          orc_kv_pool_elems(const orc_kv *kv);

/* ---- cache view: how (sequence b, kv head g, token t) maps to memory ----
 *   elem(b,g,t) = base + blk(b, t >> log2_blk) * blk_stride
 *                      + (t & (2^log2_blk - 1)) * tok_stride + g * head_stride
 *   blk(b, j)   = block_table ? block_table[b * bt_stride + j] : b
 * The reference cache (kv_cache.cpp:69-80, 226-233) is the view with
 *   base = pool + layer*2*M*Hkv*D (+ M*Hkv*D for V), block = slot index,
 *   log2_blk = 30 (one block per sequence), blk_stride = 2*L*M*Hkv*D,
 *   tok_stride = Hkv*D, head_stride = D.
 * The compact [B][H][S][D] layout of attention.cu:12-14 is
 *   block_table = NULL, log2_blk = 30, blk_stride = H*S*D, tok_stride = D,
 *   head_stride = S*D.                                                      */
typedef struct {
    const uint16_t *k_base;
    const uint16_t *v_base;
    const int32_t  *block_table;
    int             bt_stride;
    int             log2_blk;
    int64_t         blk_stride;
    int64_t         tok_stride;
    int64_t         head_stride;
} orc_kv_view;

/* Decode attention, reference arithmetic, GQA over a cache view.
 * q: [B][Hq][D]; seq_lens[b] = attended length S_b; out: [B][Hq][D].
 * out_f32 (may be NULL) receives the fp32 value before the final fp16 round,
 * out_f16 (may be NULL) the RNE-rounded value. nthreads <= 0: one thread.   */
void orc_attn_decode_gqa(const uint16_t *q, const orc_kv_view *kv, const int32_t *seq_lens,
                         int B, int Hq, int Hkv, int D, float scale, float *out_f32,
                         uint16_t *out_f16, int nthreads);
/* The same function with the same arithmetic per (b, h) row (the same bits),
 * vectorised (AVX2 + F16C: eight tokens per register for the scores, eight d
 * for P.V) and reading each K/V row once per GQA group: the timing form of
 * the CPU baseline.  head_dim not a multiple of 8 falls back to
 * orc_attn_decode_gqa. */
void orc_attn_decode_gqa_fast(const uint16_t *q, const orc_kv_view *kv, const int32_t *seq_lens,
                              int B, int Hq, int Hkv, int D, float scale, float *out_f32,
                              uint16_t *out_f16, int nthreads);

/* Literal attention_decode contract: compact [B][H][S][D] K/V, MHA. */
void orc_attention_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *out_f32,
                          uint16_t *out_f16, float scale, int B, int H, int S, int D);

/* attention_prefill (attention.cu:131-237): compact [B][H][S][D] Q/K/V/out,
 * MHA; row (b, h, i) scores every key p < S, masked to -FLT_MAX for p > i,
 * then softmax with 1/(sum+1e-6) and o_d = sum over all S keys of w_p v_pd.
 * Silent no-op on non-positive dimensions (:228-230).  out_f32 may be NULL. */
void orc_attention_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           float *out_f32, uint16_t *out_f16, float scale, int B, int H, int S,
                           int D, int nthreads);

/* softmax (attention.cu:288-354): rows of S fp16 values, softmax with
 * 1/(sum+1e-6), fp16 output.  out_f32 may be NULL. */
void orc_softmax(const uint16_t *in, float *out_f32, uint16_t *out_f16, int rows, int S);

/* get_attention_weights (attention.cu:240-286): fp16(scale * q.k) for every
 * (b, h, query i, key p) of [B][H][Lq][Lk]; 0 where causal and p > i.  No
 * softmax.  out_f32 (may be NULL) holds the value before rounding. */
void orc_get_attention_weights(const uint16_t *q, const uint16_t *k, float *out_f32,
                               uint16_t *out_f16, float scale, int B, int H, int Lq, int Lk, int D,
                               int causal);

/* Gather: out[b][g][t][d] = cache(b,g,t,d) for t < seq_lens[b], 0 otherwise.
 * out is [B][Hkv][S_max][D]; which = 0 gathers K, 1 gathers V.             */
/* ---- W8A16 matmul (kernels/w8a16_matmul.cu:71-98, the reference kernel
 * that w8a16_matmul also uses for M*N < 4096, :225-228):
 *   out[m][n] = fp16( sum_k f(x[m][k]) * ((float)w[k][n] * f(s[k/gs][n])) )
 * summed over k in order in fp32; `sum += a * w` is an FMA under nvcc's
 * default contraction (--fmad=true), so each step is fmaf(a, w, sum).
 * Silent no-op on non-positive dimensions (:101-104).  out_f32 may be NULL. */
void orc_w8a16_matmul(const uint16_t *x, const int8_t *w, const uint16_t *s, float *out_f32,
                      uint16_t *out_f16, int M, int N, int K, int group_size);

/* add_inplace (kernels/elementwise.cu:7-14): data[i] = fp16(f(data[i]) + f(add[i])). */
void orc_add_inplace(uint16_t *data, const uint16_t *add, size_t n);

void orc_kv_gather(const orc_kv_view *kv, int which, const int32_t *seq_lens, int B, int Hkv,
                   int D, int S_max, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
