// extern "C" surface of libtinyllm_kv.so (declared in include/tinyllm_kv.h).
// Thin: argument marshalling, Result -> status code, exceptions -> TL_ERR_HIP.
#include "tinyllm_kv.h"

#include "kernels/kv_kernels.h"
#include "kernels/prefill.h"
#include "runtime.h"
#include "tiny_llm/kernels/attention.h"
#include "tiny_llm/kv_cache.h"
#include "tl_log.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace tiny_llm {
namespace detail {
std::string attn_decode_view(const __half *q, const KvView &kv, const int32_t *seq_lens_host, int B,
                             int Hq, int Hkv, int D, float scale, __half *out, hipStream_t stream);
std::string attn_decode_compact(const __half *q, const __half *k, const __half *v, __half *out,
                                float scale, int B, int H, int S, int D, hipStream_t stream);
std::string attn_prefill_compact(const __half *q, const __half *k, const __half *v, __half *out,
                                 float scale, int B, int H, int S, int D, hipStream_t stream);
std::string w8a16_call(const __half *x, const int8_t *w, const __half *s, __half *out, int M, int N,
                       int K, int gs, bool residual, hipStream_t stream, bool packed);
std::string w8a16_pack_call(const int8_t *w, int K, int N, int8_t *out, hipStream_t stream);
void        w8a16_force_generic(int on);
} // namespace detail
} // namespace tiny_llm

using tiny_llm::DecodeBatch;
using tiny_llm::PrefillBatch;
using tiny_llm::KVCacheManager;
using tiny_llm::Result;

struct tl_kv_manager {
    std::unique_ptr<KVCacheManager> m;
};
struct tl_kv_batch {
    std::unique_ptr<DecodeBatch> b;
};

struct tl_kv_prefill {
    std::unique_ptr<PrefillBatch> b;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

template <typename T>
int status(const Result<T> &r) {
    if (r.isOk()) {
        g_last_error.clear();
        return TL_OK;
    }
    return fail(TL_ERR_INVALID, r.error());
}

// Runs f(); maps exceptions to status codes.
template <typename F>
int guarded(F &&f) {
    try {
        return f();
    } catch (const tiny_llm::HipException &e) {
        return fail(TL_ERR_HIP, e.what());
    } catch (const std::exception &e) {
        return fail(TL_ERR_INVALID, e.what());
    }
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }
const half *as_half(const void *p) { return static_cast<const half *>(p); }
half       *as_half(void *p) { return static_cast<half *>(p); }

} // namespace

extern "C" {

const char *tl_last_error(void) { return g_last_error.c_str(); }

const char *tl_version(void) {
#ifdef TL_ATTN_PV_DOT2
    return "tinyllm_kv 0.1.0 gfx950 (comparison build: decode P.V on v_dot2)";
#else
    return "tinyllm_kv 0.1.0 gfx950";
#endif
}

int tl_kv_create(const tl_kv_config *cfg, tl_kv_manager **out) {
    if (!out) return fail(TL_ERR_INVALID, "tl_kv_create: out is null");
    *out = nullptr;
    if (!cfg) return fail(TL_ERR_INVALID, "tl_kv_create: cfg is null");
    return guarded([&] {
        tiny_llm::KVCacheConfig c;
        c.num_layers = cfg->num_layers;
        c.num_heads = cfg->num_heads;
        c.head_dim = cfg->head_dim;
        c.max_seq_len = cfg->max_seq_len;
        c.max_batch_size = cfg->max_batch_size;
        auto r = KVCacheManager::create(c);
        if (r.isErr()) return fail(TL_ERR_INVALID, r.error());
        *out = new tl_kv_manager{std::move(r.value())};
        g_last_error.clear();
        return TL_OK;
    });
}

void tl_kv_destroy(tl_kv_manager *mgr) { delete mgr; }

int tl_kv_allocate_sequence(tl_kv_manager *mgr, int max_len, int *seq_id) {
    if (!mgr || !seq_id) return fail(TL_ERR_INVALID, "tl_kv_allocate_sequence: null argument");
    auto r = mgr->m->allocateSequence(max_len);
    if (r.isOk()) *seq_id = r.value();
    return status(r);
}

int tl_kv_release_sequence(tl_kv_manager *mgr, int seq_id) {
    if (!mgr) return fail(TL_ERR_INVALID, "tl_kv_release_sequence: null manager");
    return status(mgr->m->releaseSequence(seq_id));
}

int tl_kv_get_cache(tl_kv_manager *mgr, int seq_id, int layer, void **k_cache, void **v_cache) {
    if (!mgr) return fail(TL_ERR_INVALID, "tl_kv_get_cache: null manager");
    auto r = mgr->m->getCacheChecked(seq_id, layer);
    if (k_cache) *k_cache = r.isOk() ? r.value().first : nullptr;
    if (v_cache) *v_cache = r.isOk() ? r.value().second : nullptr;
    return status(r);
}

int tl_kv_append(tl_kv_manager *mgr, int seq_id, int layer, const void *new_k, const void *new_v,
                 int num_tokens, void *stream) {
    if (!mgr) return fail(TL_ERR_INVALID, "tl_kv_append: null manager");
    return guarded([&] {
        return status(mgr->m->appendKV(seq_id, layer, as_half(new_k), as_half(new_v), num_tokens,
                                       as_stream(stream)));
    });
}

int tl_kv_advance(tl_kv_manager *mgr, int seq_id, int num_tokens) {
    if (!mgr) return fail(TL_ERR_INVALID, "tl_kv_advance: null manager");
    return status(mgr->m->advanceSeqLen(seq_id, num_tokens));
}

int tl_kv_seq_len(const tl_kv_manager *mgr, int seq_id) { return mgr ? mgr->m->getSeqLen(seq_id) : 0; }
int tl_kv_has_sequence(const tl_kv_manager *mgr, int seq_id) {
    return mgr && mgr->m->hasSequence(seq_id) ? 1 : 0;
}
size_t tl_kv_used_memory(const tl_kv_manager *mgr) { return mgr ? mgr->m->getUsedMemory() : 0; }
size_t tl_kv_total_memory(const tl_kv_manager *mgr) { return mgr ? mgr->m->getTotalMemory() : 0; }
size_t tl_kv_free_memory(const tl_kv_manager *mgr) { return mgr ? mgr->m->getFreeMemory() : 0; }
int    tl_kv_active_count(const tl_kv_manager *mgr) {
    return mgr ? mgr->m->getActiveSequenceCount() : 0;
}

int tl_kv_get_config(const tl_kv_manager *mgr, tl_kv_config *out) {
    if (!mgr || !out) return fail(TL_ERR_INVALID, "tl_kv_get_config: null argument");
    const auto &c = mgr->m->getConfig();
    out->num_layers = c.num_layers;
    out->num_heads = c.num_heads;
    out->head_dim = c.head_dim;
    out->max_seq_len = c.max_seq_len;
    out->max_batch_size = c.max_batch_size;
    return TL_OK;
}

void  *tl_kv_pool(const tl_kv_manager *mgr) { return mgr ? mgr->m->pool() : nullptr; }
size_t tl_kv_slot_bytes(const tl_kv_manager *mgr) { return mgr ? mgr->m->slotBytes() : 0; }
int    tl_kv_slot_of(const tl_kv_manager *mgr, int seq_id) { return mgr ? mgr->m->slotOf(seq_id) : -1; }

int tl_kv_create_paged(const tl_kv_config *cfg, int block_tokens, int num_blocks,
                       tl_kv_manager **out) {
    if (!out) return fail(TL_ERR_INVALID, "tl_kv_create_paged: out is null");
    *out = nullptr;
    if (!cfg) return fail(TL_ERR_INVALID, "tl_kv_create_paged: cfg is null");
    return guarded([&] {
        tiny_llm::KVCacheConfig c;
        c.num_layers = cfg->num_layers;
        c.num_heads = cfg->num_heads;
        c.head_dim = cfg->head_dim;
        c.max_seq_len = cfg->max_seq_len;
        c.max_batch_size = cfg->max_batch_size;
        auto r = KVCacheManager::createPaged(c, block_tokens, num_blocks);
        if (r.isErr()) return fail(TL_ERR_INVALID, r.error());
        *out = new tl_kv_manager{std::move(r.value())};
        g_last_error.clear();
        return TL_OK;
    });
}

int    tl_kv_num_blocks(const tl_kv_manager *mgr) { return mgr ? mgr->m->numBlocks() : 0; }
int    tl_kv_free_blocks(const tl_kv_manager *mgr) { return mgr ? mgr->m->freeBlocks() : 0; }
size_t tl_kv_block_bytes(const tl_kv_manager *mgr) { return mgr ? mgr->m->blockBytes() : 0; }

int tl_kv_block_table(const tl_kv_manager *mgr, int seq_id, int32_t *out, int *n) {
    if (!mgr || !n || (*n > 0 && !out)) return fail(TL_ERR_INVALID, "tl_kv_block_table: null argument");
    return guarded([&] {
        auto r = mgr->m->blockTable(seq_id);
        if (r.isErr()) return fail(TL_ERR_INVALID, r.error());
        const auto &t = r.value();
        const int   m = static_cast<int>(t.size());
        for (int i = 0; i < std::min(*n, m); ++i) out[i] = t[static_cast<size_t>(i)];
        *n = m;
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_kv_set_block_map(tl_kv_manager *mgr, int block_tokens, const int32_t *perm, size_t n) {
    if (!mgr) return fail(TL_ERR_INVALID, "tl_kv_set_block_map: null manager");
    return guarded([&] { return status(mgr->m->setBlockMap(block_tokens, perm, n)); });
}

int tl_kv_batch_create(tl_kv_manager *mgr, int max_seqs, int num_q_heads, tl_kv_batch **out) {
    if (!mgr || !out) return fail(TL_ERR_INVALID, "tl_kv_batch_create: null argument");
    *out = nullptr;
    return guarded([&] {
        auto r = DecodeBatch::create(*mgr->m, max_seqs, num_q_heads);
        if (r.isErr()) return fail(TL_ERR_INVALID, r.error());
        *out = new tl_kv_batch{std::move(r.value())};
        g_last_error.clear();
        return TL_OK;
    });
}

void tl_kv_batch_destroy(tl_kv_batch *batch) { delete batch; }

int tl_kv_batch_prepare(tl_kv_batch *batch, const int *seq_ids, int n, void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_prepare: null batch");
    return guarded([&] { return status(batch->b->prepare(seq_ids, n, as_stream(stream))); });
}

int tl_kv_batch_prepare_lengths(tl_kv_batch *batch, const int *seq_ids, const int *attended, int n,
                                void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_prepare_lengths: null batch");
    return guarded(
        [&] { return status(batch->b->prepareLengths(seq_ids, attended, n, as_stream(stream))); });
}

int tl_kv_batch_info(const tl_kv_batch *batch, int *n, int *chunk_tokens, int *work_items) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_info: null batch");
    if (n) *n = batch->b->size();
    if (chunk_tokens) *chunk_tokens = batch->b->chunkTokens();
    if (work_items) *work_items = batch->b->workItems();
    return TL_OK;
}

int tl_kv_batch_append(tl_kv_batch *batch, int layer_begin, int num_layers, const void *new_k,
                       const void *new_v, void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_append: null batch");
    return guarded([&] {
        return status(batch->b->append(layer_begin, num_layers, as_half(new_k), as_half(new_v),
                                       as_stream(stream)));
    });
}

int tl_kv_batch_attention(tl_kv_batch *batch, int layer, const void *q, void *out, float scale,
                          void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_attention: null batch");
    return guarded([&] {
        return status(batch->b->attention(layer, as_half(q), as_half(out), scale, as_stream(stream)));
    });
}

int tl_kv_batch_decode(tl_kv_batch *batch, int layer, const void *q, const void *new_k,
                       const void *new_v, void *out, float scale, void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_decode: null batch");
    return guarded([&] {
        return status(batch->b->decode(layer, as_half(q), as_half(new_k), as_half(new_v),
                                       as_half(out), scale, as_stream(stream)));
    });
}

int tl_kv_batch_gather(tl_kv_batch *batch, int layer, void *k_out, void *v_out, int s_max,
                       void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_gather: null batch");
    return guarded([&] {
        return status(batch->b->gather(layer, as_half(k_out), as_half(v_out), s_max, as_stream(stream)));
    });
}

int tl_kv_batch_project(tl_kv_batch *batch, int layer, const void *x, int hidden, int group_size,
                        const int8_t *wk, const void *sk, const int8_t *wv, const void *sv,
                        const int8_t *wq, const void *sq, void *q_out, int packed, void *stream) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_project: null batch");
    return guarded([&] {
        return status(batch->b->project(layer, as_half(x), hidden, group_size, wk, as_half(sk), wv,
                                        as_half(sv), wq, as_half(sq), as_half(q_out),
                                        as_stream(stream), packed != 0));
    });
}

int tl_kv_batch_commit(tl_kv_batch *batch, int num_tokens) {
    if (!batch) return fail(TL_ERR_INVALID, "tl_kv_batch_commit: null batch");
    return guarded([&] { return status(batch->b->commit(num_tokens)); });
}

int tl_attn_decode_gqa(const void *q, const tl_kv_view *kv, const int32_t *seq_lens_host, int B,
                       int Hq, int Hkv, int D, float scale, void *out, void *stream) {
    if (!kv) return fail(TL_ERR_INVALID, "tl_attn_decode_gqa: kv is null");
    return guarded([&] {
        tiny_llm::detail::KvView v;
        v.k_base = as_half(kv->k_base);
        v.v_base = as_half(kv->v_base);
        v.block_table = kv->block_table;
        v.seq_row = nullptr;
        v.bt_stride = kv->bt_stride;
        v.log2_blk = kv->log2_blk;
        v.blk_stride = kv->blk_stride;
        v.tok_stride = kv->tok_stride;
        v.head_stride = kv->head_stride;
        const std::string err = tiny_llm::detail::attn_decode_view(
            as_half(q), v, seq_lens_host, B, Hq, Hkv, D, scale, as_half(out), as_stream(stream));
        if (!err.empty()) return fail(TL_ERR_INVALID, err);
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_attn_decode_gqa_noalloc(const void *q, const tl_kv_view *kv, const int32_t *seq_lens_host,
                               int B, int Hq, int Hkv, int D, float scale, void *out,
                               void *stream) {
    if (!kv) return fail(TL_ERR_INVALID, "tl_attn_decode_gqa_noalloc: kv is null");
    return guarded([&] {
        tiny_llm::detail::KvView v;
        v.k_base = as_half(kv->k_base);
        v.v_base = as_half(kv->v_base);
        v.block_table = kv->block_table;
        v.seq_row = nullptr;
        v.bt_stride = kv->bt_stride;
        v.log2_blk = kv->log2_blk;
        v.blk_stride = kv->blk_stride;
        v.tok_stride = kv->tok_stride;
        v.head_stride = kv->head_stride;
        const std::string err = tiny_llm::detail::attn_decode_view_noalloc(
            as_half(q), v, seq_lens_host, B, Hq, Hkv, D, scale, as_half(out), as_stream(stream));
        if (!err.empty()) return fail(TL_ERR_INVALID, err);
        g_last_error.clear();
        return TL_OK;
    });
}

size_t tl_attn_noalloc_scratch_bytes(void) { return tiny_llm::detail::attn_noalloc_scratch_bytes(); }

int tl_w8a16_matmul(const void *input, const int8_t *weight, const void *scales, void *output, int M,
                    int N, int K, int group_size, void *stream) {
    return guarded([&] {
        const std::string err = tiny_llm::detail::w8a16_call(as_half(input), weight, as_half(scales),
                                                             as_half(output), M, N, K, group_size,
                                                             false, as_stream(stream), false);
        if (!err.empty()) return fail(TL_ERR_INVALID, err);
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_w8a16_matmul_residual(const void *input, const int8_t *weight, const void *scales,
                             void *hidden, int M, int N, int K, int group_size, int packed,
                             void *stream) {
    return guarded([&] {
        const std::string err = tiny_llm::detail::w8a16_call(as_half(input), weight, as_half(scales),
                                                             as_half(hidden), M, N, K, group_size,
                                                             true, as_stream(stream), packed != 0);
        if (!err.empty()) return fail(TL_ERR_INVALID, err);
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_w8a16_pack(const int8_t *weight, int K, int N, int8_t *packed, void *stream) {
    return guarded([&] {
        const std::string err =
            tiny_llm::detail::w8a16_pack_call(weight, K, N, packed, as_stream(stream));
        if (!err.empty()) return fail(TL_ERR_INVALID, err);
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_w8a16_set_path(int path) {
    if (path != 0 && path != 1) return fail(TL_ERR_INVALID, "tl_w8a16_set_path: path must be 0 or 1");
    tiny_llm::detail::w8a16_force_generic(path);
    g_last_error.clear();
    return TL_OK;
}

void tl_attention_decode(const void *q, const void *k, const void *v, void *out, float scale,
                         int batch, int num_heads, int seq_len, int head_dim, void *stream) {
    if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return;
    (void)guarded([&] {
        const std::string err = tiny_llm::detail::attn_decode_compact(
            as_half(q), as_half(k), as_half(v), as_half(out), scale, batch, num_heads, seq_len,
            head_dim, as_stream(stream));
        if (!err.empty()) {
            TL_LOG_ERROR("%s", err.c_str());
            return fail(TL_ERR_INVALID, err);
        }
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_kv_prefill_create(tl_kv_manager *mgr, int max_seqs, int num_q_heads, tl_kv_prefill **out) {
    if (!mgr || !out) return fail(TL_ERR_INVALID, "tl_kv_prefill_create: null argument");
    *out = nullptr;
    return guarded([&] {
        auto r = PrefillBatch::create(*mgr->m, max_seqs, num_q_heads);
        if (r.isErr()) return fail(TL_ERR_INVALID, r.error());
        *out = new tl_kv_prefill{std::move(r.value())};
        g_last_error.clear();
        return TL_OK;
    });
}

void tl_kv_prefill_destroy(tl_kv_prefill *p) { delete p; }

int tl_kv_prefill_prepare(tl_kv_prefill *p, const int *seq_ids, const int *num_tokens, int n,
                          void *stream) {
    if (!p) return fail(TL_ERR_INVALID, "tl_kv_prefill_prepare: null batch");
    return guarded([&] { return status(p->b->prepare(seq_ids, num_tokens, n, as_stream(stream))); });
}

int tl_kv_prefill_info(const tl_kv_prefill *p, int *n, int *tokens) {
    if (!p || !n || !tokens) return fail(TL_ERR_INVALID, "tl_kv_prefill_info: null argument");
    *n = p->b->size();
    *tokens = p->b->tokens();
    return TL_OK;
}

int tl_kv_prefill_append(tl_kv_prefill *p, int layer, const void *new_k, const void *new_v,
                         void *stream) {
    if (!p) return fail(TL_ERR_INVALID, "tl_kv_prefill_append: null batch");
    return guarded([&] {
        return status(p->b->append(layer, as_half(new_k), as_half(new_v), as_stream(stream)));
    });
}

int tl_kv_prefill_attention(tl_kv_prefill *p, int layer, const void *q, void *out, float scale,
                            void *stream) {
    if (!p) return fail(TL_ERR_INVALID, "tl_kv_prefill_attention: null batch");
    return guarded([&] {
        return status(p->b->attention(layer, as_half(q), as_half(out), scale, as_stream(stream)));
    });
}

int tl_kv_prefill_run(tl_kv_prefill *p, int layer, const void *q, const void *new_k,
                      const void *new_v, void *out, float scale, void *stream) {
    if (!p) return fail(TL_ERR_INVALID, "tl_kv_prefill_run: null batch");
    return guarded([&] {
        return status(p->b->prefill(layer, as_half(q), as_half(new_k), as_half(new_v), as_half(out),
                                    scale, as_stream(stream)));
    });
}

int tl_kv_prefill_commit(tl_kv_prefill *p) {
    if (!p) return fail(TL_ERR_INVALID, "tl_kv_prefill_commit: null batch");
    return guarded([&] { return status(p->b->commit()); });
}

int tl_prefill_set_waves(int waves) {
    if (waves != 0 && waves != 4 && waves != 8)
        return fail(TL_ERR_INVALID, "tl_prefill_set_waves: waves must be 0 (auto), 4 or 8");
    tiny_llm::detail::set_prefill_waves(waves);
    return TL_OK;
}

int tl_prefill_get_waves(void) { return tiny_llm::detail::prefill_waves_setting(); }

int tl_prefill_plan_waves(const int32_t *prefix_lens, const int32_t *num_tokens, int n,
                          int num_q_heads, int num_kv_heads, int head_dim, int num_cus, int *waves) {
    namespace d = tiny_llm::detail;
    if (!waves) return fail(TL_ERR_INVALID, "tl_prefill_plan_waves: waves is null");
    if (n < 0 || (n > 0 && (!prefix_lens || !num_tokens)))
        return fail(TL_ERR_INVALID, "tl_prefill_plan_waves: invalid lengths");
    if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 || num_cus < 0 ||
        !d::prefill_shape_supported(head_dim, num_q_heads / num_kv_heads))
        return fail(TL_ERR_INVALID, "tl_prefill_plan_waves: unsupported heads, head_dim or num_cus");
    std::vector<d::PrefillEntry> e(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) {
        if (prefix_lens[i] < 0 || num_tokens[i] < 1)
            return fail(TL_ERR_INVALID, "tl_prefill_plan_waves: invalid lengths");
        e[static_cast<size_t>(i)] = {0, prefix_lens[i], num_tokens[i], i, 0};
    }
    return guarded([&] {
        *waves = d::prefill_waves(e.data(), n, head_dim, num_q_heads / num_kv_heads, num_kv_heads,
                                  num_cus > 0 ? num_cus : d::device_cus());
        return TL_OK;
    });
}

void tl_attention_prefill(const void *q, const void *k, const void *v, void *out, float scale,
                          int batch, int num_heads, int seq_len, int head_dim, void *stream) {
    if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return;
    (void)guarded([&] {
        const std::string err = tiny_llm::detail::attn_prefill_compact(
            as_half(q), as_half(k), as_half(v), as_half(out), scale, batch, num_heads, seq_len,
            head_dim, as_stream(stream));
        if (!err.empty()) {
            TL_LOG_ERROR("%s", err.c_str());
            return fail(TL_ERR_INVALID, err);
        }
        g_last_error.clear();
        return TL_OK;
    });
}

void tl_softmax(const void *input, void *output, int batch, int seq_len, void *stream) {
    tiny_llm::kernels::softmax(as_half(input), as_half(output), batch, seq_len, as_stream(stream));
}

void tl_get_attention_weights(const void *q, const void *k, void *weights, float scale, int batch,
                              int num_heads, int query_len, int key_len, int head_dim, int causal,
                              void *stream) {
    tiny_llm::kernels::get_attention_weights(as_half(q), as_half(k), as_half(weights), scale, batch,
                                             num_heads, query_len, key_len, head_dim, causal != 0,
                                             as_stream(stream));
}

int tl_attn_set_score_path(int path) {
    if (path < 0 || path > 3)
        return fail(TL_ERR_INVALID,
                    "tl_attn_set_score_path: path must be 0 (valu), 1 (mfma), 2 (auto) or 3 (mma)");
    tiny_llm::detail::set_score_path(path);
    return TL_OK;
}

int tl_attn_get_score_path(void) { return tiny_llm::detail::score_path(); }

int tl_attn_set_waves(int waves) {
    if (waves != 0 && waves != 4 && waves != 8)
        return fail(TL_ERR_INVALID, "tl_attn_set_waves: waves must be 0 (auto), 4 or 8");
    tiny_llm::detail::set_waves(waves);
    return TL_OK;
}

int tl_attn_get_waves(void) { return tiny_llm::detail::waves(); }

int tl_attn_set_head_fuse(int mode) {
    if (mode != 0 && mode != 1 && mode != 2 && mode != 4 && mode != 8)
        return fail(TL_ERR_INVALID,
                    "tl_attn_set_head_fuse: mode must be 0 (auto), 1 (off), 2, 4 or 8 (heads per workgroup)");
    tiny_llm::detail::set_head_fuse(mode);
    return TL_OK;
}

int tl_attn_get_head_fuse(void) { return tiny_llm::detail::head_fuse(); }

int tl_attn_set_fused_merge(int on) {
    if (on != 0 && on != 1)
        return fail(TL_ERR_INVALID, "tl_attn_set_fused_merge: on must be 0 (second launch) or 1 (in the launch)");
    tiny_llm::detail::set_fused_merge(on != 0);
    return TL_OK;
}

int tl_attn_get_fused_merge(void) { return tiny_llm::detail::fused_merge_enabled() ? 1 : 0; }

int tl_attn_plan(const int32_t *seq_lens, int n, int num_kv_heads, int head_dim, int num_cus,
                 int forced_chunk, int waves_setting, int head_fuse, int with_rows,
                 tl_attn_plan_info *info, int32_t *part_base, int32_t *work) {
    if (!info) return fail(TL_ERR_INVALID, "tl_attn_plan: info is null");
    if (n < 0 || (n > 0 && !seq_lens)) return fail(TL_ERR_INVALID, "tl_attn_plan: invalid lengths");
    if (num_kv_heads <= 0 || num_cus <= 0)
        return fail(TL_ERR_INVALID, "tl_attn_plan: num_kv_heads and num_cus must be positive");
    if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(TL_ERR_INVALID, "tl_attn_plan: head_dim must be 32, 64, 128 or 256");
    if (waves_setting != 0 && waves_setting != 4 && waves_setting != 8)
        return fail(TL_ERR_INVALID, "tl_attn_plan: waves_setting must be 0 (auto), 4 or 8");
    if (head_fuse != TL_PLAN_HF_CURRENT && head_fuse != 0 && head_fuse != 1 && head_fuse != 2 &&
        head_fuse != 4 && head_fuse != 8)
        return fail(TL_ERR_INVALID, "tl_attn_plan: head_fuse must be TL_PLAN_HF_CURRENT (-1), "
                                    "0 (auto), 1 (off), 2, 4 or 8");
    if (forced_chunk < 0) return fail(TL_ERR_INVALID, "tl_attn_plan: forced_chunk must be >= 0");
    for (int i = 0; i < n; ++i)
        if (seq_lens[i] < 0) return fail(TL_ERR_INVALID, "tl_attn_plan: negative sequence length");
    return guarded([&] {
        namespace d = tiny_llm::detail;
        d::WorkList wl;
        int fuse; // planner argument: 0 = per head, 1 = auto, 2 / 4 / 8 = forced
        if (head_fuse == TL_PLAN_HF_CURRENT) {
            // exactly the entry points' plan: the process settings
            if (forced_chunk == 0) forced_chunk = d::chunk_override_from_env();
            if (waves_setting == 0) waves_setting = d::waves();
            fuse = d::planner_head_fuse(head_dim);
        } else {
            // the setter's codes; a head-fused form exists for head_dim 128
            // when waves are not forced to 4
            fuse = head_dim != 128 || waves_setting == 4 || head_fuse == 1 ? 0
                   : head_fuse == 0                                        ? 1
                                                                           : head_fuse;
        }
        d::plan_work_list(seq_lens, n, num_kv_heads, num_cus, forced_chunk, fuse, wl);
        info->chunk_tokens = wl.chunk;
        info->work_items = wl.n_work;
        info->waves = !wl.n_work       ? 0
                      : wl.fused_heads ? 8
                                      : d::plan_waves((int64_t)wl.n_work * num_kv_heads, num_cus,
                                                      waves_setting);
        info->head_fused = wl.fused_heads;
        info->fused_chunked = wl.fused_chunked ? 1 : 0;
        info->any_multi = wl.any_multi ? 1 : 0;
        info->any_empty = wl.any_empty ? 1 : 0;
        info->max_len = wl.max_len;
        const int words = d::inline_words(wl, n, with_rows != 0);
        info->inline_compact = 0;
        if (n > 0 && words <= d::kInlineWords) {
            info->inline_words = words;
        } else {
            // the compact encoding stores a row per entry either way
            const int cw = d::inline_words_compact(seq_lens, wl, nullptr, n);
            info->inline_compact = (cw > 0 && cw <= d::kInlineWords) ? 1 : 0;
            info->inline_words = info->inline_compact ? cw : -1;
        }
        if (part_base) std::memcpy(part_base, wl.part_base.data(), wl.part_base.size() * 4);
        if (work && wl.n_work) std::memcpy(work, wl.work.data(), wl.work.size() * 4);
        g_last_error.clear();
        return TL_OK;
    });
}

int tl_fill_normal_f16(uint64_t seed, uint64_t first, float stddev, void *out, size_t n,
                       void *stream) {
    if (n == 0) return TL_OK;
    if (!out) return fail(TL_ERR_INVALID, "tl_fill_normal_f16: out is null");
    return guarded([&] {
        tiny_llm::detail::launch_fill_normal(seed, first, stddev, static_cast<__half *>(out), n,
                                             static_cast<hipStream_t>(stream));
        g_last_error.clear();
        return TL_OK;
    });
}

void tl_profile_enable(int on) { tiny_llm::detail::profile_set(on != 0); }
void tl_profile_reset(void) { tiny_llm::detail::profile_reset(); }

int tl_profile_query(const char *kernel, double *total_ms, long long *launches) {
    static const char *names[] = {"attn_chunk", "attn_merge",   "kv_append",   "kv_gather",
                                  "w8a16",      "w8a16_reduce", "attn_prefill"};
    constexpr int      kNames = static_cast<int>(sizeof(names) / sizeof(names[0]));
    static_assert(kNames == static_cast<int>(tiny_llm::detail::KernelId::Count), "profile names");
    if (!kernel || !total_ms || !launches) return fail(TL_ERR_INVALID, "tl_profile_query: null argument");
    for (int i = 0; i < kNames; ++i)
        if (std::strcmp(kernel, names[i]) == 0)
            return guarded([&] {
                tiny_llm::detail::profile_query(i, total_ms, launches);
                return TL_OK;
            });
    return fail(TL_ERR_INVALID, std::string("tl_profile_query: unknown kernel ") + kernel);
}

} // extern "C"
