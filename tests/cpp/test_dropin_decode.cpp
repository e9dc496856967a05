// C++ drop-in test: tiny-llm's decode call sequence, compiled with hipcc in
// the include order of the C++ drop-in (tiny-llm_amd/include first, then the
// caller's own include directory) and linked against libtinyllm_kv.so.
//
//  - reference_decode_branch: the decode branch of TransformerLayer::attention
//    (src/transformer.cpp:222-237) restated line for line for one sequence and
//    two layers -- getCache, appendKV(n=1), attended = getSeqLen + 1,
//    kernels::attention_decode(q, K*, V*, out, 1/sqrt(D), 1, num_heads,
//    attended, head_dim) -- with InferenceEngine's commit once per step after
//    all layers (inference_engine.cpp:287-291) and the input checks of
//    TransformerLayer::forward (transformer.cpp:123-141), whose errors go
//    through fmt-style TLLM_ERROR calls of the caller's logger.  Output
//    against the oracle's literal attention_decode on the same bytes (the
//    reference reads K*/V* as compact [H][S][D], kernels/attention.cu:12-14),
//    appended rows bit-exact.
//  - batched_gqa_decode: the batched replacement (DecodeBatch::prepare /
//    decode / commit) at group 4 against the oracle's GQA decode.
//
// Prints "ok <name>" per check and "library <path>" (the libtinyllm_kv.so it
// runs); any failure exits non-zero.
#include "tiny_llm/kernels/attention.h"
#include "tiny_llm/kv_cache.h"
#include "tiny_llm/logger.h" // the caller's logger: must not be the library's
#include "tiny_llm/types.h"
#include "tinyllm_kv.h"

#include "kv_oracle.h"

#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#ifndef TINYLLM_TEST_CALLER_LOGGER
#error "tiny_llm/logger.h resolved to a header other than the caller's"
#endif

using namespace tiny_llm;

#define CHECK(c)                                                                                   \
    do {                                                                                           \
        if (!(c)) {                                                                                \
            std::fprintf(stderr, "check failed: %s (%s:%d)\n", #c, __FILE__, __LINE__);          \
            std::exit(1);                                                                          \
        }                                                                                          \
    } while (0)
#define HIP_OK(call) CHECK((call) == hipSuccess)

namespace {

std::vector<uint16_t> normal_f16(uint64_t seed, size_t n) {
    std::vector<uint16_t> v(n);
    orc_fill_normal_f16(seed, 1.0f, v.data(), n);
    return v;
}

half *to_device(const std::vector<uint16_t> &h) {
    half *d = nullptr;
    HIP_OK(hipMalloc(reinterpret_cast<void **>(&d), h.size() * 2));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    return d;
}

std::vector<uint16_t> to_host(const half *d, size_t n) {
    std::vector<uint16_t> h(n);
    HIP_OK(hipMemcpy(h.data(), d, n * 2, hipMemcpyDeviceToHost));
    return h;
}

// Normwise max|a - b| / max(|a|, |b|) (tests/test_transformer.cu:80-92).
double rel_err(const std::vector<uint16_t> &got, const std::vector<float> &ref) {
    double num = 0, den = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
        const double a = orc_h2f(got[i]), b = ref[i];
        num = std::max(num, std::fabs(a - b));
        den = std::max(den, std::max(std::fabs(a), std::fabs(b)));
    }
    return den > 0 ? num / den : 0;
}

// TransformerLayer's attention sublayer, decode branch only, for one layer
// (src/transformer.cpp:203-237 without the projections: q_buf_, k_buf_ and
// v_buf_ hold the projected rows).
struct DecodeLayer {
    int         layer_idx_;
    ModelConfig config_;

    void forward_attention(const half *q_buf_, const half *k_buf_, const half *v_buf_,
                           half *attn_output_, KVCacheManager &kv_cache, int seq_id, int position,
                           hipStream_t stream) {
        // input checks of TransformerLayer::forward (transformer.cpp:123-141)
        if (position < 0 || position >= config_.max_seq_len) {
            TLLM_ERROR("forward: invalid position {} for layer {}, max_seq_len={}", position,
                       layer_idx_, config_.max_seq_len);
            return;
        }
        if (!kv_cache.hasSequence(seq_id)) {
            TLLM_ERROR("forward: invalid seq_id {} for layer {}", seq_id, layer_idx_);
            return;
        }
        const int num_tokens = 1;
        const int num_heads = config_.num_heads;
        const int head_dim = config_.head_dim;
        auto [k_cache, v_cache] = kv_cache.getCache(seq_id, layer_idx_);
        auto appended = kv_cache.appendKV(seq_id, layer_idx_, k_buf_, v_buf_, num_tokens, stream);
        if (appended.isErr()) TLLM_ERROR("forward: {}", appended.error());
        const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
        const int   current_seq_len = kv_cache.getSeqLen(seq_id);
        const int   attended_seq_len = current_seq_len + 1;
        kernels::attention_decode(q_buf_, k_cache, v_cache, attn_output_, scale, 1, num_heads,
                                  attended_seq_len, head_dim, stream);
    }
};

void reference_decode_branch() {
    ModelConfig mc;
    mc.num_layers = 2;
    mc.num_heads = 4;
    mc.num_kv_heads = 4; // attention_decode reads num_heads heads of the cache
    mc.head_dim = 64;
    mc.max_seq_len = 160;
    KVCacheConfig kc;
    kc.num_layers = mc.num_layers;
    kc.num_heads = mc.num_kv_heads;
    kc.head_dim = mc.head_dim;
    kc.max_seq_len = mc.max_seq_len;
    kc.max_batch_size = 2;
    auto created = KVCacheManager::create(kc);
    CHECK(created.isOk());
    auto &kv = *created.value();
    const int H = mc.num_heads, D = mc.head_dim, M = mc.max_seq_len, row = H * D, ctx = 37;
    auto      sid = kv.allocateSequence(M);
    CHECK(sid.isOk());
    const int seq = sid.value();
    // prefill of the context (InferenceEngine::prefill: appendKV per layer,
    // one advance after all layers)
    std::vector<half *> keep;
    for (int l = 0; l < mc.num_layers; ++l) {
        auto k = to_device(normal_f16(100 + l, (size_t)ctx * row));
        auto v = to_device(normal_f16(200 + l, (size_t)ctx * row));
        keep.push_back(k);
        keep.push_back(v);
        CHECK(kv.appendKV(seq, l, k, v, ctx, nullptr).isOk());
    }
    CHECK(kv.advanceSeqLen(seq, ctx).isOk());
    // one decode step over both layers
    for (int l = 0; l < mc.num_layers; ++l) {
        DecodeLayer layer{l, mc};
        const auto  q = normal_f16(300 + l, row), nk = normal_f16(400 + l, row),
                   nv = normal_f16(500 + l, row);
        half *dq = to_device(q), *dk = to_device(nk), *dv = to_device(nv), *dout = nullptr;
        HIP_OK(hipMalloc(reinterpret_cast<void **>(&dout), row * 2));
        layer.forward_attention(dq, dk, dv, dout, kv, seq, kv.getSeqLen(seq), nullptr);
        HIP_OK(hipDeviceSynchronize());
        auto cache = kv.getCacheChecked(seq, l);
        CHECK(cache.isOk());
        const auto kh = to_host(cache.value().first, (size_t)M * row);
        const auto vh = to_host(cache.value().second, (size_t)M * row);
        CHECK(std::equal(nk.begin(), nk.end(), kh.begin() + (size_t)ctx * row));
        CHECK(std::equal(nv.begin(), nv.end(), vh.begin() + (size_t)ctx * row));
        std::vector<float>    ref(row);
        std::vector<uint16_t> ref16(row);
        orc_attention_decode(q.data(), kh.data(), vh.data(), ref.data(), ref16.data(),
                             1.0f / std::sqrt((float)D), 1, H, ctx + 1, D);
        const double e = rel_err(to_host(dout, row), ref);
        std::printf("reference_decode_branch layer %d rel_err %.3e\n", l, e);
        CHECK(e <= 1e-3);
        for (half *p : {dq, dk, dv, dout}) HIP_OK(hipFree(p));
    }
    CHECK(kv.advanceSeqLen(seq, 1).isOk()); // InferenceEngine::decodeStep's commit
    CHECK(kv.getSeqLen(seq) == ctx + 1);
    for (half *p : keep) HIP_OK(hipFree(p));
    std::printf("ok reference_decode_branch\n");

    // error paths through the caller's fmt-style logger
    const int before = test_log::error_count();
    DecodeLayer layer{0, mc};
    layer.forward_attention(nullptr, nullptr, nullptr, nullptr, kv, 999, 0, nullptr);
    layer.forward_attention(nullptr, nullptr, nullptr, nullptr, kv, seq, M + 5, nullptr);
    auto bad = kv.appendKV(999, 0, nullptr, nullptr, 1, nullptr);
    CHECK(bad.isErr());
    TLLM_ERROR("appendKV: {}", bad.error());
    CHECK(bad.error().find("null") != std::string::npos || bad.error().find("not found") != std::string::npos);
    CHECK(test_log::error_count() == before + 3);
    std::printf("ok caller_logger_fmt\n");
}

void batched_gqa_decode() {
    KVCacheConfig kc;
    kc.num_layers = 1;
    kc.num_heads = 2;
    kc.head_dim = 128;
    kc.max_seq_len = 1200;
    kc.max_batch_size = 3;
    const int Hkv = kc.num_heads, D = kc.head_dim, M = kc.max_seq_len, Hq = 8, row = Hkv * D;
    auto      created = KVCacheManager::create(kc);
    CHECK(created.isOk());
    auto                &kv = *created.value();
    const int            ctx[3] = {1000, 5, 513};
    std::vector<int>     ids;
    std::vector<half *>  keep;
    for (int b = 0; b < 3; ++b) {
        auto sid = kv.allocateSequence(M);
        CHECK(sid.isOk());
        auto k = to_device(normal_f16(600 + b, (size_t)ctx[b] * row));
        auto v = to_device(normal_f16(700 + b, (size_t)ctx[b] * row));
        keep.push_back(k);
        keep.push_back(v);
        CHECK(kv.appendKV(sid.value(), 0, k, v, ctx[b], nullptr).isOk());
        CHECK(kv.advanceSeqLen(sid.value(), ctx[b]).isOk());
        ids.push_back(sid.value());
    }
    auto batch = DecodeBatch::create(kv, 3, Hq);
    CHECK(batch.isOk());
    const auto q = normal_f16(800, (size_t)3 * Hq * D), nk = normal_f16(801, (size_t)3 * row),
               nv = normal_f16(802, (size_t)3 * row);
    half *dq = to_device(q), *dk = to_device(nk), *dv = to_device(nv), *dout = nullptr;
    HIP_OK(hipMalloc(reinterpret_cast<void **>(&dout), (size_t)3 * Hq * D * 2));
    CHECK(batch.value()->prepare(ids.data(), 3, nullptr).isOk());
    CHECK(batch.value()->decode(0, dq, dk, dv, dout, 1.0f / std::sqrt((float)D), nullptr).isOk());
    CHECK(batch.value()->commit(1).isOk());
    HIP_OK(hipDeviceSynchronize());
    const auto out = to_host(dout, (size_t)3 * Hq * D);
    for (int b = 0; b < 3; ++b) {
        auto cache = kv.getCacheChecked(ids[b], 0);
        CHECK(cache.isOk());
        const auto    kh = to_host(cache.value().first, (size_t)M * row);
        const auto    vh = to_host(cache.value().second, (size_t)M * row);
        const int32_t bt = 0, len = ctx[b] + 1;
        orc_kv_view   view = {kh.data(), vh.data(), &bt, 1, 30, (int64_t)M * row, row, D};
        std::vector<float>    ref((size_t)Hq * D);
        std::vector<uint16_t> ref16(ref.size());
        orc_attn_decode_gqa(q.data() + (size_t)b * Hq * D, &view, &len, 1, Hq, Hkv, D,
                            1.0f / std::sqrt((float)D), ref.data(), ref16.data(), 1);
        std::vector<uint16_t> got(out.begin() + (size_t)b * Hq * D, out.begin() + (size_t)(b + 1) * Hq * D);
        const double e = rel_err(got, ref);
        std::printf("batched_gqa_decode entry %d rel_err %.3e\n", b, e);
        CHECK(e <= 1e-3);
        CHECK(kv.getSeqLen(ids[b]) == ctx[b] + 1);
    }
    for (half *p : {dq, dk, dv, dout}) HIP_OK(hipFree(p));
    for (half *p : keep) HIP_OK(hipFree(p));
    std::printf("ok batched_gqa_decode\n");
}

} // namespace

int main() {
    Dl_info info;
    // tl_version() returns a string in the library's own read-only data
    // (a function's address could resolve to this executable's PLT stub)
    CHECK(dladdr(tl_version(), &info) != 0 && info.dli_fname);
    std::printf("library %s\n", info.dli_fname);
    reference_decode_branch();
    batched_gqa_decode();
    return 0;
}
