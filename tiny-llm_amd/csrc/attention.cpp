// Stateless decode-attention entry points: the reference's
// tiny_llm::kernels::attention_decode (kernels/attention.cu:114-128) and the
// view-based GQA call.  Both run the split-K kernels of
// kernels/attention_decode.hip with the per-device workspace.
#include "tiny_llm/kernels/attention.h"

#include "kernels/kv_kernels.h"
#include "kernels/prefill.h"
#include "runtime.h"
#include "tiny_llm/hip_utils.h"
#include "tl_log.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace tiny_llm {
namespace detail {

namespace {
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
} // namespace

std::string check_decode_view_args(const char *who, const __half *q, const KvView &kv,
                                   const int32_t *seq_lens_host, int B, int Hq, int Hkv, int D,
                                   const __half *out) {
    const std::string w(who);
    if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return w + ": invalid dimensions";
    if (B == 0) return "";
    if (Hq % Hkv != 0) return w + ": Hq must be a multiple of Hkv";
    if (!attn_shape_supported(D, Hq / Hkv))
        return w + ": unsupported head_dim/group (head_dim in {32,64,128,256}, Hq/Hkv in {1,2,4,8})";
    if (!q || !out || !kv.k_base || !kv.v_base || !seq_lens_host) return w + ": null pointer argument";
    if (!aligned16(q) || !aligned16(kv.k_base) || !aligned16(kv.v_base))
        return w + ": q, k_base and v_base must be 16-byte aligned";
    if (kv.tok_stride % 8 != 0 || kv.head_stride % 8 != 0 || kv.blk_stride % 8 != 0)
        return w + ": strides must be multiples of 8 elements";
    if (kv.log2_blk < 4 || kv.log2_blk > 30) return w + ": log2_blk must be in [4, 30]";
    for (int b = 0; b < B; ++b)
        if (seq_lens_host[b] < 0) return w + ": negative sequence length";
    return "";
}

// Returns "" on success, else the reason the call was rejected.
std::string attn_decode_view(const __half *q, const KvView &kv, const int32_t *seq_lens_host, int B,
                             int Hq, int Hkv, int D, float scale, __half *out, hipStream_t stream) {
    const std::string bad =
        check_decode_view_args("tl_attn_decode_gqa", q, kv, seq_lens_host, B, Hq, Hkv, D, out);
    if (!bad.empty() || B == 0) return bad;

    WorkList wl;
    plan_work(seq_lens_host, B, Hkv, D, wl);
    const int      n_work = wl.n_work;
    if (kv.seq_row == nullptr) { // small plans travel in the kernel arguments
        InlineMeta inl;
        if (pack_inline(seq_lens_host, wl, nullptr, B, inl)) {
            DeviceContext &ctx = DeviceContext::get(current_device());
            std::lock_guard<std::mutex> lk(ctx.mu);
            ctx.claim(stream);
            AttnPlan plan;
            plan.n_work = n_work;
            plan.chunk = wl.chunk;
            plan.any_multi = wl.any_multi;
            plan.any_empty = wl.any_empty;
            plan.max_len = wl.max_len;
            plan.fused_heads = wl.fused_heads;
            plan.fused_chunked = wl.fused_chunked;
            float *part = wl.any_multi ? ctx.ws.get(attn_workspace_floats(n_work, Hq, D)) : nullptr;
            int   *cnt = wl.any_multi && fused_merge_enabled()
                                 ? ctx.ws.counters(attn_counters_ints(B, Hkv), stream)
                                 : nullptr;
            launch_attn_decode(q, kv, plan, B, Hq, Hkv, D, scale, out, part, nullptr, nullptr, stream,
                               &inl, true, cnt);
            return "";
        }
    }
    const size_t   nb = static_cast<size_t>(B);
    DeviceContext &ctx = DeviceContext::get(current_device());
    std::lock_guard<std::mutex> lk(ctx.mu);
    ctx.claim(stream);
    const size_t words = nb + (nb + 1) + 2 * static_cast<size_t>(n_work);
    int32_t     *h = static_cast<int32_t *>(ctx.ring.begin(words * 4));
    std::memcpy(h, seq_lens_host, nb * 4);
    std::memcpy(h + nb, wl.part_base.data(), (nb + 1) * 4);
    if (n_work > 0) std::memcpy(h + 2 * nb + 1, wl.work.data(), 2 * static_cast<size_t>(n_work) * 4);
    const int32_t *d = static_cast<const int32_t *>(ctx.ring.commit(stream));
    AttnPlan       plan;
    plan.seq_lens = d;
    plan.part_base = d + nb;
    plan.work = d + 2 * nb + 1;
    plan.n_work = n_work;
    plan.chunk = wl.chunk;
    plan.any_multi = wl.any_multi;
    plan.any_empty = wl.any_empty;
    plan.max_len = wl.max_len;
    plan.fused_heads = wl.fused_heads;
    plan.fused_chunked = wl.fused_chunked;
    float *part = wl.any_multi ? ctx.ws.get(attn_workspace_floats(n_work, Hq, D)) : nullptr;
    int   *cnt = wl.any_multi && fused_merge_enabled()
                         ? ctx.ws.counters(attn_counters_ints(B, Hkv), stream)
                         : nullptr;
    launch_attn_decode(q, kv, plan, B, Hq, Hkv, D, scale, out, part, nullptr, nullptr, stream, nullptr,
                       true, cnt);
    return "";
}

std::string attn_decode_compact(const __half *q, const __half *k, const __half *v, __half *out,
                                float scale, int B, int H, int S, int D, hipStream_t stream) {
    if (!attn_shape_supported(D, 1))
        return "attention_decode: unsupported head_dim " + std::to_string(D) +
               " (supported: 32, 64, 128, 256)";
    if (!q || !k || !v || !out) return "attention_decode: null pointer argument";
    if (!aligned16(q) || !aligned16(k) || !aligned16(v))
        return "attention_decode: query, k_cache and v_cache must be 16-byte aligned";
    KvView kv;
    kv.k_base = k;
    kv.v_base = v;
    kv.log2_blk = 30;
    kv.blk_stride = static_cast<int64_t>(H) * S * D;
    kv.tok_stride = D;
    kv.head_stride = static_cast<int64_t>(S) * D;
    AttnPlan plan;
    plan.uniform_len = S;
    plan.chunk = choose_chunk(nullptr, B, H, S, D);
    plan.nchunk = (S + plan.chunk - 1) / plan.chunk;
    plan.n_work = B * plan.nchunk;
    plan.any_multi = plan.nchunk > 1;
    plan.max_len = S;
    DeviceContext &ctx = DeviceContext::get(current_device());
    std::lock_guard<std::mutex> lk(ctx.mu);
    ctx.claim(stream);
    float *part = plan.any_multi ? ctx.ws.get(attn_workspace_floats(plan.n_work, H, D)) : nullptr;
    int   *cnt = plan.any_multi && fused_merge_enabled() ? ctx.ws.counters(attn_counters_ints(B, H), stream)
                                                        : nullptr;
    launch_attn_decode(q, kv, plan, B, H, H, D, scale, out, part, nullptr, nullptr, stream, nullptr, true,
                       cnt);
    return "";
}

std::string attn_prefill_compact(const __half *q, const __half *k, const __half *v, __half *out,
                                float scale, int B, int H, int S, int D, hipStream_t stream) {
    if (!prefill_shape_supported(D, 1))
        return "attention_prefill: unsupported head_dim " + std::to_string(D) +
               " (supported: 32, 64, 128, 256)";
    if (!q || !k || !v || !out) return "attention_prefill: null pointer argument";
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return "attention_prefill: query, key, value and output must be 16-byte aligned";
    KvView kv;
    kv.k_base = k;
    kv.v_base = v;
    kv.log2_blk = 30;
    kv.blk_stride = static_cast<int64_t>(H) * S * D;
    kv.tok_stride = D;
    kv.head_stride = static_cast<int64_t>(S) * D;
    PrefillLaunch p;
    p.q = q;
    p.out = out;
    p.q_tok_stride = D;
    p.q_head_stride = static_cast<int64_t>(S) * D;
    p.q_entry_stride = static_cast<int64_t>(H) * S * D;
    p.uniform_b = B;
    p.uniform_n = S;
    p.max_keys = S;
    launch_attn_prefill(p, kv, H, H, D, scale, stream);
    return "";
}

} // namespace detail

namespace kernels {

void attention_prefill(const half *query, const half *key, const half *value, half *output,
                       float scale, int batch_size, int num_heads, int seq_len, int head_dim,
                       hipStream_t stream) {
    if (batch_size <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return;
    std::string err;
    try {
        err = detail::attn_prefill_compact(query, key, value, output, scale, batch_size, num_heads,
                                           seq_len, head_dim, stream);
    } catch (const std::exception &e) {
        err = e.what();
    }
    if (!err.empty()) TL_LOG_ERROR("%s", err.c_str());
}

void softmax(const half *input, half *output, int batch_size, int seq_len, hipStream_t stream) {
    if (batch_size <= 0 || seq_len <= 0) return;
    try {
        detail::launch_softmax(input, output, batch_size, seq_len, stream);
    } catch (const std::exception &e) {
        TL_LOG_ERROR("softmax: %s", e.what());
    }
}

void get_attention_weights(const half *query, const half *key, half *weights, float scale,
                           int batch_size, int num_heads, int query_len, int key_len, int head_dim,
                           bool apply_causal_mask, hipStream_t stream) {
    if (batch_size <= 0 || num_heads <= 0 || query_len <= 0 || key_len <= 0 || head_dim <= 0) return;
    try {
        detail::launch_attention_weights(query, key, weights, scale, batch_size, num_heads,
                                         query_len, key_len, head_dim, apply_causal_mask, stream);
    } catch (const std::exception &e) {
        TL_LOG_ERROR("get_attention_weights: %s", e.what());
    }
}

void attention_decode(const half *query, const half *k_cache, const half *v_cache, half *output,
                      float scale, int batch_size, int num_heads, int seq_len, int head_dim,
                      hipStream_t stream) {
    if (batch_size <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return;
    std::string err;
    try {
        err = detail::attn_decode_compact(query, k_cache, v_cache, output, scale, batch_size,
                                          num_heads, seq_len, head_dim, stream);
    } catch (const std::exception &e) {
        err = e.what();
    }
    if (!err.empty()) TL_LOG_ERROR("%s", err.c_str());
}

} // namespace kernels
} // namespace tiny_llm
