// No-allocation variant of the view-based GQA decode attention
// (tl_attn_decode_gqa_noalloc), for callers that cannot allocate device
// memory: code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc.
//
// It runs the same launches as tl_attn_decode_gqa (attn_decode_kernel and,
// for split sequences, attn_merge_kernel, with the same plan), but the
// device memory beyond the caller's inputs and outputs lives in `scratch`, a
// file-scope device array of kScratchBytes that every GPU holds from the
// moment the library's code object is loaded on it until the process ends:
//   [plan metadata, when it does not fit in the kernel arguments | 256-byte
//    aligned split-K partials o[items][Hq][D], (m, l)[items][Hq] fp32]
// The metadata reaches the scratch through meta_fill_kernel, whose words
// travel in its kernel arguments (no host-to-device copy, no pinned memory).
// Nothing in the scratch needs to start at zero: every partial row the merge
// reads is written by the same call, and entries with no tokens take the
// merge's zero-row path without reading partials.
//
// Every call on one GPU uses that GPU's single scratch array, which keeps the
// last call's contents: calls that overlap on one GPU (two host threads, or
// two streams without ordering between them) race.
#include "kv_kernels.h"

#include "runtime.h"
#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace tiny_llm {
namespace detail {

namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr int    kMaxDevices = 64;

// Host code must not take this name as a device address (in host code it is
// a stand-in symbol): kernels receive the per-device address that
// hipGetSymbolAddress returns, kept in g_scratch_addr.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void      *g_scratch_addr[kMaxDevices] = {};

// Device address of the current device's scratch array, looked up once per
// device on that device's first call.
unsigned char *scratch_on_current_device() {
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices)
        throw std::runtime_error("tl_attn_decode_gqa_noalloc: device index " + std::to_string(dev) +
                                 " beyond " + std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void *p = nullptr;
        HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) throw std::runtime_error("tl_attn_decode_gqa_noalloc: scratch address is null");
        g_scratch_addr[dev] = p;
    }
    return static_cast<unsigned char *>(g_scratch_addr[dev]);
}

struct MetaWords {
    int32_t n;
    int32_t w[kInlineWords];
};

// dst[i] = m.w[i] for i < m.n: plan metadata written from kernel arguments.
__global__ __launch_bounds__(256) void meta_fill_kernel(int32_t *dst, MetaWords m) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < m.n) dst[i] = m.w[i];
}

} // namespace

size_t attn_noalloc_scratch_bytes() { return kScratchBytes; }

std::string attn_decode_view_noalloc(const __half *q, const KvView &kv,
                                     const int32_t *seq_lens_host, int B, int Hq, int Hkv, int D,
                                     float scale, __half *out, hipStream_t stream) {
    static const char *who = "tl_attn_decode_gqa_noalloc";
    const std::string  bad = check_decode_view_args(who, q, kv, seq_lens_host, B, Hq, Hkv, D, out);
    if (!bad.empty() || B == 0) return bad;
    if (kv.seq_row != nullptr) return std::string(who) + ": per-entry row table is not supported";

    // Host planning state is reused across calls on this thread (its buffers
    // grow on the first calls only).
    thread_local WorkList             wl;
    thread_local InlineMeta           inl;
    thread_local std::vector<int32_t> words;
    plan_work(seq_lens_host, B, Hkv, D, wl);
    const bool   in_args = pack_inline(seq_lens_host, wl, nullptr, B, inl);
    const size_t nb = static_cast<size_t>(B);
    const size_t meta_words = in_args ? 0 : nb + (nb + 1) + 2 * static_cast<size_t>(wl.n_work);
    const size_t meta_bytes = (meta_words * 4 + 255) / 256 * 256;
    const size_t part_bytes = wl.any_multi ? attn_workspace_floats(wl.n_work, Hq, D) * 4 : 0;
    if (meta_bytes + part_bytes > kScratchBytes)
        return std::string(who) + ": the call needs " + std::to_string(meta_bytes + part_bytes) +
               " bytes of scratch (plan metadata " + std::to_string(meta_bytes) +
               ", split-K partials " + std::to_string(part_bytes) + "); the maximum is " +
               std::to_string(kScratchBytes);

    unsigned char *base = scratch_on_current_device();
    AttnPlan       plan;
    plan.n_work = wl.n_work;
    plan.chunk = wl.chunk;
    plan.any_multi = wl.any_multi;
    plan.any_empty = wl.any_empty;
    plan.max_len = wl.max_len;
    plan.fused_heads = wl.fused_heads;
    plan.fused_chunked = wl.fused_chunked;
    if (!in_args) {
        words.resize(meta_words);
        std::memcpy(words.data(), seq_lens_host, nb * 4);
        std::memcpy(words.data() + nb, wl.part_base.data(), (nb + 1) * 4);
        if (wl.n_work) std::memcpy(words.data() + 2 * nb + 1, wl.work.data(), wl.work.size() * 4);
        int32_t *dst = reinterpret_cast<int32_t *>(base);
        for (size_t off = 0; off < meta_words; off += kInlineWords) {
            MetaWords m;
            m.n = static_cast<int32_t>(std::min<size_t>(kInlineWords, meta_words - off));
            std::memcpy(m.w, words.data() + off, static_cast<size_t>(m.n) * 4);
            hipLaunchKernelGGL(meta_fill_kernel, dim3((m.n + 255) / 256), dim3(256), 0, stream,
                               dst + off, m);
            HIP_CHECK(hipGetLastError());
        }
        plan.seq_lens = dst;
        plan.part_base = dst + nb;
        plan.work = dst + 2 * nb + 1;
    }
    float *part = wl.any_multi ? reinterpret_cast<float *>(base + meta_bytes) : nullptr;
    launch_attn_decode(q, kv, plan, B, Hq, Hkv, D, scale, out, part, nullptr, nullptr, stream,
                       in_args ? &inl : nullptr, /*hooks=*/false);
    return "";
}

} // namespace detail
} // namespace tiny_llm
