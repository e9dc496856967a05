// Host entry points of the W8A16 GEMM: the reference's
// kernels::w8a16_matmul (kernels/w8a16_matmul.cu:219-236) and the fused
// o_proj + residual step.  The decode-batch projection that writes K/V rows
// straight into the cache is DecodeBatch::project (kv_cache.cpp).
#include "tiny_llm/kernels/w8a16_matmul.h"

#include "kernels/kv_kernels.h"
#include "kernels/w8a16.h"
#include "runtime.h"
#include "tiny_llm/hip_utils.h"
#include "tl_log.h"

#include <mutex>
#include <string>

namespace tiny_llm {
namespace detail {

std::string w8a16_call(const __half *x, const int8_t *w, const __half *s, __half *out, int M, int N,
                       int K, int gs, bool residual, hipStream_t stream, bool packed) {
    if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return ""; // reference: silent no-op
    if (!x || !w || !s || !out) return "w8a16_matmul: null pointer argument";
    W8A16Seg seg;
    seg.w = w;
    seg.s = s;
    seg.n = N;
    seg.kind = residual ? kEpiResidual : kEpiDense;
    seg.out = out;
    seg.ld = N;
    seg.res = residual ? out : nullptr;
    DeviceContext              &ctx = DeviceContext::get(current_device());
    std::lock_guard<std::mutex> lk(ctx.mu);
    ctx.claim(stream);
    float *ws = nullptr;
    if (const size_t f = w8a16_workspace_floats(M, K, gs, &seg, 1)) ws = ctx.ws.get(f);
    if (packed && !w8a16_mfma_ok(K, gs, &seg, 1))
        return "w8a16_matmul: packed weights need K % 32 == 0, N % 16 == 0 and group_size in "
               "{32, 64, 128, 256, 512}";
    launch_w8a16(x, K, M, K, gs, &seg, 1, nullptr, ws, stream, packed);
    return "";
}

std::string w8a16_pack_call(const int8_t *w, int K, int N, int8_t *out, hipStream_t stream) {
    if (!w || !out) return "w8a16_pack: null pointer argument";
    if (K <= 0 || N <= 0 || K % 32 != 0 || N % 16 != 0)
        return "w8a16_pack: K must be a positive multiple of 32 and N of 16";
    launch_w8a16_pack(w, K, N, out, stream);
    return "";
}

} // namespace detail

namespace kernels {

void w8a16_matmul(const half *input, const int8_t *weight, const half *scales, half *output, int M,
                  int N, int K, int group_size, hipStream_t stream) {
    std::string err;
    try {
        err = detail::w8a16_call(input, weight, scales, output, M, N, K, group_size, false, stream,
                                 false);
    } catch (const std::exception &e) {
        err = e.what();
    }
    if (!err.empty()) TL_LOG_ERROR("%s", err.c_str());
}

void w8a16_matmul_residual(const half *input, const int8_t *weight, const half *scales, half *hidden,
                           int M, int N, int K, int group_size, hipStream_t stream, bool packed) {
    std::string err;
    try {
        err = detail::w8a16_call(input, weight, scales, hidden, M, N, K, group_size, true, stream,
                                 packed);
    } catch (const std::exception &e) {
        err = e.what();
    }
    if (!err.empty()) TL_LOG_ERROR("%s", err.c_str());
}

void w8a16_pack(const int8_t *weight, int K, int N, int8_t *packed, hipStream_t stream) {
    std::string err;
    try {
        err = detail::w8a16_pack_call(weight, K, N, packed, stream);
    } catch (const std::exception &e) {
        err = e.what();
    }
    if (!err.empty()) TL_LOG_ERROR("%s", err.c_str());
}

} // namespace kernels
} // namespace tiny_llm
