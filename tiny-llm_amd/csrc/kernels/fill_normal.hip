// Seeded normal fp16 generator for the synthetic inputs of the benchmarks and
// tests: splitmix64 -> Box-Muller -> fp32 -> fp16 (round to nearest even),
// element for element the generator the oracle defines (orc_fill_normal_f16).
// splitmix64 advances its state by a constant, so call k (1-based) of a stream
// seeded with `seed` mixes seed + k * gamma: element pair P (elements 2P and
// 2P + 1) takes calls 2P + 1 and 2P + 2, and any range of a stream can be
// drawn on its own.  One lane per pair; the Box-Muller transform runs in
// double precision like the host generator.
#include "kv_kernels.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <stdexcept>

namespace tiny_llm {
namespace detail {

namespace {

constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;

__device__ __forceinline__ uint64_t splitmix_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct FillArgs {
    uint64_t seed;
    uint64_t first;   // first element of the stream written to out[0]
    uint64_t n;       // elements written
    uint64_t pair0;   // first / 2
    uint64_t npairs;  // pairs touching [first, first + n)
    double   stddev;
    __half  *out;
};

// fp32 rounding, then fp16 rounding, as two steps: the fp32 value is pinned
// in a register, so the compiler cannot fold the two conversions into one
// double -> fp16 rounding, which differs from the two-step result whenever the
// fp32 value lands exactly on an fp16 midpoint.
__device__ __forceinline__ __half to_half_via_float(double x) {
    float f = (float)x;
    asm volatile("" : "+v"(f));
    return __float2half_rn(f);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(FillArgs a) {
    const uint64_t j = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (j >= a.npairs) return;
    const uint64_t P = a.pair0 + j;
    const uint64_t z1 = splitmix_mix(a.seed + (2u * P + 1u) * kGamma);
    const uint64_t z2 = splitmix_mix(a.seed + (2u * P + 2u) * kGamma);
    const double   u1 = 1.0 - (double)(z1 >> 11) * (1.0 / 9007199254740992.0);
    const double   u2 = (double)(z2 >> 11) * (1.0 / 9007199254740992.0);
    const double   two_pi = 6.283185307179586476925286766559;
    const double   r = sqrt(-2.0 * log(u1));
    const uint64_t e0 = 2u * P; // stream index of the cosine element
    if (e0 >= a.first && e0 < a.first + a.n)
        a.out[e0 - a.first] = to_half_via_float(r * cos(two_pi * u2) * a.stddev);
    if (e0 + 1u >= a.first && e0 + 1u < a.first + a.n)
        a.out[e0 + 1u - a.first] = to_half_via_float(r * sin(two_pi * u2) * a.stddev);
}

} // namespace

void launch_fill_normal(uint64_t seed, uint64_t first, float stddev, __half *out, uint64_t n,
                        hipStream_t stream) {
    if (n == 0) return;
    FillArgs a;
    a.seed = seed;
    a.first = first;
    a.n = n;
    a.pair0 = first / 2;
    a.npairs = (first + n + 1) / 2 - a.pair0;
    a.stddev = stddev;
    a.out = out;
    const uint64_t blocks = (a.npairs + 255) / 256;
    if (blocks > 0x7fffffffull) throw std::invalid_argument("fill_normal: too many elements");
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    HIP_CHECK(hipGetLastError());
}

} // namespace detail
} // namespace tiny_llm
