// Byte-moving kernels of the KV path: fused batched append and gather.
// Both are HBM-bound integer work; each lane moves one 16-byte piece with a
// vector load and a vector store, consecutive lanes on consecutive pieces.
#include "kv_kernels.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace tiny_llm {
namespace detail {

namespace {

constexpr int kCopyThreads = 256;

__device__ __forceinline__ int64_t row_offset(const KvView &v, int b, int t) {
    const int     row = v.seq_row ? v.seq_row[b] : b;
    const int64_t blk =
        v.block_table ? (int64_t)v.block_table[(int64_t)row * v.bt_stride + (t >> v.log2_blk)] : row;
    return blk * v.blk_stride + (int64_t)(t & ((1 << v.log2_blk) - 1)) * v.tok_stride;
}

struct AppendArgs {
    KvView         view;
    int64_t        layer_stride;
    const int32_t *wpos;
    int            first_pos;
    int            n;
    int            row_pieces; // 16-byte pieces per token row (Hkv*D/8)
    const __half  *new_k;
    const __half  *new_v;
};

// grid (ceil(row_pieces/256), n entries, num_layers): the same bytes as the
// two cudaMemcpyAsync of appendKV (kv_cache.cpp:230-233) for each entry and
// layer, written as one coalesced launch.
__global__ __launch_bounds__(kCopyThreads) void kv_append_kernel(AppendArgs a) {
    const int piece = blockIdx.x * kCopyThreads + threadIdx.x;
    if (piece >= a.row_pieces) return;
    const int     i = blockIdx.y;
    const int     l = blockIdx.z;
    const int     t = a.wpos ? a.wpos[i] : a.first_pos + i;
    const int64_t dst = row_offset(a.view, i, t) + (int64_t)l * a.layer_stride + (int64_t)piece * 8;
    const int64_t src = ((int64_t)l * a.n + i) * (int64_t)a.row_pieces * 8 + (int64_t)piece * 8;
    const uint4   k = *reinterpret_cast<const uint4 *>(a.new_k + src);
    const uint4   v = *reinterpret_cast<const uint4 *>(a.new_v + src);
    *reinterpret_cast<uint4 *>(const_cast<__half *>(a.view.k_base) + dst) = k;
    *reinterpret_cast<uint4 *>(const_cast<__half *>(a.view.v_base) + dst) = v;
}

// Token ranges of one append launch: range r writes rows tok0[r] ..
// tok0[r+1]-1 of new_k/new_v (counted from src_tok) to cache row row[r] at
// positions pos0[r], pos0[r]+1, ...  The table travels in the kernel
// arguments, so the launch needs no metadata copy.
constexpr int kAppendRanges = 64;
constexpr int kAppendTokens = 32768; // tokens per launch (grid y)
struct RangeArgs {
    KvView        view;
    int           n;
    int           row_pieces;
    int64_t       src_tok;
    const __half *new_k;
    const __half *new_v;
    int32_t       row[kAppendRanges];
    int32_t       pos0[kAppendRanges];
    int32_t       tok0[kAppendRanges + 1];
};

// grid (ceil(row_pieces/256), tokens of the launch): one token row per block
// row, the bytes of appendKV (kv_cache.cpp:226-233) for every range.
__global__ __launch_bounds__(kCopyThreads) void kv_append_ranges_kernel(RangeArgs a) {
    const int piece = blockIdx.x * kCopyThreads + threadIdx.x;
    if (piece >= a.row_pieces) return;
    const int t = blockIdx.y;
    int       r = 0; // the range holding token t (uniform over the block)
    while (r + 1 < a.n && a.tok0[r + 1] <= t) ++r;
    const int     pos = a.pos0[r] + (t - a.tok0[r]);
    const int64_t blk =
        a.view.block_table
            ? (int64_t)a.view.block_table[(int64_t)a.row[r] * a.view.bt_stride + (pos >> a.view.log2_blk)]
            : (int64_t)a.row[r];
    const int64_t dst = blk * a.view.blk_stride +
                        (int64_t)(pos & ((1 << a.view.log2_blk) - 1)) * a.view.tok_stride + (int64_t)piece * 8;
    const int64_t src = (a.src_tok + t) * (int64_t)a.row_pieces * 8 + (int64_t)piece * 8;
    const uint4   k = *reinterpret_cast<const uint4 *>(a.new_k + src);
    const uint4   v = *reinterpret_cast<const uint4 *>(a.new_v + src);
    *reinterpret_cast<uint4 *>(const_cast<__half *>(a.view.k_base) + dst) = k;
    *reinterpret_cast<uint4 *>(const_cast<__half *>(a.view.v_base) + dst) = v;
}

struct GatherArgs {
    KvView         view;
    const int32_t *lens;
    int            uniform_len;
    int            Hkv;
    int            D;
    int            s_max;
    const __half  *src;
    __half        *out;
};

// grid (ceil(s_max*D/8 / 256), Hkv, n): out[b][g][t][:] from the cache.
__global__ __launch_bounds__(kCopyThreads) void kv_gather_kernel(GatherArgs a) {
    const int pieces_per_tok = a.D >> 3;
    const int piece = blockIdx.x * kCopyThreads + threadIdx.x;
    const int t = piece / pieces_per_tok;
    if (t >= a.s_max) return;
    const int e = piece - t * pieces_per_tok;
    const int g = blockIdx.y;
    const int b = blockIdx.z;
    const int len = a.lens ? a.lens[b] : a.uniform_len;
    uint4     val = make_uint4(0u, 0u, 0u, 0u);
    if (t < len) {
        const int64_t off = row_offset(a.view, b, t) + (int64_t)g * a.view.head_stride + e * 8;
        val = *reinterpret_cast<const uint4 *>(a.src + off);
    }
    const int64_t dst = (((int64_t)b * a.Hkv + g) * a.s_max + t) * a.D + e * 8;
    *reinterpret_cast<uint4 *>(a.out + dst) = val;
}

struct TableArgs {
    int32_t *table;
    int32_t  n;
    int32_t  idx[kTableBatch];
    int32_t  val[kTableBatch];
};

__global__ __launch_bounds__(256) void table_update_kernel(TableArgs a) {
    const int i = (int)threadIdx.x;
    if (i < a.n) a.table[a.idx[i]] = a.val[i];
}

} // namespace

void launch_table_update(int32_t *table, const std::pair<int32_t, int32_t> *upd, size_t n,
                         hipStream_t stream) {
    static_assert(kTableBatch <= 256, "one thread per pair");
    for (size_t first = 0; first < n; first += kTableBatch) {
        TableArgs a;
        a.table = table;
        a.n = (int32_t)std::min<size_t>(kTableBatch, n - first);
        for (int i = 0; i < a.n; ++i) {
            a.idx[i] = upd[first + (size_t)i].first;
            a.val[i] = upd[first + (size_t)i].second;
        }
        hipLaunchKernelGGL(table_update_kernel, dim3(1), dim3(256), 0, stream, a);
        HIP_CHECK(hipGetLastError());
    }
}

void launch_kv_append(const KvView &view, int64_t layer_stride, const int32_t *wpos, int first_pos,
                      int n, int num_layers, int row_elems, const __half *new_k,
                      const __half *new_v, hipStream_t stream) {
    if (n <= 0 || num_layers <= 0) return;
    AppendArgs a;
    a.view = view;
    a.layer_stride = layer_stride;
    a.wpos = wpos;
    a.first_pos = first_pos;
    a.n = n;
    a.row_pieces = row_elems / 8;
    a.new_k = new_k;
    a.new_v = new_v;
    dim3 grid((unsigned)((a.row_pieces + kCopyThreads - 1) / kCopyThreads), (unsigned)n,
              (unsigned)num_layers);
    profile_begin(KernelId::KvAppend, stream);
    hipLaunchKernelGGL(kv_append_kernel, grid, dim3(kCopyThreads), 0, stream, a);
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::KvAppend, stream);
}

void launch_kv_append_ranges(const KvView &view, const int32_t *rows, const int32_t *pos0,
                             const int32_t *counts, int n, int row_elems, const __half *new_k,
                             const __half *new_v, hipStream_t stream) {
    RangeArgs a;
    a.view = view;
    a.row_pieces = row_elems / 8;
    a.new_k = new_k;
    a.new_v = new_v;
    a.n = 0;
    a.tok0[0] = 0;
    int64_t done = 0; // tokens of earlier launches
    auto flush = [&]() {
        if (a.n == 0) return;
        dim3 grid((unsigned)((a.row_pieces + kCopyThreads - 1) / kCopyThreads), (unsigned)a.tok0[a.n]);
        a.src_tok = done;
        profile_begin(KernelId::KvAppend, stream);
        hipLaunchKernelGGL(kv_append_ranges_kernel, grid, dim3(kCopyThreads), 0, stream, a);
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::KvAppend, stream);
        done += a.tok0[a.n];
        a.n = 0;
        a.tok0[0] = 0;
    };
    for (int i = 0; i < n; ++i) {
        int off = 0; // a range longer than a launch holds continues in the next
        while (off < counts[i]) {
            if (a.n == kAppendRanges || a.tok0[a.n] == kAppendTokens) flush();
            const int take = std::min(counts[i] - off, kAppendTokens - a.tok0[a.n]);
            a.row[a.n] = rows[i];
            a.pos0[a.n] = pos0[i] + off;
            a.tok0[a.n + 1] = a.tok0[a.n] + take;
            ++a.n;
            off += take;
        }
    }
    flush();
}

void launch_kv_gather(const KvView &view, int which, const int32_t *lens, int uniform_len, int n,
                      int Hkv, int D, int s_max, __half *out, hipStream_t stream) {
    if (n <= 0 || s_max <= 0 || !out) return;
    GatherArgs a;
    a.view = view;
    a.lens = lens;
    a.uniform_len = uniform_len;
    a.Hkv = Hkv;
    a.D = D;
    a.s_max = s_max;
    a.src = which ? view.v_base : view.k_base;
    a.out = out;
    const long pieces = (long)s_max * (D / 8);
    dim3       grid((unsigned)((pieces + kCopyThreads - 1) / kCopyThreads), (unsigned)Hkv, (unsigned)n);
    profile_begin(KernelId::KvGather, stream);
    hipLaunchKernelGGL(kv_gather_kernel, grid, dim3(kCopyThreads), 0, stream, a);
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::KvGather, stream);
}

} // namespace detail
} // namespace tiny_llm
