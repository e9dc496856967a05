// Launch interface of the HIP kernels of the KV decode path (gfx950).
// Host code (kv_cache.cpp, capi.cpp) calls only these launchers.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include "attn_plan.h"

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace tiny_llm {
namespace detail {

// Addressing of (batch entry b, kv head g, token t), in fp16 elements from
// k_base / v_base:
//   row(b)  = seq_row ? seq_row[b] : b
//   blk     = block_table ? block_table[row(b) * bt_stride + (t >> log2_blk)] : row(b)
//   offset  = blk * blk_stride + (t & (2^log2_blk - 1)) * tok_stride + g * head_stride
// The reference pool (kv_cache.cpp:69-80, 226-233) is block_table = NULL,
// seq_row = slot of each entry, blk_stride = slot size, log2_blk = 30.
struct KvView {
    const __half  *k_base = nullptr;
    const __half  *v_base = nullptr;
    const int32_t *block_table = nullptr;
    const int32_t *seq_row = nullptr;
    int            bt_stride = 0;
    int            log2_blk = 30;
    int64_t        blk_stride = 0;
    int64_t        tok_stride = 0;
    int64_t        head_stride = 0;
};

// How the split-K work of one attention call is laid out.
//  - uniform: every entry has uniform_len tokens and nchunk chunks; work item
//    w = b * nchunk + c (work, seq_lens and part_base are NULL).
//  - ragged:  seq_lens[b] tokens; work[2w], work[2w+1] = (b, c); the items of
//    entry b own partial rows part_base[b] .. part_base[b+1]-1 in chunk
//    order; the work list itself is ordered longest item first.
struct AttnPlan {
    const int32_t *seq_lens = nullptr;
    const int32_t *work = nullptr;
    const int32_t *part_base = nullptr;
    int            uniform_len = 0;
    int            nchunk = 1;
    int            n_work = 0;
    int            chunk = 256;  // tokens per work item, a positive multiple of the
                                 // kernel's quantum (waves per workgroup x 64)
    bool           any_multi = false;  // some entry spans more than one chunk
    bool           any_empty = false;  // some entry attends to zero tokens
    int            max_len = 0;        // longest attended length (offset-width check)
    // Head-fused plan (WorkList::fused_heads): 8-wave workgroups of
    // fused_heads kv heads, an entry's items interleaving its tiles; 0: per head.
    int            fused_heads = 0;
    bool           fused_chunked = false; // head-fused over chunk items (ragged plans)
};

// Chunk length for the current device (TL_ATTN_CHUNK overrides), see
// plan_chunk.
int choose_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len, int head_dim);
// The ragged plan for the current device (TL_ATTN_CHUNK overrides), see
// plan_work_list.
void plan_work(const int32_t *lens, int n, int num_kv_heads, int head_dim, WorkList &out);

// Partials workspace (floats) needed by launch_attn_decode for n_work items.
size_t attn_workspace_floats(int n_work, int Hq, int D);

// True when (D, Hq/Hkv) has a kernel instantiation.
bool attn_shape_supported(int D, int G);

// q, out: [B][Hq][D]; part: workspace of attn_workspace_floats() floats
// (needed only when plan.any_multi).
// new_k/new_v ([B][Hkv][D], or null): append that token at position
// seq_lens[b]-1 before attending (the decode branch of a transformer layer).
// Throws HipException on launch failure, std::invalid_argument when a token
// offset of a non-paged view does not fit in 32 bits.
// inl (optional): the plan's metadata in kernel arguments; when given, the
// seq_lens / work / part_base pointers of plan and kv.seq_row are not read.
// hooks = false: no tl_profile_* event hooks around the launches (the
// no-allocation entry point).
// counters (optional): attn_counters_ints() ints, zero before the call (and
// left zero by it): with fused_merge_enabled(), a multi-chunk plan without
// empty entries then merges the partials inside the attention launch instead
// of a second launch.
void launch_attn_decode(const __half *q, const KvView &kv, const AttnPlan &plan, int B, int Hq,
                        int Hkv, int D, float scale, __half *out, float *part, const __half *new_k,
                        const __half *new_v, hipStream_t stream, const InlineMeta *inl = nullptr,
                        bool hooks = true, int *counters = nullptr);

// Merge counters (ints) launch_attn_decode uses for B entries of Hkv kv heads.
inline size_t attn_counters_ints(int B, int Hkv) { return (size_t)B * (size_t)Hkv; }

// Argument checks shared by the view-based decode entry points: "" when the
// call is valid, else the reason, prefixed by `who`.
std::string check_decode_view_args(const char *who, const __half *q, const KvView &kv,
                                   const int32_t *seq_lens_host, int B, int Hq, int Hkv, int D,
                                   const __half *out);

// tl_attn_decode_gqa_noalloc: the same launches as the view-based decode,
// with the split-K partials and, when the plan does not fit in the kernel
// arguments, its metadata in the library's static device scratch array
// (no allocation).  "" on success, else the reason the call was rejected.
std::string attn_decode_view_noalloc(const __half *q, const KvView &kv,
                                     const int32_t *seq_lens_host, int B, int Hq, int Hkv, int D,
                                     float scale, __half *out, hipStream_t stream);
// Bytes of the static scratch array of attn_decode_view_noalloc.
size_t attn_noalloc_scratch_bytes();

// One token row ([Hkv][D] contiguous: tok_stride == Hkv*D, head_stride == D)
// per (entry i, layer l) for n entries and num_layers layers.
//   position  = wpos ? wpos[i] : first_pos + i
//   src_k/v   = new_k/new_v + ((l * n) + i) * Hkv*D
//   dst       = view (shifted by l * layer_stride elements) at (i, position)
void launch_kv_append(const KvView &view, int64_t layer_stride, const int32_t *wpos, int first_pos,
                      int n, int num_layers, int row_elems, const __half *new_k,
                      const __half *new_v, hipStream_t stream);

// Multi-token append of n sequences for one layer: sequence i's counts[i]
// token rows ([Hkv][D] contiguous) follow those of sequences 0..i-1 in
// new_k/new_v and go to cache row rows[i] (view.seq_row is not read) at
// positions pos0[i], pos0[i]+1, ...  rows/pos0/counts are host memory: they
// travel in kernel arguments (no metadata copy).
void launch_kv_append_ranges(const KvView &view, const int32_t *rows, const int32_t *pos0,
                             const int32_t *counts, int n, int row_elems, const __half *new_k,
                             const __half *new_v, hipStream_t stream);

// out[b][g][t][:] = cache(b, g, t) for t < lens[b] (lens NULL: uniform_len),
// +0.0 for lens[b] <= t < s_max.  which: 0 = K, 1 = V.
void launch_kv_gather(const KvView &view, int which, const int32_t *lens, int uniform_len, int n,
                      int Hkv, int D, int s_max, __half *out, hipStream_t stream);

// Writes table[idx[i]] = val[i] for the n (index, value) pairs, in stream
// order: the device copy of a block table follows its host mirror with only
// the entries that changed.  Pairs travel in kernel arguments, kTableBatch per
// launch.
constexpr int kTableBatch = 240;
void launch_table_update(int32_t *table, const std::pair<int32_t, int32_t> *upd, size_t n,
                         hipStream_t stream);

// Score path of the attention kernels: 0 = VALU dot products over the
// loaded rows, 1 = MFMA over an LDS-transposed K tile, 2 = auto (VALU for
// every supported group).
void set_score_path(int path);
int  score_path();

// Waves per attention workgroup: 0 = auto, 4 or 8.
void set_waves(int waves);
int  waves();

// Head-fused decode plans: 0 = auto, 1 = off, 2 / 4 / 8 = that many kv
// heads per workgroup where a plan with it applies.
void set_head_fuse(int mode);
int  head_fuse();
// Merge of multi-chunk plans inside the attention launch (true) or by
// attn_merge_kernel (false, the default); initial value from TL_ATTN_MERGE
// ("fused": true).
void set_fused_merge(bool on);
bool fused_merge_enabled();
// The head_fuse argument plan_work passes to plan_work_list for this
// head_dim under the current settings (head-fuse mode, waves, score path):
// 0 = per-head plans only, 1 = auto, 2 / 4 / 8 = forced heads per workgroup.
int planner_head_fuse(int head_dim);

// out[j] = element first + j of the seeded normal fp16 stream (splitmix64 ->
// Box-Muller -> fp16 RNE, times stddev before rounding), j < n.
void launch_fill_normal(uint64_t seed, uint64_t first, float stddev, __half *out, uint64_t n,
                        hipStream_t stream);

// Compute units of the current device (cached per device).
int device_cus();

// Per-kernel event timing (tl_profile_*).
enum class KernelId {
    AttnChunk = 0,
    AttnMerge = 1,
    KvAppend = 2,
    KvGather = 3,
    W8A16 = 4,       // main GEMM kernel (either path)
    W8A16Reduce = 5, // split-K reduction + epilogue
    AttnPrefill = 6,
    Count = 7
};
void profile_begin(KernelId id, hipStream_t stream);
void profile_end(KernelId id, hipStream_t stream);

} // namespace detail
} // namespace tiny_llm
