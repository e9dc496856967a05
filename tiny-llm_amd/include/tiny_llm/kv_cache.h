// KVCacheManager for MI355X: the reference API (include/tiny_llm/kv_cache.h:
// 15-111) with its semantics and pool layout unchanged, plus the batched
// decode surface (DecodeBatch) that drives the fused HIP kernels.
//
// Pool layout (kv_cache.cpp:69-80, 226-233), one hipMalloc'd block:
//   [slot][layer][K|V][max_seq_len][num_heads][head_dim]  fp16
// so a token's K (or V) row of num_heads*head_dim halves is contiguous.
//
// A block-granular pool (createPaged) instead holds num_blocks blocks of
// block_tokens tokens plus one spare block:
//   [layer][K|V][num_blocks + 1][block_tokens][num_heads][head_dim]  fp16
// and a sequence is handed blocks as it grows (see BlockAllocator).
#pragma once

#include "tiny_llm/hip_utils.h"
#include "tiny_llm/result.h"
#include "tiny_llm/types.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <unordered_map>
#include <utility>
#include <vector>

namespace tiny_llm {

namespace detail {
struct KvView;
struct WorkList;
class BlockAllocator;
struct InlineMeta;
struct PrefillEntry;
class MetaRing;
class Workspace;
} // namespace detail

// Per-sequence cache state (kv_cache.h:15-20).
struct SequenceCache {
    int  seq_id = -1;
    int  current_len = 0;
    int  max_len = 0;
    bool active = false;
};

class KVCacheManager {
  public:
    static Result<std::unique_ptr<KVCacheManager>> create(const KVCacheConfig &config);

    ~KVCacheManager();
    KVCacheManager(const KVCacheManager &) = delete;
    KVCacheManager &operator=(const KVCacheManager &) = delete;
    KVCacheManager(KVCacheManager &&) = delete;
    KVCacheManager &operator=(KVCacheManager &&) = delete;

    Result<int>  allocateSequence(int max_len);
    Result<void> releaseSequence(int seq_id);

    std::pair<half *, half *>         getCache(int seq_id, int layer_idx);
    Result<std::pair<half *, half *>> getCacheChecked(int seq_id, int layer_idx);

    // Copies num_tokens tokens to the sequence tail; does NOT advance the
    // visible length (the caller advances once after all layers).
    Result<void> appendKV(int seq_id, int layer_idx, const half *new_k, const half *new_v,
                          int num_tokens, hipStream_t stream = 0);
    Result<void> advanceSeqLen(int seq_id, int num_tokens);

    int    getSeqLen(int seq_id) const noexcept;
    bool   hasSequence(int seq_id) const noexcept;
    size_t getUsedMemory() const noexcept;
    size_t getTotalMemory() const noexcept;
    size_t getFreeMemory() const noexcept;
    int    getActiveSequenceCount() const noexcept;

    const KVCacheConfig &getConfig() const noexcept { return config_; }

    // ---- additions of the batched path ----
    // Block-granular pool: the reference's API over num_blocks blocks of
    // block_tokens tokens (a power of two >= 16) instead of max_batch_size
    // full max_seq_len slots.  max_batch_size bounds the live sequences;
    // memory follows the tokens held.  appendKV, advanceSeqLen and
    // DecodeBatch::prepare map the blocks they need and fail with "KV cache
    // exhausted" when the pool has too few free blocks; releaseSequence
    // returns a sequence's blocks.  getUsedMemory / getTotalMemory count
    // blocks (num_blocks * blockBytes() in total).
    static Result<std::unique_ptr<KVCacheManager>> createPaged(const KVCacheConfig &config,
                                                               int block_tokens, int num_blocks);
    bool   isBlockPool() const noexcept { return blocks_ != nullptr; }
    int    numBlocks() const noexcept;
    int    freeBlocks() const noexcept;
    size_t blockBytes() const noexcept;
    // Physical blocks of a sequence of a block pool, in token order.
    Result<std::vector<int32_t>> blockTable(int seq_id) const;
    // Patches the device block table with the entries changed since the last
    // call, on `stream` (no-op for other pools).  Every call that launches a
    // kernel reading the table calls this first.
    void syncTable(hipStream_t stream);
    // Maps blocks so that every listed slot holds tokens[i] tokens: all or
    // nothing.
    Result<void> reserveSlots(const int32_t *slots, const int32_t *tokens, int n);
    // Elements from layer l's K base to layer l+1's.
    int64_t layerStride() const noexcept { return layer_stride_; }

    // Paged addressing over the same pool (see tl_kv_set_block_map).
    Result<void>         setBlockMap(int block_tokens, const int32_t *perm, size_t n);
    bool                 isPaged() const noexcept { return block_tokens_ > 0; }
    int                  blockTokens() const noexcept { return block_tokens_; }
    int                  slotOf(int seq_id) const noexcept;
    const SequenceCache *sequence(int seq_id) const noexcept;
    half                *pool() const noexcept { return memory_pool_; }
    size_t               slotBytes() const noexcept { return slot_size_; }
    int                  device() const noexcept { return device_; }
    // Layer view for batch kernels; seq_row_dev holds the slot of each entry.
    detail::KvView layerView(int layer_idx, const int32_t *seq_row_dev) const;

  private:
    explicit KVCacheManager(const KVCacheConfig &config);
    static Result<std::unique_ptr<KVCacheManager>> build(const KVCacheConfig &config,
                                                         int block_tokens, int num_blocks);
    Result<void> exhausted(int64_t need) const;

    size_t calculateOffset(int slot_idx, int layer_idx, bool is_value) const;
    int    findFreeSlot() const;

    KVCacheConfig config_;
    half         *memory_pool_ = nullptr;
    size_t        pool_size_ = 0;
    std::vector<SequenceCache>   slots_;
    std::unordered_map<int, int> seq_to_slot_;
    int                          next_seq_id_ = 0;
    size_t                       slot_size_ = 0;
    int                          device_ = 0;

    int      block_tokens_ = 0;          // 0: reference layout
    int32_t *block_map_dev_ = nullptr;   // [max_batch][max_seq_len/bt] physical block ids
    std::vector<int32_t> block_map_host_;
    int64_t  layer_stride_ = 0;          // elements between consecutive layers' K bases
    std::unique_ptr<detail::BlockAllocator> blocks_;  // block pool only
};

// A decode step over n sequences of one manager.  prepare() snapshots the
// write position (getSeqLen) and attended length (getSeqLen + 1) of each
// sequence and uploads them once; every layer's append / attention / gather
// then reads that snapshot.  One batch is used from one stream (or the caller
// orders streams); entries must be distinct live sequences.
class DecodeBatch {
  public:
    static Result<std::unique_ptr<DecodeBatch>> create(KVCacheManager &mgr, int max_seqs,
                                                       int num_q_heads);
    ~DecodeBatch();
    DecodeBatch(const DecodeBatch &) = delete;
    DecodeBatch &operator=(const DecodeBatch &) = delete;

    Result<void> prepare(const int *seq_ids, int n, hipStream_t stream);
    Result<void> prepareLengths(const int *seq_ids, const int *attended, int n, hipStream_t stream);

    Result<void> append(int layer_begin, int num_layers, const half *new_k, const half *new_v,
                        hipStream_t stream);
    Result<void> attention(int layer_idx, const half *q, half *out, float scale, hipStream_t stream);
    Result<void> decode(int layer_idx, const half *q, const half *new_k, const half *new_v, half *out,
                        float scale, hipStream_t stream);
    Result<void> gather(int layer_idx, half *k_out, half *v_out, int s_max, hipStream_t stream);
    // The K/V projections of the decode step with the append fused into their
    // epilogue: for every entry i, K_i = x_i @ dequant(wk, sk) and V_i likewise
    // (W8A16, kernels/w8a16_matmul.cu) are written straight into the cache at
    // the entry's write position -- the bytes w8a16_matmul + appendKV(n=1)
    // leave there (transformer.cpp:214-226), without the k_buf_/v_buf_ round
    // trip.  x: [n][hidden] fp16; wk/wv: [hidden][num_heads*head_dim] int8;
    // scales [ceil(hidden/group_size)][num_heads*head_dim].  Optionally also
    // q_out[n][num_q_heads*head_dim] = x @ dequant(wq, sq) in the same launch
    // (wq/sq/q_out all null to skip).  packed: the weights are in the layout
    // of kernels::w8a16_pack.
    Result<void> project(int layer_idx, const half *x, int hidden, int group_size, const int8_t *wk,
                         const half *sk, const int8_t *wv, const half *sv, const int8_t *wq,
                         const half *sq, half *q_out, hipStream_t stream, bool packed = false);
    // advanceSeqLen(seq, num_tokens) for every sequence of the last prepare.
    Result<void> commit(int num_tokens);

    int size() const noexcept { return n_; }
    int chunkTokens() const noexcept { return chunk_; }
    int workItems() const noexcept { return n_work_; }
    const std::vector<int32_t> &attendedLengths() const noexcept { return lens_; }

  private:
    DecodeBatch(KVCacheManager &mgr, int max_seqs, int num_q_heads);
    Result<void> upload(const int *seq_ids, const int *attended, int n, bool appendable,
                        hipStream_t stream);
    Result<void> run_attention(int layer_idx, const half *q, const half *new_k, const half *new_v,
                               half *out, float scale, hipStream_t stream);
    void         upload_device(hipStream_t stream);

    KVCacheManager &mgr_;
    int             max_seqs_;
    int             num_q_heads_;
    int             n_ = 0;
    bool            appendable_ = false;
    int             chunk_ = 0;
    int             n_work_ = 0;
    int             fused_heads_ = 0;
    bool            fused_chunked_ = false;
    bool            any_multi_ = false;
    bool            any_empty_ = false;
    std::vector<int32_t> ids_, lens_, wpos_, slot_;
    std::unique_ptr<detail::MetaRing>  meta_;
    std::unique_ptr<detail::Workspace> work_;
    std::unique_ptr<detail::Workspace> gemm_work_;
    std::unique_ptr<detail::WorkList>  plan_;
    std::unique_ptr<detail::InlineMeta> inl_;
    bool                               inline_ok_ = false; // metadata fits in kernel arguments
    bool                               uploaded_ = false;  // device copy of this prepare made
    const int32_t  *d_lens_ = nullptr, *d_wpos_ = nullptr, *d_slot_ = nullptr;
    const int32_t  *d_part_base_ = nullptr, *d_work_ = nullptr;
};

// A prefill step over n sequences of one manager: sequence i brings
// num_tokens[i] new tokens at positions getSeqLen .. getSeqLen+num_tokens-1.
// prepare() snapshots the write positions (and, for a block pool, maps the
// blocks they need); every layer's append / attention then reads that
// snapshot; commit() advances each sequence by its token count.  New tokens
// are token-major and sequences back to back: K/V rows [T][num_heads *
// head_dim], queries and outputs [T][num_q_heads][head_dim], T = the sum of
// num_tokens.  Query token j of sequence i attends to the sequence's cache
// positions 0 .. getSeqLen + j (causal, the new tokens included), which is
// the prefill branch of TransformerLayer::attention (transformer.cpp:
// 222-241) reading the cache instead of k_buf_/v_buf_; with getSeqLen > 0 it
// continues a prompt chunk by chunk.
class PrefillBatch {
  public:
    static Result<std::unique_ptr<PrefillBatch>> create(KVCacheManager &mgr, int max_seqs,
                                                        int num_q_heads);
    ~PrefillBatch();
    PrefillBatch(const PrefillBatch &) = delete;
    PrefillBatch &operator=(const PrefillBatch &) = delete;

    Result<void> prepare(const int *seq_ids, const int *num_tokens, int n, hipStream_t stream);
    // appendKV of every sequence's new tokens for one layer.
    Result<void> append(int layer_idx, const half *new_k, const half *new_v, hipStream_t stream);
    // Causal attention of the new tokens over the cache (after append).
    Result<void> attention(int layer_idx, const half *q, half *out, float scale, hipStream_t stream);
    // append + attention in one launch: keys at or past a sequence's write
    // position are read from new_k/new_v, and the attention kernel writes
    // those rows into the cache (the bytes of append()).
    Result<void> prefill(int layer_idx, const half *q, const half *new_k, const half *new_v,
                         half *out, float scale, hipStream_t stream);
    // advanceSeqLen(seq, num_tokens[i]) for every sequence of the last prepare.
    Result<void> commit();

    int size() const noexcept { return n_; }
    int tokens() const noexcept { return tokens_; }

  private:
    PrefillBatch(KVCacheManager &mgr, int max_seqs, int num_q_heads);
    Result<void> launch(int layer_idx, const half *q, const half *new_k, const half *new_v, half *out,
                        float scale, hipStream_t stream);
    // Device copy of the attention work list, made on the first launch that
    // reads it (append() needs none).
    void upload_device(hipStream_t stream);

    KVCacheManager      &mgr_;
    int                  max_seqs_;
    int                  num_q_heads_;
    int                  n_ = 0;
    int                  tokens_ = 0;
    int                  n_items_ = 0;
    int                  waves_ = 8; // waves per attention workgroup the work list was planned for
    int                  max_keys_ = 0;
    std::vector<int32_t> ids_, counts_, slots_, pos0_, work_;
    bool                 uploaded_ = false;
    std::unique_ptr<detail::MetaRing> meta_;
    const int32_t       *d_work_ = nullptr;
};

} // namespace tiny_llm
