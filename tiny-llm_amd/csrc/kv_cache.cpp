// KVCacheManager and DecodeBatch for MI355X.
//
// Bookkeeping follows src/kv_cache.cpp of the reference (cited per function):
// the same validation order, error texts, slot policy, id policy, layout and
// "append does not advance" contract.  Device work is HIP: the pool is one
// hipMalloc'd block zeroed at create; appendKV keeps the reference's two
// stream-ordered D2D copies; the batched surface launches the fused kernels
// of csrc/kernels/.
#include "tiny_llm/kv_cache.h"

#include "block_allocator.h"
#include "kernels/kv_kernels.h"
#include "kernels/prefill.h"
#include "kernels/w8a16.h"
#include "runtime.h"
#include "tl_log.h"

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace tiny_llm {

using detail::KvView;

KVCacheManager::KVCacheManager(const KVCacheConfig &config) : config_(config) {}

// KVCacheManager::create (kv_cache.cpp:8-60).
Result<std::unique_ptr<KVCacheManager>> KVCacheManager::create(const KVCacheConfig &config) {
    return build(config, 0, 0);
}

Result<std::unique_ptr<KVCacheManager>> KVCacheManager::createPaged(const KVCacheConfig &config,
                                                                    int block_tokens,
                                                                    int num_blocks) {
    using R = Result<std::unique_ptr<KVCacheManager>>;
    if (block_tokens < 16 || (block_tokens & (block_tokens - 1)) != 0)
        return R::err("KVCacheManager: block_tokens must be a power of two >= 16 (got " +
                      std::to_string(block_tokens) + ")");
    if (num_blocks <= 0 || num_blocks == INT32_MAX)
        return R::err("KVCacheManager: num_blocks must be in [1, 2^31 - 2] (got " +
                      std::to_string(num_blocks) + ")");
    // The kernels address a token inside its block with a 32-bit byte offset.
    if (config.num_heads > 0 && config.head_dim > 0 &&
        static_cast<int64_t>(block_tokens) * config.num_heads * config.head_dim * 2 >
            static_cast<int64_t>(UINT32_MAX))
        return R::err("KVCacheManager: a block of " + std::to_string(block_tokens) +
                      " tokens exceeds 4 GiB per layer and K/V region");
    return build(config, block_tokens, num_blocks);
}

// The checks and pool set-up of create (kv_cache.cpp:8-60); with
// block_tokens > 0 the pool is the block pool of createPaged.
Result<std::unique_ptr<KVCacheManager>> KVCacheManager::build(const KVCacheConfig &config,
                                                              int block_tokens, int num_blocks) {
    using R = Result<std::unique_ptr<KVCacheManager>>;
    if (config.num_layers <= 0 || config.num_heads <= 0 || config.head_dim <= 0 ||
        config.max_seq_len <= 0 || config.max_batch_size <= 0) {
        return R::err("KVCacheManager: invalid configuration parameters");
    }
    auto manager = std::unique_ptr<KVCacheManager>(new KVCacheManager(config));

    const size_t kv_per_layer =
        static_cast<size_t>(config.num_heads) * config.max_seq_len * config.head_dim;
    const size_t kv_total = kv_per_layer * static_cast<size_t>(config.num_layers) * 2;
    if (kv_total > SIZE_MAX / sizeof(half)) return R::err("KVCacheManager: memory size overflow");
    manager->slot_size_ = kv_total * sizeof(half);
    if (block_tokens == 0) {
        if (manager->slot_size_ > SIZE_MAX / static_cast<size_t>(config.max_batch_size))
            return R::err("KVCacheManager: pool size overflow");
        manager->pool_size_ = manager->slot_size_ * static_cast<size_t>(config.max_batch_size);
        manager->layer_stride_ = 2 * static_cast<int64_t>(kv_per_layer);
    } else {
        const size_t block_elems =
            static_cast<size_t>(block_tokens) * config.num_heads * config.head_dim;
        const size_t per_kv = block_elems * (static_cast<size_t>(num_blocks) + 1);
        if (per_kv > SIZE_MAX / (2 * sizeof(half) * static_cast<size_t>(config.num_layers)))
            return R::err("KVCacheManager: pool size overflow");
        manager->pool_size_ = per_kv * 2 * static_cast<size_t>(config.num_layers) * sizeof(half);
        manager->layer_stride_ = 2 * static_cast<int64_t>(per_kv);
        manager->block_tokens_ = block_tokens;
        const int bpr = (config.max_seq_len + block_tokens - 1) / block_tokens;
        manager->blocks_.reset(new detail::BlockAllocator(config.max_batch_size, bpr, num_blocks));
    }

    hipError_t err = hipGetDevice(&manager->device_);
    if (err != hipSuccess)
        return R::err(std::string("KVCacheManager: hipGetDevice failed: ") + hipGetErrorString(err));
    err = hipMalloc(reinterpret_cast<void **>(&manager->memory_pool_), manager->pool_size_);
    if (err != hipSuccess) {
        manager->memory_pool_ = nullptr;
        return R::err(std::string("KVCacheManager: hipMalloc failed: ") + hipGetErrorString(err));
    }
    err = hipMemset(manager->memory_pool_, 0, manager->pool_size_);
    if (err != hipSuccess) {
        (void)hipFree(manager->memory_pool_);
        manager->memory_pool_ = nullptr;
        return R::err(std::string("KVCacheManager: hipMemset failed: ") + hipGetErrorString(err));
    }
    if (manager->blocks_) {
        // Every entry starts at the spare block.
        const std::vector<int32_t> &t = manager->blocks_->table();
        err = hipMalloc(reinterpret_cast<void **>(&manager->block_map_dev_), t.size() * sizeof(int32_t));
        if (err == hipSuccess)
            err = hipMemcpy(manager->block_map_dev_, t.data(), t.size() * sizeof(int32_t),
                            hipMemcpyHostToDevice);
        if (err != hipSuccess)
            return R::err(std::string("KVCacheManager: block table: ") + hipGetErrorString(err));
    }

    manager->slots_.resize(static_cast<size_t>(config.max_batch_size));
    for (auto &slot : manager->slots_) {
        slot.active = false;
        slot.seq_id = -1;
        slot.current_len = 0;
        slot.max_len = config.max_seq_len;
    }
    return R::ok(std::move(manager));
}

// ~KVCacheManager (kv_cache.cpp:62-67).
KVCacheManager::~KVCacheManager() {
    if (block_map_dev_) (void)hipFree(block_map_dev_);
    if (memory_pool_) {
        (void)hipFree(memory_pool_);
        memory_pool_ = nullptr;
    }
}

// calculateOffset (kv_cache.cpp:69-80): [Layer 0 K][Layer 0 V][Layer 1 K]...
size_t KVCacheManager::calculateOffset(int slot_idx, int layer_idx, bool is_value) const {
    const size_t kv_per_layer =
        static_cast<size_t>(config_.num_heads) * config_.max_seq_len * config_.head_dim;
    const size_t slot_offset = static_cast<size_t>(slot_idx) * slot_size_ / sizeof(half);
    const size_t layer_offset = static_cast<size_t>(layer_idx) * kv_per_layer * 2;
    const size_t kv_offset = is_value ? kv_per_layer : 0;
    return slot_offset + layer_offset + kv_offset;
}

// findFreeSlot (kv_cache.cpp:82-89): lowest inactive slot.
int KVCacheManager::findFreeSlot() const {
    for (int i = 0; i < static_cast<int>(slots_.size()); ++i)
        if (!slots_[static_cast<size_t>(i)].active) return i;
    return -1;
}

// allocateSequence (kv_cache.cpp:91-119).
Result<int> KVCacheManager::allocateSequence(int max_len) {
    if (max_len <= 0 || max_len > config_.max_seq_len) {
        return Result<int>::err("Invalid max_len: " + std::to_string(max_len) + " (must be 1-" +
                                std::to_string(config_.max_seq_len) + ")");
    }
    const int slot_idx = findFreeSlot();
    if (slot_idx < 0) {
        return Result<int>::err("KV cache exhausted: no free slots available. Used: " +
                                std::to_string(getUsedMemory()) +
                                " bytes, Total: " + std::to_string(getTotalMemory()) + " bytes");
    }
    const int seq_id = next_seq_id_++;
    auto     &slot = slots_[static_cast<size_t>(slot_idx)];
    slot.seq_id = seq_id;
    slot.current_len = 0;
    slot.max_len = max_len;
    slot.active = true;
    seq_to_slot_[seq_id] = slot_idx;
    return Result<int>::ok(seq_id);
}

// releaseSequence (kv_cache.cpp:121-137).  Device bytes are not cleared.
Result<void> KVCacheManager::releaseSequence(int seq_id) {
    auto it = seq_to_slot_.find(seq_id);
    if (it == seq_to_slot_.end()) {
        TL_LOG_WARN("releaseSequence: sequence not found: %d", seq_id);
        return Result<void>::err("Sequence not found: " + std::to_string(seq_id));
    }
    auto &slot = slots_[static_cast<size_t>(it->second)];
    if (blocks_) blocks_->release(it->second);
    slot.active = false;
    slot.seq_id = -1;
    slot.current_len = 0;
    TL_LOG_DEBUG("KVCache: released sequence %d (slot %d)", seq_id, it->second);
    seq_to_slot_.erase(it);
    return Result<void>::ok();
}

// getCacheChecked (kv_cache.cpp:139-157).
Result<std::pair<half *, half *>> KVCacheManager::getCacheChecked(int seq_id, int layer_idx) {
    using R = Result<std::pair<half *, half *>>;
    auto it = seq_to_slot_.find(seq_id);
    if (it == seq_to_slot_.end()) return R::err("Sequence not found: " + std::to_string(seq_id));
    if (layer_idx < 0 || layer_idx >= config_.num_layers) {
        return R::err("getCache: Invalid layer_idx: " + std::to_string(layer_idx) +
                      " (valid range: 0-" + std::to_string(config_.num_layers - 1) + ")");
    }
    if (isPaged()) {
        return R::err("getCache: paged layout (block_tokens=" + std::to_string(block_tokens_) +
                      ") has no contiguous per-sequence region");
    }
    const size_t k_offset = calculateOffset(it->second, layer_idx, false);
    const size_t v_offset = calculateOffset(it->second, layer_idx, true);
    return R::ok({memory_pool_ + k_offset, memory_pool_ + v_offset});
}

// getCache (kv_cache.cpp:159-166).
std::pair<half *, half *> KVCacheManager::getCache(int seq_id, int layer_idx) {
    auto result = getCacheChecked(seq_id, layer_idx);
    if (result.isErr()) {
        TL_LOG_WARN("getCache: %s", result.error().c_str());
        return {nullptr, nullptr};
    }
    return result.value();
}

// appendKV (kv_cache.cpp:168-238).
Result<void> KVCacheManager::appendKV(int seq_id, int layer_idx, const half *new_k,
                                      const half *new_v, int num_tokens, hipStream_t stream) {
    if (new_k == nullptr) {
        TL_LOG_ERROR("appendKV: new_k is null");
        return Result<void>::err("new_k is null");
    }
    if (new_v == nullptr) {
        TL_LOG_ERROR("appendKV: new_v is null");
        return Result<void>::err("new_v is null");
    }
    if (num_tokens <= 0) {
        TL_LOG_ERROR("appendKV: invalid num_tokens: %d", num_tokens);
        return Result<void>::err("appendKV: num_tokens must be positive: " +
                                 std::to_string(num_tokens));
    }
    if (layer_idx < 0 || layer_idx >= config_.num_layers) {
        std::string msg = "appendKV: Invalid layer_idx: " + std::to_string(layer_idx) +
                          " (valid range: 0-" + std::to_string(config_.num_layers - 1) + ")";
        TL_LOG_ERROR("%s", msg.c_str());
        return Result<void>::err(msg);
    }
    auto it = seq_to_slot_.find(seq_id);
    if (it == seq_to_slot_.end()) {
        TL_LOG_ERROR("appendKV: sequence not found: %d", seq_id);
        return Result<void>::err("appendKV: sequence not found: " + std::to_string(seq_id));
    }
    const int slot_idx = it->second;
    auto     &slot = slots_[static_cast<size_t>(slot_idx)];
    // All layers of a step see the same write position: the length is
    // advanced once after the last layer (kv_cache.cpp:204-208).
    const int write_pos = slot.current_len;
    if (write_pos + num_tokens > slot.max_len) {
        TL_LOG_ERROR("appendKV: cache overflow. seq_id=%d, write_pos=%d, num_tokens=%d, max_len=%d",
                   seq_id, write_pos, num_tokens, slot.max_len);
        return Result<void>::err("appendKV: cache overflow. Current: " + std::to_string(write_pos) +
                                 ", appending: " + std::to_string(num_tokens) +
                                 ", max: " + std::to_string(slot.max_len));
    }
    const int row = config_.num_heads * config_.head_dim;
    if (blocks_) {
        const int need = (write_pos + num_tokens + block_tokens_ - 1) / block_tokens_;
        if (!blocks_->ensure(slot_idx, need)) {
            auto r = exhausted(need - blocks_->mapped(slot_idx));
            TL_LOG_ERROR("appendKV: %s", r.error().c_str());
            return r;
        }
        syncTable(stream);
    }
    if (!isPaged()) {
        half        *k_cache = memory_pool_ + calculateOffset(slot_idx, layer_idx, false);
        half        *v_cache = memory_pool_ + calculateOffset(slot_idx, layer_idx, true);
        const size_t pos_offset = static_cast<size_t>(write_pos) * row;
        const size_t copy_size = static_cast<size_t>(num_tokens) * row * sizeof(half);
        HIP_CHECK(hipMemcpyAsync(k_cache + pos_offset, new_k, copy_size, hipMemcpyDeviceToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(v_cache + pos_offset, new_v, copy_size, hipMemcpyDeviceToDevice, stream));
    } else {
        // Paged pool: the tokens cross blocks, so scatter them with the
        // append kernel through this slot's row of the block map.
        KvView v = layerView(layer_idx, nullptr);
        v.block_table = block_map_dev_ + static_cast<size_t>(slot_idx) * v.bt_stride;
        v.bt_stride = 0;
        detail::launch_kv_append(v, 0, nullptr, write_pos, num_tokens, 1, row, new_k, new_v, stream);
    }
    TL_LOG_TRACE("appendKV: seq_id=%d, layer=%d, num_tokens=%d, write_pos=%d", seq_id, layer_idx,
               num_tokens, write_pos);
    return Result<void>::ok();
}

// advanceSeqLen (kv_cache.cpp:240-259).
Result<void> KVCacheManager::advanceSeqLen(int seq_id, int num_tokens) {
    if (num_tokens <= 0) {
        TL_LOG_ERROR("advanceSeqLen: invalid num_tokens: %d", num_tokens);
        return Result<void>::err("advanceSeqLen: num_tokens must be positive: " +
                                 std::to_string(num_tokens));
    }
    auto it = seq_to_slot_.find(seq_id);
    if (it == seq_to_slot_.end()) {
        TL_LOG_ERROR("advanceSeqLen: sequence not found: %d", seq_id);
        return Result<void>::err("advanceSeqLen: sequence not found: " + std::to_string(seq_id));
    }
    auto     &slot = slots_[static_cast<size_t>(it->second)];
    const int old_len = slot.current_len;
    const int new_len = std::min(slot.current_len + num_tokens, slot.max_len);
    if (blocks_) {
        // Positions made visible without an append still get blocks, so
        // that every visible token of a block pool is backed.
        const int need = (new_len + block_tokens_ - 1) / block_tokens_;
        if (!blocks_->ensure(it->second, need)) {
            auto r = exhausted(need - blocks_->mapped(it->second));
            TL_LOG_ERROR("advanceSeqLen: %s", r.error().c_str());
            return r;
        }
    }
    slot.current_len = new_len;
    TL_LOG_TRACE("advanceSeqLen: seq_id=%d, %d -> %d", seq_id, old_len, slot.current_len);
    (void)old_len;
    return Result<void>::ok();
}

// getSeqLen / hasSequence / memory statistics (kv_cache.cpp:261-295).
int KVCacheManager::getSeqLen(int seq_id) const noexcept {
    auto it = seq_to_slot_.find(seq_id);
    return it == seq_to_slot_.end() ? 0 : slots_[static_cast<size_t>(it->second)].current_len;
}
bool KVCacheManager::hasSequence(int seq_id) const noexcept {
    return seq_to_slot_.find(seq_id) != seq_to_slot_.end();
}
size_t KVCacheManager::getUsedMemory() const noexcept {
    if (blocks_) return static_cast<size_t>(blocks_->usedBlocks()) * blockBytes();
    return static_cast<size_t>(getActiveSequenceCount()) * slot_size_;
}
size_t KVCacheManager::getTotalMemory() const noexcept {
    return blocks_ ? static_cast<size_t>(blocks_->numBlocks()) * blockBytes() : pool_size_;
}
size_t KVCacheManager::getFreeMemory() const noexcept { return getTotalMemory() - getUsedMemory(); }
int    KVCacheManager::getActiveSequenceCount() const noexcept {
    int count = 0;
    for (const auto &slot : slots_) count += slot.active ? 1 : 0;
    return count;
}

int KVCacheManager::slotOf(int seq_id) const noexcept {
    auto it = seq_to_slot_.find(seq_id);
    return it == seq_to_slot_.end() ? -1 : it->second;
}

const SequenceCache *KVCacheManager::sequence(int seq_id) const noexcept {
    const int s = slotOf(seq_id);
    return s < 0 ? nullptr : &slots_[static_cast<size_t>(s)];
}

int KVCacheManager::numBlocks() const noexcept { return blocks_ ? blocks_->numBlocks() : 0; }
int KVCacheManager::freeBlocks() const noexcept { return blocks_ ? blocks_->freeBlocks() : 0; }
size_t KVCacheManager::blockBytes() const noexcept {
    return blocks_ ? static_cast<size_t>(block_tokens_) * config_.num_heads * config_.head_dim *
                         config_.num_layers * 2 * sizeof(half)
                   : 0;
}

Result<std::vector<int32_t>> KVCacheManager::blockTable(int seq_id) const {
    using R = Result<std::vector<int32_t>>;
    const int slot = slotOf(seq_id);
    if (!blocks_ && block_map_host_.empty()) return R::err("blockTable: not a paged pool");
    if (slot < 0) return R::err("Sequence not found: " + std::to_string(seq_id));
    if (!blocks_) { // block map over the slot pool: every block of the slot is mapped
        const size_t per_slot = static_cast<size_t>(config_.max_seq_len / block_tokens_);
        const auto   first = block_map_host_.begin() + static_cast<std::ptrdiff_t>(slot * per_slot);
        return R::ok(std::vector<int32_t>(first, first + static_cast<std::ptrdiff_t>(per_slot)));
    }
    const auto  &t = blocks_->table();
    const size_t base = static_cast<size_t>(slot) * static_cast<size_t>(blocks_->blocksPerRow());
    return R::ok(std::vector<int32_t>(t.begin() + static_cast<std::ptrdiff_t>(base),
                                      t.begin() + static_cast<std::ptrdiff_t>(base) + blocks_->mapped(slot)));
}

Result<void> KVCacheManager::exhausted(int64_t need) const {
    return Result<void>::err("KV cache exhausted: no free blocks available. Needed: " +
                             std::to_string(need) + " blocks, free: " +
                             std::to_string(blocks_->freeBlocks()) + " of " +
                             std::to_string(blocks_->numBlocks()));
}

void KVCacheManager::syncTable(hipStream_t stream) {
    if (!blocks_ || !blocks_->hasUpdates()) return;
    const auto upd = blocks_->takeUpdates();
    detail::launch_table_update(block_map_dev_, upd.data(), upd.size(), stream);
}

Result<void> KVCacheManager::reserveSlots(const int32_t *slots, const int32_t *tokens, int n) {
    if (!blocks_ || n <= 0) return Result<void>::ok();
    std::vector<int> rows(static_cast<size_t>(n)), need(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) {
        rows[static_cast<size_t>(i)] = slots[i];
        need[static_cast<size_t>(i)] = (tokens[i] + block_tokens_ - 1) / block_tokens_;
    }
    const int64_t short_by = blocks_->shortfall(rows.data(), need.data(), n);
    if (short_by > 0) return exhausted(short_by + blocks_->freeBlocks());
    for (int i = 0; i < n; ++i) blocks_->ensure(rows[static_cast<size_t>(i)], need[static_cast<size_t>(i)]);
    return Result<void>::ok();
}

Result<void> KVCacheManager::setBlockMap(int block_tokens, const int32_t *perm, size_t n) {
    if (blocks_) return Result<void>::err("setBlockMap: a block pool maps its blocks itself");
    if (getActiveSequenceCount() != 0)
        return Result<void>::err("setBlockMap: the block map can only change with no live sequences");
    if (perm == nullptr) {
        if (block_map_dev_) HIP_CHECK(hipFree(block_map_dev_));
        block_map_dev_ = nullptr;
        block_map_host_.clear();
        block_tokens_ = 0;
        return Result<void>::ok();
    }
    if (block_tokens < 16 || (block_tokens & (block_tokens - 1)) != 0 ||
        config_.max_seq_len % block_tokens != 0) {
        return Result<void>::err("setBlockMap: block_tokens must be a power of two >= 16 dividing "
                                 "max_seq_len (got " + std::to_string(block_tokens) + ")");
    }
    const size_t per_slot = static_cast<size_t>(config_.max_seq_len / block_tokens);
    const size_t total = per_slot * static_cast<size_t>(config_.max_batch_size);
    if (n != total) {
        return Result<void>::err("setBlockMap: expected " + std::to_string(total) +
                                 " entries, got " + std::to_string(n));
    }
    // Physical block ids in units of block_tokens*num_heads*head_dim elements
    // from a layer's K base: slot s' block j' -> s' * (2*L*M/bt) + j'.
    const size_t slot_blocks = 2 * static_cast<size_t>(config_.num_layers) * per_slot;
    if ((static_cast<size_t>(config_.max_batch_size) - 1) * slot_blocks + per_slot > INT32_MAX)
        return Result<void>::err("setBlockMap: pool too large for 32-bit block ids");
    std::vector<char>    seen(total, 0);
    std::vector<int32_t> phys(total);
    for (size_t x = 0; x < total; ++x) {
        const int32_t y = perm[x];
        if (y < 0 || static_cast<size_t>(y) >= total || seen[static_cast<size_t>(y)])
            return Result<void>::err("setBlockMap: perm is not a permutation (entry " +
                                     std::to_string(x) + ")");
        seen[static_cast<size_t>(y)] = 1;
        const size_t s = static_cast<size_t>(y) / per_slot, j = static_cast<size_t>(y) % per_slot;
        phys[x] = static_cast<int32_t>(s * slot_blocks + j);
    }
    if (block_map_dev_) HIP_CHECK(hipFree(block_map_dev_));
    block_map_dev_ = nullptr;
    HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&block_map_dev_), total * sizeof(int32_t)));
    HIP_CHECK(hipMemcpy(block_map_dev_, phys.data(), total * sizeof(int32_t), hipMemcpyHostToDevice));
    block_map_host_ = std::move(phys);
    block_tokens_ = block_tokens;
    return Result<void>::ok();
}

KvView KVCacheManager::layerView(int layer_idx, const int32_t *seq_row_dev) const {
    KvView v;
    v.k_base = memory_pool_ + static_cast<int64_t>(layer_idx) * layer_stride_;
    v.v_base = v.k_base + layer_stride_ / 2;
    v.seq_row = seq_row_dev;
    v.tok_stride = static_cast<int64_t>(config_.num_heads) * config_.head_dim;
    v.head_stride = config_.head_dim;
    if (isPaged()) {
        int lg = 0;
        while ((1 << lg) < block_tokens_) ++lg;
        v.block_table = block_map_dev_;
        v.bt_stride = blocks_ ? blocks_->blocksPerRow() : config_.max_seq_len / block_tokens_;
        v.log2_blk = lg;
        v.blk_stride = static_cast<int64_t>(block_tokens_) * v.tok_stride;
    } else {
        v.block_table = nullptr;
        v.bt_stride = 0;
        v.log2_blk = 30;
        v.blk_stride = static_cast<int64_t>(slot_size_ / sizeof(half));
    }
    return v;
}

// ======================================================================
// DecodeBatch
// ======================================================================

DecodeBatch::DecodeBatch(KVCacheManager &mgr, int max_seqs, int num_q_heads)
    : mgr_(mgr), max_seqs_(max_seqs), num_q_heads_(num_q_heads), meta_(new detail::MetaRing(4)),
      work_(new detail::Workspace()), gemm_work_(new detail::Workspace()),
      plan_(new detail::WorkList()),
      inl_(new detail::InlineMeta()) {}

DecodeBatch::~DecodeBatch() = default;

Result<std::unique_ptr<DecodeBatch>> DecodeBatch::create(KVCacheManager &mgr, int max_seqs,
                                                         int num_q_heads) {
    using R = Result<std::unique_ptr<DecodeBatch>>;
    const KVCacheConfig &cfg = mgr.getConfig();
    if (max_seqs <= 0) return R::err("DecodeBatch: max_seqs must be positive");
    if (num_q_heads <= 0 || num_q_heads % cfg.num_heads != 0)
        return R::err("DecodeBatch: num_q_heads (" + std::to_string(num_q_heads) +
                      ") must be a positive multiple of num_heads (" +
                      std::to_string(cfg.num_heads) + ")");
    if (!detail::attn_shape_supported(cfg.head_dim, num_q_heads / cfg.num_heads))
        return R::err("DecodeBatch: unsupported head_dim/group (head_dim in {32,64,128,256}, "
                      "num_q_heads/num_heads in {1,2,4,8})");
    std::unique_ptr<DecodeBatch> batch(new DecodeBatch(mgr, max_seqs, num_q_heads));
    // Size the metadata ring for a full batch now, so that no step allocates
    // pinned or device memory: 4 words per entry and 2 per work item, with at
    // most one item per entry plus 2 per resident workgroup slot (the planner
    // never splits finer than the slots need), 4 MiB at most.
    const size_t slots = 2 * static_cast<size_t>(detail::kPlanSlotsPerCU) *
                         static_cast<size_t>(detail::device_cus());
    const size_t n = static_cast<size_t>(max_seqs);
    const size_t words = 4 * n + 1 + 2 * (n + slots);
    batch->meta_->reserve(std::min<size_t>(words * 4, size_t(4) << 20));
    return R::ok(std::move(batch));
}

Result<void> DecodeBatch::upload(const int *seq_ids, const int *attended, int n, bool appendable,
                                 hipStream_t stream) {
    if (n < 0 || n > max_seqs_)
        return Result<void>::err("DecodeBatch: n=" + std::to_string(n) + " outside [0, " +
                                 std::to_string(max_seqs_) + "]");
    if (n > 0 && seq_ids == nullptr) return Result<void>::err("DecodeBatch: seq_ids is null");
    // A failed prepare leaves an empty batch.
    n_ = 0;
    appendable_ = false;
    ids_.clear();
    const KVCacheConfig &cfg = mgr_.getConfig();
    std::vector<char>    taken(static_cast<size_t>(cfg.max_batch_size), 0);
    lens_.assign(static_cast<size_t>(n), 0);
    wpos_.assign(static_cast<size_t>(n), 0);
    slot_.assign(static_cast<size_t>(n), 0);
    for (int i = 0; i < n; ++i) {
        const int            id = seq_ids[i];
        const SequenceCache *sc = mgr_.sequence(id);
        if (!sc) return Result<void>::err("DecodeBatch: sequence not found: " + std::to_string(id));
        const int slot = mgr_.slotOf(id);
        if (taken[static_cast<size_t>(slot)])
            return Result<void>::err("DecodeBatch: duplicate sequence in batch: " + std::to_string(id));
        taken[static_cast<size_t>(slot)] = 1;
        slot_[static_cast<size_t>(i)] = slot;
        wpos_[static_cast<size_t>(i)] = sc->current_len;
        if (appendable) {
            if (sc->current_len + 1 > sc->max_len) {
                return Result<void>::err("appendKV: cache overflow. Current: " +
                                         std::to_string(sc->current_len) +
                                         ", appending: 1, max: " + std::to_string(sc->max_len));
            }
            lens_[static_cast<size_t>(i)] = sc->current_len + 1;
        } else {
            const int a = attended[i];
            if (a < 0 || a > sc->max_len)
                return Result<void>::err("DecodeBatch: attended length " + std::to_string(a) +
                                         " of sequence " + std::to_string(id) + " outside [0, " +
                                         std::to_string(sc->max_len) + "]");
            lens_[static_cast<size_t>(i)] = a;
        }
    }
    if (mgr_.isBlockPool()) {
        // Back the decode token's position (and, for attended lengths, what
        // the kernels read) with blocks before any kernel of the step runs.
        if (appendable) {
            auto r = mgr_.reserveSlots(slot_.data(), lens_.data(), n);
            if (r.isErr()) return r;
        }
        mgr_.syncTable(stream);
    }
    // Split-K plan: work items (entry, chunk), longest first.
    detail::WorkList &wl = *plan_;
    detail::plan_work(lens_.data(), n, cfg.num_heads, cfg.head_dim, wl);
    chunk_ = wl.chunk;
    fused_heads_ = wl.fused_heads;
    fused_chunked_ = wl.fused_chunked;
    any_multi_ = wl.any_multi;
    any_empty_ = wl.any_empty;
    n_work_ = wl.n_work;
    n_ = n;
    appendable_ = appendable;
    ids_.assign(seq_ids, seq_ids + n);
    // Small batches carry their metadata in the attention kernel's arguments;
    // the device copy is made only when a kernel that reads it is launched.
    inline_ok_ = detail::pack_inline(lens_.data(), wl, slot_.data(), n, *inl_);
    uploaded_ = false;
    if (!inline_ok_) upload_device(stream);
    return Result<void>::ok();
}

// Device copy of [lens | wpos | slot | part_base | work] through the ring.
void DecodeBatch::upload_device(hipStream_t stream) {
    if (uploaded_) return;
    const detail::WorkList &wl = *plan_;
    const size_t            n1 = static_cast<size_t>(n_);
    const size_t            words = 3 * n1 + (n1 + 1) + 2 * static_cast<size_t>(n_work_);
    int32_t                *h = static_cast<int32_t *>(meta_->begin(words * sizeof(int32_t)));
    std::memcpy(h, lens_.data(), n1 * 4);
    std::memcpy(h + n1, wpos_.data(), n1 * 4);
    std::memcpy(h + 2 * n1, slot_.data(), n1 * 4);
    std::memcpy(h + 3 * n1, wl.part_base.data(), (n1 + 1) * 4);
    if (n_work_ > 0) std::memcpy(h + 4 * n1 + 1, wl.work.data(), 2 * static_cast<size_t>(n_work_) * 4);
    const int32_t *d = static_cast<const int32_t *>(meta_->commit(stream));
    d_lens_ = d;
    d_wpos_ = d + n1;
    d_slot_ = d + 2 * n1;
    d_part_base_ = d + 3 * n1;
    d_work_ = d + 4 * n1 + 1;
    uploaded_ = true;
}

Result<void> DecodeBatch::prepare(const int *seq_ids, int n, hipStream_t stream) {
    return upload(seq_ids, nullptr, n, true, stream);
}

// The commit of InferenceEngine::decodeStep (inference_engine.cpp:291),
// advanceSeqLen(seq, num_tokens), for every sequence of the last prepare.
Result<void> DecodeBatch::commit(int num_tokens) {
    for (const int id : ids_) {
        auto r = mgr_.advanceSeqLen(id, num_tokens);
        if (r.isErr()) return r;
    }
    return Result<void>::ok();
}

Result<void> DecodeBatch::prepareLengths(const int *seq_ids, const int *attended, int n,
                                         hipStream_t stream) {
    if (n > 0 && attended == nullptr) return Result<void>::err("DecodeBatch: attended is null");
    return upload(seq_ids, attended, n, false, stream);
}

Result<void> DecodeBatch::append(int layer_begin, int num_layers, const half *new_k,
                                 const half *new_v, hipStream_t stream) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (!appendable_)
        return Result<void>::err("DecodeBatch: append needs a batch made by prepare()");
    if (new_k == nullptr) return Result<void>::err("new_k is null");
    if (new_v == nullptr) return Result<void>::err("new_v is null");
    if (num_layers <= 0 || layer_begin < 0 || layer_begin + num_layers > cfg.num_layers)
        return Result<void>::err("DecodeBatch: layers [" + std::to_string(layer_begin) + ", " +
                                 std::to_string(layer_begin + num_layers) + ") outside [0, " +
                                 std::to_string(cfg.num_layers) + ")");
    if (n_ == 0) return Result<void>::ok();
    upload_device(stream);
    const KvView v = mgr_.layerView(layer_begin, d_slot_);
    detail::launch_kv_append(v, mgr_.layerStride(), d_wpos_, 0, n_, num_layers,
                             cfg.num_heads * cfg.head_dim, new_k, new_v, stream);
    return Result<void>::ok();
}

Result<void> DecodeBatch::attention(int layer_idx, const half *q, half *out, float scale,
                                    hipStream_t stream) {
    return run_attention(layer_idx, q, nullptr, nullptr, out, scale, stream);
}

Result<void> DecodeBatch::run_attention(int layer_idx, const half *q, const half *new_k,
                                        const half *new_v, half *out, float scale,
                                        hipStream_t stream) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (q == nullptr || out == nullptr) return Result<void>::err("DecodeBatch: q/out is null");
    if (layer_idx < 0 || layer_idx >= cfg.num_layers)
        return Result<void>::err("DecodeBatch: Invalid layer_idx: " + std::to_string(layer_idx));
    if (n_ == 0) return Result<void>::ok();
    if (!inline_ok_) upload_device(stream);
    detail::AttnPlan plan;
    plan.seq_lens = d_lens_;
    plan.work = d_work_;
    plan.part_base = d_part_base_;
    plan.n_work = n_work_;
    plan.chunk = chunk_;
    plan.any_multi = any_multi_;
    plan.any_empty = any_empty_;
    plan.max_len = cfg.max_seq_len;
    plan.fused_heads = fused_heads_;
    plan.fused_chunked = fused_chunked_;
    float *part = nullptr;
    int   *cnt = nullptr;
    if (any_multi_) {
        part = work_->get(detail::attn_workspace_floats(n_work_, num_q_heads_, cfg.head_dim));
        if (detail::fused_merge_enabled()) // only the in-launch merge counts in them
            cnt = work_->counters(detail::attn_counters_ints(n_, cfg.num_heads), stream);
    }
    detail::launch_attn_decode(q, mgr_.layerView(layer_idx, d_slot_), plan, n_, num_q_heads_,
                               cfg.num_heads, cfg.head_dim, scale, out, part, new_k, new_v, stream,
                               inline_ok_ ? inl_.get() : nullptr, true, cnt);
    return Result<void>::ok();
}

// Append and attention in one launch: the workgroup that owns the last chunk
// of each (entry, kv head) writes the new token, then attends over it.
Result<void> DecodeBatch::decode(int layer_idx, const half *q, const half *new_k,
                                 const half *new_v, half *out, float scale, hipStream_t stream) {
    if (!appendable_)
        return Result<void>::err("DecodeBatch: append needs a batch made by prepare()");
    if (new_k == nullptr) return Result<void>::err("new_k is null");
    if (new_v == nullptr) return Result<void>::err("new_v is null");
    return run_attention(layer_idx, q, new_k, new_v, out, scale, stream);
}

Result<void> DecodeBatch::gather(int layer_idx, half *k_out, half *v_out, int s_max,
                                 hipStream_t stream) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (layer_idx < 0 || layer_idx >= cfg.num_layers)
        return Result<void>::err("DecodeBatch: Invalid layer_idx: " + std::to_string(layer_idx));
    if (s_max < 0) return Result<void>::err("DecodeBatch: s_max must be >= 0");
    if (n_ == 0 || s_max == 0) return Result<void>::ok();
    upload_device(stream);
    const KvView v = mgr_.layerView(layer_idx, d_slot_);
    if (k_out)
        detail::launch_kv_gather(v, 0, d_lens_, 0, n_, cfg.num_heads, cfg.head_dim, s_max, k_out, stream);
    if (v_out)
        detail::launch_kv_gather(v, 1, d_lens_, 0, n_, cfg.num_heads, cfg.head_dim, s_max, v_out, stream);
    return Result<void>::ok();
}

Result<void> DecodeBatch::project(int layer_idx, const half *x, int hidden, int group_size,
                                  const int8_t *wk, const half *sk, const int8_t *wv,
                                  const half *sv, const int8_t *wq, const half *sq, half *q_out,
                                  hipStream_t stream, bool packed) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (!appendable_)
        return Result<void>::err("DecodeBatch: project needs a batch made by prepare()");
    if (layer_idx < 0 || layer_idx >= cfg.num_layers)
        return Result<void>::err("DecodeBatch: Invalid layer_idx: " + std::to_string(layer_idx));
    if (hidden <= 0 || group_size <= 0)
        return Result<void>::err("DecodeBatch: hidden and group_size must be positive");
    if (!x || !wk || !sk || !wv || !sv) return Result<void>::err("DecodeBatch: null x or K/V weights");
    const bool with_q = wq || sq || q_out;
    if (with_q && (!wq || !sq || !q_out))
        return Result<void>::err("DecodeBatch: wq, sq and q_out must be all set or all null");
    if (n_ == 0) return Result<void>::ok();
    upload_device(stream);
    const KvView v = mgr_.layerView(layer_idx, d_slot_);
    detail::CacheRows rows;
    rows.seq_row = d_slot_;
    rows.wpos = d_wpos_;
    rows.block_table = v.block_table;
    rows.bt_stride = v.bt_stride;
    rows.log2_blk = v.log2_blk;
    rows.blk_stride = v.blk_stride;
    rows.tok_stride = v.tok_stride;
    const int        row = cfg.num_heads * cfg.head_dim;
    detail::W8A16Seg segs[3];
    int              nseg = 0;
    auto add = [&](const int8_t *w, const half *s, int n, int kind, half *out, int64_t ld) {
        segs[nseg].w = w;
        segs[nseg].s = s;
        segs[nseg].n = n;
        segs[nseg].kind = kind;
        segs[nseg].out = out;
        segs[nseg].ld = ld;
        ++nseg;
    };
    add(wk, sk, row, detail::kEpiCache, const_cast<half *>(v.k_base), 0);
    add(wv, sv, row, detail::kEpiCache, const_cast<half *>(v.v_base), 0);
    if (with_q) add(wq, sq, num_q_heads_ * cfg.head_dim, detail::kEpiDense, q_out, num_q_heads_ * cfg.head_dim);
    float *ws = nullptr;
    if (const size_t f = detail::w8a16_workspace_floats(n_, hidden, group_size, segs, nseg))
        ws = gemm_work_->get(f);
    if (packed && !detail::w8a16_mfma_ok(hidden, group_size, segs, nseg))
        return Result<void>::err("DecodeBatch: packed weights need hidden % 32 == 0 and group_size "
                                 "in {32, 64, 128, 256, 512}");
    detail::launch_w8a16(x, hidden, n_, hidden, group_size, segs, nseg, &rows, ws, stream, packed);
    return Result<void>::ok();
}

// ======================================================================
// PrefillBatch
// ======================================================================

PrefillBatch::PrefillBatch(KVCacheManager &mgr, int max_seqs, int num_q_heads)
    : mgr_(mgr), max_seqs_(max_seqs), num_q_heads_(num_q_heads), meta_(new detail::MetaRing(4)) {}

PrefillBatch::~PrefillBatch() = default;

Result<std::unique_ptr<PrefillBatch>> PrefillBatch::create(KVCacheManager &mgr, int max_seqs,
                                                           int num_q_heads) {
    using R = Result<std::unique_ptr<PrefillBatch>>;
    const KVCacheConfig &cfg = mgr.getConfig();
    if (max_seqs <= 0) return R::err("PrefillBatch: max_seqs must be positive");
    if (num_q_heads <= 0 || num_q_heads % cfg.num_heads != 0)
        return R::err("PrefillBatch: num_q_heads (" + std::to_string(num_q_heads) +
                      ") must be a positive multiple of num_heads (" +
                      std::to_string(cfg.num_heads) + ")");
    if (!detail::prefill_shape_supported(cfg.head_dim, num_q_heads / cfg.num_heads))
        return R::err("PrefillBatch: unsupported head_dim/group (head_dim in {32,64,128,256}, "
                      "num_q_heads/num_heads in {1,2,4,8})");
    return R::ok(std::unique_ptr<PrefillBatch>(new PrefillBatch(mgr, max_seqs, num_q_heads)));
}

Result<void> PrefillBatch::prepare(const int *seq_ids, const int *num_tokens, int n,
                                   hipStream_t stream) {
    // A failing prepare leaves an empty batch: append/attention/prefill and
    // commit are then no-ops, never a replay of the previous step's plan.
    n_ = 0;
    tokens_ = 0;
    n_items_ = 0;
    max_keys_ = 0;
    d_work_ = nullptr;
    uploaded_ = false;
    ids_.clear();
    counts_.clear();
    slots_.clear();
    pos0_.clear();
    work_.clear();
    if (n < 0 || n > max_seqs_)
        return Result<void>::err("PrefillBatch: n=" + std::to_string(n) + " outside [0, " +
                                 std::to_string(max_seqs_) + "]");
    if (n > 0 && (seq_ids == nullptr || num_tokens == nullptr))
        return Result<void>::err("PrefillBatch: seq_ids / num_tokens is null");
    const KVCacheConfig &cfg = mgr_.getConfig();
    std::vector<char>    taken(static_cast<size_t>(cfg.max_batch_size), 0);
    std::vector<int32_t> slots(static_cast<size_t>(n)), ends(static_cast<size_t>(n));
    std::vector<detail::PrefillEntry> entries(static_cast<size_t>(n));
    int64_t total = 0;
    int     max_keys = 0;
    for (int i = 0; i < n; ++i) {
        const int            id = seq_ids[i];
        const SequenceCache *sc = mgr_.sequence(id);
        if (!sc) return Result<void>::err("PrefillBatch: sequence not found: " + std::to_string(id));
        const int slot = mgr_.slotOf(id);
        if (taken[static_cast<size_t>(slot)])
            return Result<void>::err("PrefillBatch: duplicate sequence in batch: " + std::to_string(id));
        taken[static_cast<size_t>(slot)] = 1;
        const int nt = num_tokens[i];
        if (nt <= 0)
            return Result<void>::err("appendKV: num_tokens must be positive: " + std::to_string(nt));
        if (sc->current_len + nt > sc->max_len)
            return Result<void>::err("appendKV: cache overflow. Current: " +
                                     std::to_string(sc->current_len) + ", appending: " +
                                     std::to_string(nt) + ", max: " + std::to_string(sc->max_len));
        slots[static_cast<size_t>(i)] = slot;
        ends[static_cast<size_t>(i)] = sc->current_len + nt;
        max_keys = std::max(max_keys, sc->current_len + nt);
        entries[static_cast<size_t>(i)] = {total * num_q_heads_ * cfg.head_dim, sc->current_len, nt,
                                           slot, static_cast<int32_t>(total)};
        total += nt;
    }
    if (total > INT32_MAX / 2)
        return Result<void>::err("PrefillBatch: too many tokens in one prefill step");
    if (mgr_.isBlockPool()) {
        auto r = mgr_.reserveSlots(slots.data(), ends.data(), n);
        if (r.isErr()) return r;
        mgr_.syncTable(stream);
    }
    waves_ = detail::prefill_waves(entries.data(), n, cfg.head_dim, num_q_heads_ / cfg.num_heads,
                                   cfg.num_heads, detail::device_cus());
    detail::plan_prefill(entries.data(), n, cfg.head_dim, num_q_heads_ / cfg.num_heads, waves_, work_);
    n_items_ = static_cast<int>(work_.size() / detail::kPrefillItemWords);
    slots_ = std::move(slots);
    pos0_.resize(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) pos0_[static_cast<size_t>(i)] = entries[static_cast<size_t>(i)].p0;
    ids_.assign(seq_ids, seq_ids + n);
    counts_.assign(num_tokens, num_tokens + n);
    n_ = n;
    tokens_ = static_cast<int>(total);
    max_keys_ = max_keys;
    return Result<void>::ok();
}

Result<void> PrefillBatch::append(int layer_idx, const half *new_k, const half *new_v,
                                  hipStream_t stream) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (new_k == nullptr) return Result<void>::err("new_k is null");
    if (new_v == nullptr) return Result<void>::err("new_v is null");
    if (layer_idx < 0 || layer_idx >= cfg.num_layers)
        return Result<void>::err("PrefillBatch: Invalid layer_idx: " + std::to_string(layer_idx));
    if (tokens_ == 0) return Result<void>::ok();
    // Ranges (slot, write position, tokens) travel in kernel arguments.
    detail::launch_kv_append_ranges(mgr_.layerView(layer_idx, nullptr), slots_.data(), pos0_.data(),
                                    counts_.data(), n_, cfg.num_heads * cfg.head_dim, new_k, new_v,
                                    stream);
    return Result<void>::ok();
}

void PrefillBatch::upload_device(hipStream_t stream) {
    if (uploaded_) return;
    // [work items (8 words each, the first 32-byte aligned)]
    int32_t *h = static_cast<int32_t *>(meta_->begin(std::max<size_t>(work_.size(), 1) * 4));
    if (!work_.empty()) std::memcpy(h, work_.data(), work_.size() * 4);
    d_work_ = static_cast<const int32_t *>(meta_->commit(stream));
    uploaded_ = true;
}

Result<void> PrefillBatch::attention(int layer_idx, const half *q, half *out, float scale,
                                     hipStream_t stream) {
    return launch(layer_idx, q, nullptr, nullptr, out, scale, stream);
}

Result<void> PrefillBatch::prefill(int layer_idx, const half *q, const half *new_k,
                                   const half *new_v, half *out, float scale, hipStream_t stream) {
    if (new_k == nullptr) return Result<void>::err("new_k is null");
    if (new_v == nullptr) return Result<void>::err("new_v is null");
    return launch(layer_idx, q, new_k, new_v, out, scale, stream);
}

Result<void> PrefillBatch::launch(int layer_idx, const half *q, const half *new_k, const half *new_v,
                                  half *out, float scale, hipStream_t stream) {
    const KVCacheConfig &cfg = mgr_.getConfig();
    if (layer_idx < 0 || layer_idx >= cfg.num_layers)
        return Result<void>::err("PrefillBatch: Invalid layer_idx: " + std::to_string(layer_idx));
    if (q == nullptr || out == nullptr) return Result<void>::err("PrefillBatch: q/out is null");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
         reinterpret_cast<uintptr_t>(new_k) | reinterpret_cast<uintptr_t>(new_v)) & 15u)
        return Result<void>::err("PrefillBatch: q, out, new_k and new_v must be 16-byte aligned");
    if (n_items_ == 0) return Result<void>::ok();
    upload_device(stream);
    detail::PrefillLaunch p;
    p.q = q;
    p.out = out;
    p.q_tok_stride = static_cast<int64_t>(num_q_heads_) * cfg.head_dim;
    p.q_head_stride = cfg.head_dim;
    p.work = d_work_;
    p.n_items = n_items_;
    p.waves = waves_;
    p.max_keys = max_keys_;
    p.new_k = new_k;
    p.new_v = new_v;
    detail::launch_attn_prefill(p, mgr_.layerView(layer_idx, nullptr), num_q_heads_, cfg.num_heads,
                                cfg.head_dim, scale, stream);
    return Result<void>::ok();
}

// InferenceEngine::prefill's commit (inference_engine.cpp:272):
// advanceSeqLen(seq, prompt tokens) once after all layers.
Result<void> PrefillBatch::commit() {
    for (size_t i = 0; i < ids_.size(); ++i) {
        auto r = mgr_.advanceSeqLen(ids_[i], counts_[i]);
        if (r.isErr()) return r;
    }
    return Result<void>::ok();
}

} // namespace tiny_llm
