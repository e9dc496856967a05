// Host bookkeeping of a block-granular KV pool (no HIP calls).
#include "block_allocator.h"

#include <stdexcept>

namespace tiny_llm {
namespace detail {

BlockAllocator::BlockAllocator(int rows, int blocks_per_row, int num_blocks)
    : rows_(rows), bpr_(blocks_per_row), num_blocks_(num_blocks) {
    if (rows <= 0 || blocks_per_row <= 0 || num_blocks <= 0)
        throw std::invalid_argument("BlockAllocator: rows, blocks_per_row and num_blocks must be positive");
    table_.assign(static_cast<size_t>(rows) * static_cast<size_t>(blocks_per_row), num_blocks);
    mapped_.assign(static_cast<size_t>(rows), 0);
    is_dirty_.assign(table_.size(), 0);
    // Stack order hands out block 0 first, then 1, 2, ...
    free_.reserve(static_cast<size_t>(num_blocks));
    for (int b = num_blocks - 1; b >= 0; --b) free_.push_back(b);
}

void BlockAllocator::touch(size_t idx) {
    if (!is_dirty_[idx]) {
        is_dirty_[idx] = 1;
        dirty_.push_back(static_cast<int32_t>(idx));
    }
}

bool BlockAllocator::ensure(int row, int blocks) {
    if (row < 0 || row >= rows_ || blocks > bpr_) return false;
    const int have = mapped_[static_cast<size_t>(row)];
    if (blocks <= have) return true;
    if (blocks - have > freeBlocks()) return false;
    const size_t base = static_cast<size_t>(row) * static_cast<size_t>(bpr_);
    for (int j = have; j < blocks; ++j) {
        table_[base + static_cast<size_t>(j)] = free_.back();
        free_.pop_back();
        touch(base + static_cast<size_t>(j));
    }
    mapped_[static_cast<size_t>(row)] = blocks;
    return true;
}

int64_t BlockAllocator::shortfall(const int *rows, const int *blocks, int n) const {
    int64_t need = 0;
    for (int i = 0; i < n; ++i) {
        const int have = mapped_[static_cast<size_t>(rows[i])];
        if (blocks[i] > have) need += blocks[i] - have;
    }
    return need - freeBlocks();
}

void BlockAllocator::release(int row) {
    if (row < 0 || row >= rows_) return;
    const size_t base = static_cast<size_t>(row) * static_cast<size_t>(bpr_);
    // Push in reverse so the row's first block is handed out first again.
    for (int j = mapped_[static_cast<size_t>(row)] - 1; j >= 0; --j) {
        free_.push_back(table_[base + static_cast<size_t>(j)]);
        table_[base + static_cast<size_t>(j)] = num_blocks_;
        touch(base + static_cast<size_t>(j));
    }
    mapped_[static_cast<size_t>(row)] = 0;
}

std::vector<std::pair<int32_t, int32_t>> BlockAllocator::takeUpdates() {
    std::vector<std::pair<int32_t, int32_t>> out;
    out.reserve(dirty_.size());
    for (const int32_t idx : dirty_) {
        out.emplace_back(idx, table_[static_cast<size_t>(idx)]);
        is_dirty_[static_cast<size_t>(idx)] = 0;
    }
    dirty_.clear();
    return out;
}

} // namespace detail
} // namespace tiny_llm
