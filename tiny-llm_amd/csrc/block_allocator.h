// Host bookkeeping of a block-granular KV pool.
//
// The pool holds num_blocks physical blocks; one block stores block_tokens
// consecutive tokens of one sequence for every layer, K and V.  A sequence
// (one row of the block table) is handed blocks as it grows and gives them
// all back when it is released, so memory follows the tokens actually held
// instead of a full max_seq_len reservation per sequence (the slot policy of
// src/kv_cache.cpp:91-119 in the reference).
//
// Entry j of a row names the physical block of the row's tokens
// [j*block_tokens, (j+1)*block_tokens).  Unmapped entries name the spare
// block (id num_blocks), which is never handed out, so a read past a row's
// mapped tokens stays inside the pool.  Entries changed since the last
// takeUpdates() are kept as a dirty list, so the device copy of the table
// is patched with only what changed.
//
// No HIP here: this class is plain C++ and is unit-tested on the host.
#pragma once

#include <cstddef>
#include <cstdint>
#include <utility>
#include <vector>

namespace tiny_llm {
namespace detail {

class BlockAllocator {
  public:
    BlockAllocator(int rows, int blocks_per_row, int num_blocks);

    int rows() const noexcept { return rows_; }
    int blocksPerRow() const noexcept { return bpr_; }
    int numBlocks() const noexcept { return num_blocks_; }
    int spare() const noexcept { return num_blocks_; }
    int freeBlocks() const noexcept { return static_cast<int>(free_.size()); }
    int usedBlocks() const noexcept { return num_blocks_ - freeBlocks(); }
    int mapped(int row) const noexcept { return mapped_[static_cast<size_t>(row)]; }

    // Map blocks so that `row` covers its first `blocks` entries.  All or
    // nothing: false, with no change, when the free list is too short or
    // `blocks` exceeds the row length.
    bool ensure(int row, int blocks);
    // Extra blocks the rows would need to cover the given block counts
    // (rows[i] -> blocks[i]); used to check a whole batch before mapping any.
    int64_t shortfall(const int *rows, const int *blocks, int n) const;
    // Return every block of `row` to the free list; its entries go back to
    // the spare block.
    void release(int row);

    // Host mirror of the table, [rows][blocks_per_row].
    const std::vector<int32_t> &table() const noexcept { return table_; }
    // (entry index, new value) of every entry changed since the last call.
    std::vector<std::pair<int32_t, int32_t>> takeUpdates();
    bool hasUpdates() const noexcept { return !dirty_.empty(); }

  private:
    void touch(size_t idx);

    int                  rows_, bpr_, num_blocks_;
    std::vector<int32_t> table_;
    std::vector<int32_t> mapped_;
    std::vector<int32_t> free_;   // stack; back() is handed out next
    std::vector<int32_t> dirty_;  // entry indices
    std::vector<char>    is_dirty_;
};

} // namespace detail
} // namespace tiny_llm
