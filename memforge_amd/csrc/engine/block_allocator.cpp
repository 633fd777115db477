// Paged block allocator (semantics of engine/src/block_allocator.cpp:6-257).
#include <stdexcept>

#include "engine.hpp"

namespace mfe {

BlockAllocator::BlockAllocator(size_t total_blocks, size_t block_size)
    : total_(total_blocks), block_size_(block_size), refs_(total_blocks, 0), ring_(total_blocks) {
    for (size_t i = 0; i < total_; ++i) ring_[i] = static_cast<BlockId>(i);
    head_ = 0;
    count_ = total_;
}

BlockId BlockAllocator::pop_free_locked() {
    const BlockId b = ring_[head_];
    head_ = (head_ + 1 == total_) ? 0 : head_ + 1;
    --count_;
    refs_[b] = 1;
    return b;
}

void BlockAllocator::push_free_locked(BlockId b) {
    size_t tail = head_ + count_;
    if (tail >= total_) tail -= total_;
    ring_[tail] = b;
    ++count_;
}

// Drops one reference; true when the block went back on the free list.
bool BlockAllocator::drop_ref_locked(BlockId b) {
    if (!in_range(b) || refs_[b] <= 0) return false;
    if (--refs_[b] > 0) return false;
    push_free_locked(b);
    return true;
}

bool BlockAllocator::can_allocate(size_t n) const {
    std::lock_guard<std::mutex> g(mu_);
    return count_ >= n;
}

BlockId BlockAllocator::allocate() {
    std::lock_guard<std::mutex> g(mu_);
    return count_ ? pop_free_locked() : kInvalidBlock;
}

std::vector<BlockId> BlockAllocator::allocate_blocks(size_t n) {
    std::lock_guard<std::mutex> g(mu_);
    if (count_ < n) {
        throw std::runtime_error("Out of memory in BlockAllocator: cannot allocate " + std::to_string(n) +
                                 " blocks. Free: " + std::to_string(count_));
    }
    std::vector<BlockId> out;
    out.reserve(n);
    while (out.size() < n) out.push_back(pop_free_locked());
    return out;
}

void BlockAllocator::free(BlockId b) {
    std::lock_guard<std::mutex> g(mu_);
    drop_ref_locked(b);
}

void BlockAllocator::free_blocks(const std::vector<BlockId>& ids) {
    std::lock_guard<std::mutex> g(mu_);
    for (BlockId b : ids) drop_ref_locked(b);
}

std::vector<BlockId> BlockAllocator::release(const std::vector<BlockId>& ids) {
    std::lock_guard<std::mutex> g(mu_);
    std::vector<BlockId> freed;
    for (BlockId b : ids)
        if (drop_ref_locked(b)) freed.push_back(b);
    return freed;
}

std::vector<BlockId> BlockAllocator::free_sequence(Sequence& seq) {
    std::vector<BlockId> freed = release(seq.get_block_table());
    seq.clear_blocks();
    return freed;
}

// All-or-nothing growth of a sequence's table to `needed` blocks.
bool BlockAllocator::grow_to(Sequence& seq, size_t needed) {
    const size_t have = seq.get_num_allocated_blocks();
    if (needed <= have) return true;
    if (!can_allocate(needed - have)) return false;
    for (BlockId b : allocate_blocks(needed - have)) seq.add_block(b);
    return true;
}

bool BlockAllocator::ensure_capacity(Sequence& seq) { return grow_to(seq, seq.get_num_required_blocks()); }

bool BlockAllocator::ensure_capacity_with_lookahead(Sequence& seq, size_t lookahead) {
    return grow_to(seq, seq.get_num_required_blocks_with_lookahead(lookahead));
}

bool BlockAllocator::add_ref(BlockId b) {
    std::lock_guard<std::mutex> g(mu_);
    if (!in_range(b) || refs_[b] <= 0) return false;
    ++refs_[b];
    return true;
}

std::optional<std::pair<BlockId, BlockId>> BlockAllocator::prepare_write(Sequence& seq, size_t logical) {
    std::lock_guard<std::mutex> g(mu_);
    const std::vector<BlockId>& table = seq.get_block_table();
    if (logical >= table.size()) return std::nullopt;
    const BlockId old = table[logical];
    if (!in_range(old) || refs_[old] <= 1) return std::nullopt;  // private already
    if (count_ == 0) return std::nullopt;                          // nowhere to copy to
    const BlockId fresh = pop_free_locked();
    seq.set_block(logical, fresh);
    --refs_[old];  // was > 1, so the shared block stays allocated
    return std::make_pair(old, fresh);
}

int BlockAllocator::get_ref_count(BlockId b) const {
    std::lock_guard<std::mutex> g(mu_);
    return in_range(b) ? refs_[b] : 0;
}

size_t BlockAllocator::get_num_shared_blocks() const {
    std::lock_guard<std::mutex> g(mu_);
    size_t n = 0;
    for (int32_t r : refs_) n += r > 1;
    return n;
}

size_t BlockAllocator::get_num_blocks_saved() const {
    std::lock_guard<std::mutex> g(mu_);
    size_t saved = 0;
    for (int32_t r : refs_)
        if (r > 1) saved += static_cast<size_t>(r - 1);
    return saved;
}

size_t BlockAllocator::get_num_free_blocks() const {
    std::lock_guard<std::mutex> g(mu_);
    return count_;
}

size_t BlockAllocator::get_num_allocated_blocks() const {
    std::lock_guard<std::mutex> g(mu_);
    return total_ - count_;
}

double BlockAllocator::get_utilization_ratio() const {
    std::lock_guard<std::mutex> g(mu_);
    return total_ ? static_cast<double>(total_ - count_) / static_cast<double>(total_) : 0.0;
}

void BlockAllocator::reset() {
    std::lock_guard<std::mutex> g(mu_);
    for (size_t i = 0; i < total_; ++i) {
        refs_[i] = 0;
        ring_[i] = static_cast<BlockId>(i);
    }
    head_ = 0;
    count_ = total_;
}

}  // namespace mfe
