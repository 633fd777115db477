// Chained-hash prefix cache (semantics of engine/src/prefix_cache.cpp:5-166).
#include <algorithm>

#include "engine.hpp"

namespace mfe {

PrefixCache::PrefixCache(std::shared_ptr<BlockAllocator> allocator, size_t block_size)
    : alloc_(std::move(allocator)), block_size_(block_size ? block_size : kDefaultBlockSize) {}

// Leading full blocks eligible for sharing; a prompt ending exactly on a
// block boundary keeps its last block private so the next write has a home.
size_t PrefixCache::shareable(size_t num_tokens) const {
    size_t full = num_tokens / block_size_;
    if (full > 0 && num_tokens % block_size_ == 0) --full;
    return full;
}

std::vector<BlockId> PrefixCache::acquire_shared_prefix(const std::vector<TokenId>& tokens) {
    std::lock_guard<std::mutex> g(mu_);
    std::vector<BlockId> got;
    const size_t n = shareable(tokens.size());
    uint64_t parent = 0;
    for (size_t i = 0; i < n; ++i) {
        const TokenId* blk = tokens.data() + i * block_size_;
        const uint64_t h = hash_block(parent, blk, block_size_);
        auto it = by_hash_.find(h);
        if (it == by_hash_.end() || it->second.tokens.size() != block_size_ ||
            !std::equal(it->second.tokens.begin(), it->second.tokens.end(), blk)) {
            ++misses_;
            break;
        }
        if (!alloc_->add_ref(it->second.block)) {
            // stale entry: its block went back to the pool
            ++misses_;
            by_block_.erase(it->second.block);
            by_hash_.erase(it);
            break;
        }
        got.push_back(it->second.block);
        ++hits_;
        parent = h;
    }
    return got;
}

void PrefixCache::release_acquired(const std::vector<BlockId>& ids) {
    if (ids.empty()) return;
    const std::vector<BlockId> freed = alloc_->release(ids);
    if (!freed.empty()) evict(freed);
}

size_t PrefixCache::register_full_blocks(const std::vector<TokenId>& tokens, const std::vector<BlockId>& table) {
    std::lock_guard<std::mutex> g(mu_);
    const size_t n = std::min(shareable(tokens.size()), table.size());
    size_t added = 0;
    uint64_t parent = 0;
    for (size_t i = 0; i < n; ++i) {
        const TokenId* blk = tokens.data() + i * block_size_;
        const uint64_t h = hash_block(parent, blk, block_size_);
        parent = h;
        const BlockId id = table[i];
        if (id < 0) break;
        if (by_hash_.count(h) || by_block_.count(id)) continue;  // first registration wins
        by_hash_.emplace(h, Entry{id, std::vector<TokenId>(blk, blk + block_size_)});
        by_block_.emplace(id, h);
        ++added;
    }
    return added;
}

void PrefixCache::evict(const std::vector<BlockId>& released) {
    std::lock_guard<std::mutex> g(mu_);
    for (BlockId id : released) {
        auto it = by_block_.find(id);
        if (it == by_block_.end()) continue;
        by_hash_.erase(it->second);
        by_block_.erase(it);
    }
}

void PrefixCache::clear() {
    std::lock_guard<std::mutex> g(mu_);
    by_hash_.clear();
    by_block_.clear();
    hits_ = misses_ = 0;
}

uint64_t PrefixCache::first_block_hash(const std::vector<TokenId>& tokens) const {
    if (shareable(tokens.size()) == 0) return 0;
    return hash_block(0, tokens.data(), block_size_);
}

size_t PrefixCache::num_cached_blocks() const {
    std::lock_guard<std::mutex> g(mu_);
    return by_hash_.size();
}

uint64_t PrefixCache::num_hits() const {
    std::lock_guard<std::mutex> g(mu_);
    return hits_;
}

uint64_t PrefixCache::num_misses() const {
    std::lock_guard<std::mutex> g(mu_);
    return misses_;
}

double PrefixCache::hit_rate() const {
    std::lock_guard<std::mutex> g(mu_);
    const uint64_t total = hits_ + misses_;
    return total ? static_cast<double>(hits_) / static_cast<double>(total) : 0.0;
}

}  // namespace mfe
