// Per-sequence state (semantics of engine/src/sequence.cpp:6-63) and the
// block hash (engine/include/memforge/prefix_cache.hpp:21-51).
#include "engine.hpp"

namespace mfe {

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

uint64_t hash_block(uint64_t parent_hash, const TokenId* tokens, size_t n) {
    constexpr uint64_t kFnvOffset = 0xCBF29CE484222325ULL;
    constexpr uint64_t kFnvPrime = 0x100000001B3ULL;
    uint64_t h = splitmix64(parent_hash ^ kFnvOffset);
    for (size_t i = 0; i < n; ++i) h = (h ^ static_cast<uint32_t>(tokens[i])) * kFnvPrime;
    const uint64_t out = splitmix64(h);
    return out ? out : 1;  // 0 is reserved for "not registered"
}

Sequence::Sequence(SequenceId id, std::vector<TokenId> prompt, size_t max_new_tokens, size_t block_size)
    : id_(id), prompt_(std::move(prompt)), max_new_tokens_(max_new_tokens), block_size_(block_size) {
    output_.reserve(max_new_tokens_);
}

std::vector<TokenId> Sequence::get_all_tokens() const {
    std::vector<TokenId> all(prompt_);
    all.insert(all.end(), output_.begin(), output_.end());
    return all;
}

void Sequence::set_block(size_t logical, BlockId b) {
    if (logical < table_.size()) table_[logical] = b;
}

void Sequence::append_token(TokenId t) {
    output_.push_back(t);
    if (output_.size() >= max_new_tokens_) status_ = SequenceStatus::FINISHED;
}

}  // namespace mfe
