// Host engine of the continuous-batching data path: the paged block
// allocator, per-sequence state, the iteration-level scheduler and the
// chained-hash prefix cache. Host-only C++17; it hands block tables to the
// device side through the ragged-pack entry point.
//
// The observable behaviour -- which block ids are handed out in which order,
// when a sequence is preempted, admitted, chunked or aborted -- matches the
// reference engine (engine/include/memforge/*.hpp, engine/src/*.cpp) exactly,
// because the block tables it produces are compared bit for bit.
#pragma once

#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace mfe {

using SequenceId = uint64_t;
using TokenId = int32_t;
using BlockId = int32_t;

constexpr BlockId kInvalidBlock = -1;
constexpr size_t kDefaultBlockSize = 16;

// engine/include/memforge/types.hpp:20-27
enum class SequenceStatus { WAITING, RUNNING, SWAPPED, FINISHED, ABORTED };

// One running sequence's share of a scheduler step (types.hpp:45-65).
struct SequenceStepInfo {
    SequenceId seq_id = 0;
    std::vector<BlockId> block_table;
    size_t prompt_length = 0;
    size_t output_length = 0;
    size_t total_length = 0;
    SequenceStatus status = SequenceStatus::WAITING;
    bool is_prefill = false;
    size_t num_cached_tokens = 0;
    size_t prefill_chunk_end = 0;
};

// types.hpp:70-79
struct SchedulerStepResult {
    std::vector<SequenceStepInfo> running_sequences;
    std::vector<SequenceId> finished_sequence_ids;
    std::vector<SequenceId> preempted_sequence_ids;
    std::vector<SequenceId> aborted_sequence_ids;
    size_t num_free_blocks = 0;
    size_t total_blocks = 0;
    size_t num_waiting = 0;
    double memory_utilization_ratio = 0.0;
};

// ----------------------------------------------------------------- hashing
// splitmix64 finaliser and the chained FNV-1a block hash
// (engine/include/memforge/prefix_cache.hpp:21-51). The constants are the
// published ones of both algorithms; they have to be these for the hashes to
// agree with the reference's.
uint64_t splitmix64(uint64_t x);
uint64_t hash_block(uint64_t parent_hash, const TokenId* tokens, size_t n);

// ---------------------------------------------------------------- Sequence
class Sequence {
public:
    Sequence(SequenceId id, std::vector<TokenId> prompt, size_t max_new_tokens,
             size_t block_size = kDefaultBlockSize);

    SequenceId get_id() const { return id_; }
    SequenceStatus get_status() const { return status_; }
    void set_status(SequenceStatus s) { status_ = s; }

    const std::vector<TokenId>& get_prompt_tokens() const { return prompt_; }
    const std::vector<TokenId>& get_output_tokens() const { return output_; }
    std::vector<TokenId> get_all_tokens() const;
    size_t get_prompt_len() const { return prompt_.size(); }
    size_t get_output_len() const { return output_.size(); }
    size_t get_total_len() const { return prompt_.size() + output_.size(); }
    size_t get_max_new_tokens() const { return max_new_tokens_; }
    size_t get_block_size() const { return block_size_; }

    const std::vector<BlockId>& get_block_table() const { return table_; }
    void add_block(BlockId b) { table_.push_back(b); }
    void set_block(size_t logical, BlockId b);
    void clear_blocks() { table_.clear(); }
    size_t get_num_required_blocks() const { return blocks_for(get_total_len()); }
    size_t get_num_required_blocks_with_lookahead(size_t lookahead) const {
        return blocks_for(get_total_len() + lookahead);
    }
    size_t get_num_allocated_blocks() const { return table_.size(); }

    void append_token(TokenId t);
    bool is_finished() const {
        return status_ == SequenceStatus::FINISHED || status_ == SequenceStatus::ABORTED;
    }
    void finish() { status_ = SequenceStatus::FINISHED; }

    bool has_completed_prefill() const { return prefill_done_; }
    void mark_prefill_completed() { prefill_done_ = true; }
    void reset_prefill() {
        prefill_done_ = false;
        cached_ = 0;
    }
    size_t get_num_cached_tokens() const { return cached_; }
    void set_num_cached_tokens(size_t n) { cached_ = n; }
    size_t get_num_unprefilled_tokens() const {
        const size_t total = get_total_len();
        return cached_ >= total ? 0 : total - cached_;
    }

private:
    size_t blocks_for(size_t tokens) const {
        return tokens == 0 ? 0 : (tokens + block_size_ - 1) / block_size_;
    }

    SequenceId id_;
    std::vector<TokenId> prompt_;
    std::vector<TokenId> output_;
    std::vector<BlockId> table_;
    size_t max_new_tokens_;
    size_t block_size_;
    SequenceStatus status_ = SequenceStatus::WAITING;
    bool prefill_done_ = false;
    size_t cached_ = 0;
};
using SequencePtr = std::shared_ptr<Sequence>;

// ---------------------------------------------------------- BlockAllocator
// Reference-counted physical blocks with a FIFO free list: block ids leave
// from the front in the order they were freed (initially 0..N-1) and return
// to the back. The free list is a fixed ring of N slots, which can never
// overflow because at most N blocks are ever free.
class BlockAllocator {
public:
    explicit BlockAllocator(size_t total_blocks, size_t block_size = kDefaultBlockSize);
    BlockAllocator(const BlockAllocator&) = delete;
    BlockAllocator& operator=(const BlockAllocator&) = delete;

    bool can_allocate(size_t n) const;
    BlockId allocate();
    std::vector<BlockId> allocate_blocks(size_t n);  // throws std::runtime_error
    void free(BlockId b);
    void free_blocks(const std::vector<BlockId>& ids);
    std::vector<BlockId> release(const std::vector<BlockId>& ids);
    std::vector<BlockId> free_sequence(Sequence& seq);
    bool ensure_capacity(Sequence& seq);
    bool ensure_capacity_with_lookahead(Sequence& seq, size_t lookahead);
    bool add_ref(BlockId b);
    std::optional<std::pair<BlockId, BlockId>> prepare_write(Sequence& seq, size_t logical);
    int get_ref_count(BlockId b) const;
    size_t get_num_shared_blocks() const;
    size_t get_num_blocks_saved() const;
    size_t get_num_free_blocks() const;
    size_t get_num_allocated_blocks() const;
    size_t get_total_blocks() const { return total_; }
    size_t get_block_size() const { return block_size_; }
    double get_utilization_ratio() const;
    void reset();

private:
    bool in_range(BlockId b) const { return b >= 0 && static_cast<size_t>(b) < total_; }
    BlockId pop_free_locked();
    void push_free_locked(BlockId b);
    bool drop_ref_locked(BlockId b);
    bool grow_to(Sequence& seq, size_t needed);

    size_t total_;
    size_t block_size_;
    std::vector<int32_t> refs_;  // 0 <=> free
    std::vector<BlockId> ring_;  // free list, FIFO
    size_t head_ = 0;            // next block to hand out
    size_t count_ = 0;           // blocks currently free
    mutable std::mutex mu_;
};

// -------------------------------------------------------------- PrefixCache
class PrefixCache {
public:
    PrefixCache(std::shared_ptr<BlockAllocator> allocator, size_t block_size);
    PrefixCache(const PrefixCache&) = delete;
    PrefixCache& operator=(const PrefixCache&) = delete;

    std::vector<BlockId> acquire_shared_prefix(const std::vector<TokenId>& tokens);
    void release_acquired(const std::vector<BlockId>& ids);
    size_t register_full_blocks(const std::vector<TokenId>& tokens, const std::vector<BlockId>& table);
    void evict(const std::vector<BlockId>& released);
    void clear();
    uint64_t first_block_hash(const std::vector<TokenId>& tokens) const;
    size_t num_cached_blocks() const;
    uint64_t num_hits() const;
    uint64_t num_misses() const;
    double hit_rate() const;
    size_t get_block_size() const { return block_size_; }

private:
    struct Entry {
        BlockId block;
        std::vector<TokenId> tokens;
    };
    size_t shareable(size_t num_tokens) const;

    std::shared_ptr<BlockAllocator> alloc_;
    size_t block_size_;
    std::unordered_map<uint64_t, Entry> by_hash_;
    std::unordered_map<BlockId, uint64_t> by_block_;
    uint64_t hits_ = 0;
    uint64_t misses_ = 0;
    mutable std::mutex mu_;
};

// ---------------------------------------------------------------- Scheduler
// Lock order: Scheduler -> PrefixCache -> BlockAllocator.
class Scheduler {
public:
    Scheduler(std::shared_ptr<BlockAllocator> allocator, size_t max_num_seqs = 256,
              std::shared_ptr<PrefixCache> prefix_cache = nullptr,
              size_t max_prefill_tokens_per_step = 0, size_t lookahead_slots = 0);

    SequencePtr add_sequence(SequenceId id, const std::vector<TokenId>& prompt, size_t max_new_tokens);
    SchedulerStepResult step();
    void update_sequence(SequenceId id, TokenId token, bool finished);
    bool abort_sequence(SequenceId id);
    size_t get_num_waiting() const;
    size_t get_num_running() const;
    bool has_unfinished_sequences() const;
    SequencePtr get_sequence(SequenceId id);
    std::shared_ptr<BlockAllocator> get_allocator() const { return alloc_; }
    std::shared_ptr<PrefixCache> get_prefix_cache() const { return prefix_; }
    bool prefix_sharing_enabled() const { return prefix_ != nullptr; }
    size_t get_max_prefill_tokens_per_step() const { return prefill_budget_; }
    void set_max_prefill_tokens_per_step(size_t n) { prefill_budget_ = n; }
    bool chunked_prefill_enabled() const { return prefill_budget_ > 0; }
    size_t get_lookahead_slots() const { return lookahead_; }
    void set_lookahead_slots(size_t n) { lookahead_ = n; }

private:
    void release_blocks_locked(Sequence& seq);
    void retire_running_locked(SchedulerStepResult& out);
    void admit_waiting_locked(SchedulerStepResult& out);
    void describe_running_locked(SchedulerStepResult& out);

    std::shared_ptr<BlockAllocator> alloc_;
    std::shared_ptr<PrefixCache> prefix_;
    size_t max_num_seqs_;
    size_t prefill_budget_;
    size_t lookahead_;
    std::deque<SequencePtr> waiting_;  // front = next to admit
    std::vector<SequencePtr> running_;
    std::unordered_map<SequenceId, SequencePtr> all_;
    mutable std::mutex mu_;
};

}  // namespace mfe
