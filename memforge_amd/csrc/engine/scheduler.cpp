// Iteration-level scheduler (semantics of engine/src/scheduler.cpp:7-273).
//
// One step runs three phases in a fixed order, because the order decides
// which block ids every sequence ends up with:
//   1. retire/grow: finished sequences release their blocks; every other
//      running sequence grows its table for this step's writes (one token, or
//      the lookahead reservation) or is preempted by recomputation;
//   2. admit: waiting sequences join FIFO while slots and blocks last, sharing
//      cached prefix blocks first;
//   3. describe: every running sequence's table and this step's prefill chunk,
//      charged against the shared per-step prefill budget.
#include <algorithm>
#include <unordered_set>

#include "engine.hpp"

namespace mfe {

Scheduler::Scheduler(std::shared_ptr<BlockAllocator> allocator, size_t max_num_seqs,
                     std::shared_ptr<PrefixCache> prefix_cache, size_t max_prefill_tokens_per_step,
                     size_t lookahead_slots)
    : alloc_(std::move(allocator)),
      prefix_(std::move(prefix_cache)),
      max_num_seqs_(max_num_seqs),
      prefill_budget_(max_prefill_tokens_per_step),
      lookahead_(lookahead_slots) {}

void Scheduler::release_blocks_locked(Sequence& seq) {
    const std::vector<BlockId> freed = alloc_->free_sequence(seq);
    // a block back on the free list must stop being findable by its old hash
    if (prefix_ && !freed.empty()) prefix_->evict(freed);
}

SequencePtr Scheduler::add_sequence(SequenceId id, const std::vector<TokenId>& prompt, size_t max_new_tokens) {
    std::lock_guard<std::mutex> g(mu_);
    auto seq = std::make_shared<Sequence>(id, prompt, max_new_tokens, alloc_->get_block_size());
    waiting_.push_back(seq);
    all_[id] = seq;
    return seq;
}

void Scheduler::retire_running_locked(SchedulerStepResult& out) {
    std::vector<SequencePtr> kept, preempted;
    kept.reserve(running_.size());
    for (const SequencePtr& seq : running_) {
        if (seq->is_finished()) {
            release_blocks_locked(*seq);
            out.finished_sequence_ids.push_back(seq->get_id());
            continue;
        }
        const bool room = lookahead_ ? alloc_->ensure_capacity_with_lookahead(*seq, lookahead_)
                                     : alloc_->ensure_capacity(*seq);
        if (room) {
            kept.push_back(seq);
            continue;
        }
        // Preempt by recomputation: give the blocks back, keep the tokens,
        // and requeue ahead of never-started requests.
        release_blocks_locked(*seq);
        seq->reset_prefill();
        seq->set_status(SequenceStatus::WAITING);
        preempted.push_back(seq);
        out.preempted_sequence_ids.push_back(seq->get_id());
    }
    running_ = std::move(kept);
    waiting_.insert(waiting_.begin(), preempted.begin(), preempted.end());
}

void Scheduler::admit_waiting_locked(SchedulerStepResult& out) {
    // First-block hashes of cache-missing prompts admitted this step: an
    // identical prompt behind one of them waits a step and then shares its
    // blocks instead of prefilling a second copy.
    std::unordered_set<uint64_t> fresh_prefixes;
    const size_t bs = alloc_->get_block_size();
    while (!waiting_.empty() && running_.size() < max_num_seqs_) {
        SequencePtr seq = waiting_.front();
        const size_t needed = seq->get_num_required_blocks();
        if (needed > alloc_->get_total_blocks()) {
            // can never fit: abort rather than block the queue
            waiting_.pop_front();
            seq->set_status(SequenceStatus::ABORTED);
            out.aborted_sequence_ids.push_back(seq->get_id());
            continue;
        }
        std::vector<BlockId> shared;
        if (prefix_) {
            const std::vector<TokenId> tokens = seq->get_all_tokens();
            shared = prefix_->acquire_shared_prefix(tokens);
            if (shared.empty()) {
                const uint64_t first = prefix_->first_block_hash(tokens);
                if (first != 0) {
                    if (fresh_prefixes.count(first)) break;  // FIFO: stop, do not skip
                    fresh_prefixes.insert(first);
                }
            }
        }
        const size_t fresh = needed > shared.size() ? needed - shared.size() : 0;
        if (!alloc_->can_allocate(fresh)) {
            if (prefix_ && !shared.empty()) prefix_->release_acquired(shared);
            break;
        }
        waiting_.pop_front();
        for (BlockId b : shared) seq->add_block(b);
        if (fresh)
            for (BlockId b : alloc_->allocate_blocks(fresh)) seq->add_block(b);
        seq->set_num_cached_tokens(shared.size() * bs);
        seq->set_status(SequenceStatus::RUNNING);
        running_.push_back(seq);
    }
}

void Scheduler::describe_running_locked(SchedulerStepResult& out) {
    size_t budget = prefill_budget_;
    const bool chunked = prefill_budget_ > 0;
    out.running_sequences.reserve(running_.size());
    for (const SequencePtr& seq : running_) {
        SequenceStepInfo info;
        info.seq_id = seq->get_id();
        info.block_table = seq->get_block_table();
        info.prompt_length = seq->get_prompt_len();
        info.output_length = seq->get_output_len();
        info.total_length = seq->get_total_len();
        info.status = seq->get_status();
        info.is_prefill = !seq->has_completed_prefill();
        info.num_cached_tokens = seq->get_num_cached_tokens();
        info.prefill_chunk_end = info.total_length;
        if (info.is_prefill) {
            const size_t start = info.num_cached_tokens;
            size_t chunk = start >= info.total_length ? 0 : info.total_length - start;
            if (chunked) {
                chunk = std::min(chunk, budget);
                budget -= chunk;
            }
            info.prefill_chunk_end = start + chunk;
            seq->set_num_cached_tokens(info.prefill_chunk_end);
            if (info.prefill_chunk_end >= info.total_length) seq->mark_prefill_completed();
        }
        out.running_sequences.push_back(std::move(info));
    }
}

SchedulerStepResult Scheduler::step() {
    std::lock_guard<std::mutex> g(mu_);
    SchedulerStepResult out;
    retire_running_locked(out);
    admit_waiting_locked(out);
    describe_running_locked(out);
    out.num_free_blocks = alloc_->get_num_free_blocks();
    out.total_blocks = alloc_->get_total_blocks();
    out.num_waiting = waiting_.size();
    out.memory_utilization_ratio = alloc_->get_utilization_ratio();
    return out;
}

void Scheduler::update_sequence(SequenceId id, TokenId token, bool finished) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = all_.find(id);
    if (it == all_.end()) return;
    it->second->append_token(token);
    if (finished) it->second->finish();
}

bool Scheduler::abort_sequence(SequenceId id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = all_.find(id);
    if (it == all_.end()) return false;
    Sequence& seq = *it->second;
    seq.set_status(SequenceStatus::ABORTED);
    release_blocks_locked(seq);
    // A running sequence stays in the running list until the next step
    // reports it finished; a waiting one simply leaves the queue.
    for (auto w = waiting_.begin(); w != waiting_.end(); ++w) {
        if ((*w)->get_id() == id) {
            waiting_.erase(w);
            break;
        }
    }
    return true;
}

size_t Scheduler::get_num_waiting() const {
    std::lock_guard<std::mutex> g(mu_);
    return waiting_.size();
}

size_t Scheduler::get_num_running() const {
    std::lock_guard<std::mutex> g(mu_);
    return running_.size();
}

bool Scheduler::has_unfinished_sequences() const {
    std::lock_guard<std::mutex> g(mu_);
    return !waiting_.empty() || !running_.empty();
}

SequencePtr Scheduler::get_sequence(SequenceId id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = all_.find(id);
    return it == all_.end() ? nullptr : it->second;
}

}  // namespace mfe
