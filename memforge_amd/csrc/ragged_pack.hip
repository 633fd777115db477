// Ragged pack: one step's packed token batch built on the device from the
// scheduler's step output (one descriptor per contributing sequence).
//
// Three launches, all tiny: status reset, the pack itself (grid-stride over
// rows, with the per-block prefix sum of q_len recomputed in LDS so no launch
// has to wait for another to know where an entry starts), and the bitmap clean
// that returns the duplicate-slot bitmap to all-zero.
//
// Every load is bounded by what the caller declared: an entry is used only
// when its table run and token run lie inside `tables` / `tokens`, and a
// block id is used only when it addresses the pool (num_slots > 0) or is at
// least non-negative. Rows that fail a check load nothing, get slot -1 and
// are reported in `status`, so downstream kernels never see an address
// outside the pool.
#include <algorithm>
#include <climits>

#include "mf_common.h"

namespace mf {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxEntriesLds = 4096;  // entries whose prefix sum fits in LDS

struct PackArgs {
    const int32_t* entries;
    int num_entries;
    const int32_t* tables;
    int64_t tables_len;
    const int32_t* tokens;
    int64_t tokens_len;
    int block_size;
    int max_blocks;
    int64_t total_tokens;
    int64_t* token_ids;
    int64_t* positions;
    int32_t* seq_slot;
    int64_t* slot_mapping;
    int32_t* cu_seqlens;
    int32_t* kv_lens;
    int32_t* block_tables;
    uint32_t* bitmap;
    int64_t num_slots;
    int32_t* status;
};

// An entry may be used only when every field is non-negative and both of its
// runs lie inside the arrays the caller declared.
__device__ __forceinline__ bool entry_ok(const PackArgs& a, const int32_t* en) {
    if (en[0] < 0 || en[2] < 0 || en[3] < 0 || en[4] < 0 || en[5] < 0) return false;
    return (int64_t)en[3] + en[4] <= a.tables_len && (int64_t)en[5] + en[0] <= a.tokens_len;
}

// A block id may be used when it is non-negative and, with a pool size given,
// its whole block lies inside the pool.
__device__ __forceinline__ bool block_ok(const PackArgs& a, int32_t blk) {
    return blk >= 0 && (a.num_slots <= 0 || ((int64_t)blk + 1) * a.block_size <= a.num_slots);
}

// status[1..3] hold INT_MAX - row so that "no error" is 0 and atomicMax keeps
// the smallest row; the finish kernel turns them into row indices or -1.
__global__ void pack_reset_kernel(int32_t* status) {
    if (threadIdx.x < 4) status[threadIdx.x] = 0;
}

__global__ __launch_bounds__(kThreads) void pack_kernel(PackArgs a) {
    __shared__ int64_t cu[kMaxEntriesLds + 1];
    __shared__ int64_t part[kThreads];
    const int B = a.num_entries;
    const int tid = threadIdx.x;

    // Block-wide exclusive scan of q_len (negative lengths count as 0; 64-bit
    // sums so that no descriptor can wrap them): each thread sums a
    // contiguous run of entries, the run totals are scanned, then each run is
    // re-walked.
    const int per = (B + kThreads - 1) / kThreads;
    const int e0 = min(B, tid * per), e1 = min(B, e0 + per);
    int64_t run = 0;
    for (int e = e0; e < e1; ++e) run += max(0, a.entries[e * MF_ENTRY_INTS + 0]);
    part[tid] = run;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const int64_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int64_t acc = part[tid] - run;
    for (int e = e0; e < e1; ++e) {
        cu[e] = acc;
        acc += max(0, a.entries[e * MF_ENTRY_INTS + 0]);
    }
    if (tid == kThreads - 1) cu[B] = part[kThreads - 1];
    __syncthreads();

    const int64_t gtid = (int64_t)blockIdx.x * kThreads + tid;
    const int64_t gsize = (int64_t)gridDim.x * kThreads;

    // Per-entry outputs. cu_seqlens is clamped to total_tokens so that it
    // never names a row past the packed batch, even for a malformed step.
    if (blockIdx.x == 0) {
        for (int e = tid; e <= B; e += kThreads) a.cu_seqlens[e] = (int32_t)min(cu[e], a.total_tokens);
        if (tid == 0 && cu[B] != a.total_tokens) atomicOr(&a.status[0], MF_PACK_ROW_COUNT);
        for (int e = tid; e < B; e += kThreads) {
            const int32_t* en = a.entries + e * MF_ENTRY_INTS;
            a.kv_lens[e] = max(0, en[2]);
            if (!entry_ok(a, en)) {
                atomicOr(&a.status[0], MF_PACK_BAD_ENTRY);
                atomicMax(&a.status[3], INT_MAX - e);
            }
        }
    }
    // The padded block table (block 0 is as good as any for the padding, and
    // for an id that does not address the pool).
    const int64_t nbt = (int64_t)B * a.max_blocks;
    for (int64_t idx = gtid; idx < nbt; idx += gsize) {
        const int e = (int)(idx / a.max_blocks);
        const int k = (int)(idx - (int64_t)e * a.max_blocks);
        const int32_t* en = a.entries + e * MF_ENTRY_INTS;
        int32_t blk = 0;
        if (k < en[4] && entry_ok(a, en)) {
            blk = a.tables[en[3] + k];
            if (!block_ok(a, blk)) {
                atomicOr(&a.status[0], MF_PACK_BLOCK_OUT_OF_POOL);
                blk = 0;
            }
        }
        a.block_tables[idx] = blk;
    }

    // Rows.
    for (int64_t r = gtid; r < a.total_tokens; r += gsize) {
        if (r >= cu[B]) {  // more rows than the entries hold (reported above)
            a.token_ids[r] = 0;
            a.positions[r] = 0;
            a.seq_slot[r] = -1;
            a.slot_mapping[r] = -1;
            continue;
        }
        // entry e with cu[e] <= r < cu[e+1] (upper bound search)
        int lo = 0, hi = B;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (cu[mid] <= r) lo = mid;
            else hi = mid;
        }
        const int e = lo;
        const int32_t* en = a.entries + e * MF_ENTRY_INTS;
        const int i = (int)(r - cu[e]);
        const int64_t pos = (int64_t)en[1] + i;
        const bool ok = entry_ok(a, en);
        a.token_ids[r] = ok ? a.tokens[en[5] + i] : 0;
        a.positions[r] = pos;
        a.seq_slot[r] = e;
        int64_t slot = -1;
        if (!ok) {
            // reported with its entry; loads nothing
        } else if (pos < 0) {
            atomicOr(&a.status[0], MF_PACK_NEGATIVE_POSITION);
        } else {
            const int64_t lb = pos / a.block_size;
            if (lb >= en[4]) {
                atomicOr(&a.status[0], MF_PACK_TABLE_OVERFLOW);
                atomicMax(&a.status[1], INT_MAX - (int32_t)r);
            } else {
                const int32_t blk = a.tables[en[3] + lb];
                if (block_ok(a, blk)) {
                    slot = (int64_t)blk * a.block_size + (pos - lb * a.block_size);
                } else {
                    atomicOr(&a.status[0], MF_PACK_BLOCK_OUT_OF_POOL);
                    atomicMax(&a.status[1], INT_MAX - (int32_t)r);
                }
            }
        }
        a.slot_mapping[r] = slot;
        if (a.bitmap && slot >= 0 && slot < a.num_slots) {
            const uint32_t bit = 1u << (slot & 31);
            const uint32_t old = atomicOr(&a.bitmap[slot >> 5], bit);
            if (old & bit) {
                atomicOr(&a.status[0], MF_PACK_DUPLICATE_SLOT);
                atomicMax(&a.status[2], INT_MAX - (int32_t)r);
            }
        }
    }
}

// Clears the bits pack_kernel set and turns the row fields into indices.
__global__ __launch_bounds__(kThreads) void pack_finish_kernel(PackArgs a) {
    const int64_t gtid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t gsize = (int64_t)gridDim.x * kThreads;
    if (a.bitmap) {
        for (int64_t r = gtid; r < a.total_tokens; r += gsize) {
            const int64_t slot = a.slot_mapping[r];
            if (slot >= 0 && slot < a.num_slots) atomicAnd(&a.bitmap[slot >> 5], ~(1u << (slot & 31)));
        }
    }
    if (gtid >= 1 && gtid < 4) {
        const int32_t v = a.status[gtid];
        a.status[gtid] = v == 0 ? -1 : INT_MAX - v;
    }
}

}  // namespace
}  // namespace mf

extern "C" int mf_ragged_pack(const int32_t* entries, int num_entries, const int32_t* tables,
                              int64_t tables_len, const int32_t* tokens, int64_t tokens_len,
                              int block_size, int max_blocks, int64_t total_tokens,
                              int64_t* token_ids, int64_t* positions, int32_t* seq_slot,
                              int64_t* slot_mapping, int32_t* cu_seqlens, int32_t* kv_lens,
                              int32_t* block_tables, uint32_t* slot_bitmap, int64_t num_slots,
                              int32_t* status, mf_stream_t stream) {
    using namespace mf;
    if (num_entries < 0 || num_entries > kMaxEntriesLds || block_size <= 0 || max_blocks < 0 ||
        total_tokens < 0 || total_tokens > INT_MAX || tables_len < 0 || tokens_len < 0 ||
        num_slots < 0 || !status || !cu_seqlens)
        return MF_ERR_ARG;
    if (num_entries == 0 && total_tokens > 0) return MF_ERR_ARG;  // rows without an entry
    if (num_entries > 0 && (!entries || !kv_lens)) return MF_ERR_ARG;
    if (tables_len > 0 && !tables) return MF_ERR_ARG;
    if (tokens_len > 0 && !tokens) return MF_ERR_ARG;
    if (total_tokens > 0 && (!token_ids || !positions || !seq_slot || !slot_mapping)) return MF_ERR_ARG;
    if ((int64_t)num_entries * max_blocks > 0 && !block_tables) return MF_ERR_ARG;
    if (slot_bitmap && num_slots <= 0) return MF_ERR_ARG;
    PackArgs a{entries, num_entries, tables, tables_len, tokens, tokens_len, block_size, max_blocks,
               total_tokens, token_ids, positions, seq_slot, slot_mapping, cu_seqlens, kv_lens,
               block_tables, slot_bitmap, num_slots, status};
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(pack_reset_kernel, dim3(1), dim3(64), 0, st, status);
    if (int e = check_launch()) return e;
    const int64_t work = std::max<int64_t>(total_tokens, (int64_t)num_entries * max_blocks);
    int64_t blocks = (work + kThreads - 1) / kThreads;
    blocks = std::min<int64_t>(std::max<int64_t>(blocks, 1), 1024);
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, st, a);
    if (int e = check_launch()) return e;
    int64_t fblocks = std::min<int64_t>(std::max<int64_t>((total_tokens + kThreads - 1) / kThreads, 1), 1024);
    hipLaunchKernelGGL(pack_finish_kernel, dim3((unsigned)fblocks), dim3(kThreads), 0, st, a);
    return check_launch();
}
