// Ragged pack: one step's packed token batch built on the device from the
// scheduler's step output (one descriptor per contributing sequence).
//
// Three launches, all tiny: status reset, the pack itself (grid-stride over
// rows, with the per-block prefix sum of q_len recomputed in LDS so no launch
// has to wait for another to know where an entry starts), and the bitmap clean
// that returns the duplicate-slot bitmap to all-zero.
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
    const int32_t* tokens;
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

// status[1..3] hold INT_MAX - row so that "no error" is 0 and atomicMax keeps
// the smallest row; the finish kernel turns them into row indices or -1.
__global__ void pack_reset_kernel(int32_t* status) {
    if (threadIdx.x < 4) status[threadIdx.x] = 0;
}

__global__ __launch_bounds__(kThreads) void pack_kernel(PackArgs a) {
    __shared__ int32_t cu[kMaxEntriesLds + 1];
    __shared__ int32_t part[kThreads];
    const int B = a.num_entries;
    const int tid = threadIdx.x;

    // Block-wide exclusive scan of q_len: each thread sums a contiguous run of
    // entries, the run totals are scanned, then each run is re-walked.
    const int per = (B + kThreads - 1) / kThreads;
    const int e0 = min(B, tid * per), e1 = min(B, e0 + per);
    int32_t run = 0;
    for (int e = e0; e < e1; ++e) run += max(0, a.entries[e * MF_ENTRY_INTS + 0]);
    part[tid] = run;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const int32_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int32_t acc = part[tid] - run;
    for (int e = e0; e < e1; ++e) {
        cu[e] = acc;
        acc += max(0, a.entries[e * MF_ENTRY_INTS + 0]);
    }
    if (tid == kThreads - 1) cu[B] = part[kThreads - 1];
    __syncthreads();

    const int64_t gtid = (int64_t)blockIdx.x * kThreads + tid;
    const int64_t gsize = (int64_t)gridDim.x * kThreads;

    // Per-entry outputs and the padded block table (block 0 is as good as any).
    if (blockIdx.x == 0) {
        for (int e = tid; e <= B; e += kThreads) a.cu_seqlens[e] = cu[e];
        for (int e = tid; e < B; e += kThreads) {
            const int32_t* en = a.entries + e * MF_ENTRY_INTS;
            a.kv_lens[e] = en[2];
            if (en[0] < 0 || en[2] < 0 || en[3] < 0 || en[4] < 0 || en[5] < 0) {
                atomicOr(&a.status[0], MF_PACK_BAD_ENTRY);
                atomicMax(&a.status[3], INT_MAX - e);
            }
        }
    }
    const int64_t nbt = (int64_t)B * a.max_blocks;
    for (int64_t idx = gtid; idx < nbt; idx += gsize) {
        const int e = (int)(idx / a.max_blocks);
        const int k = (int)(idx - (int64_t)e * a.max_blocks);
        const int32_t* en = a.entries + e * MF_ENTRY_INTS;
        a.block_tables[idx] = (k < en[4] && en[3] >= 0) ? a.tables[en[3] + k] : 0;
    }

    // Rows.
    for (int64_t r = gtid; r < a.total_tokens; r += gsize) {
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
        a.token_ids[r] = a.tokens[en[5] + i];
        a.positions[r] = pos;
        a.seq_slot[r] = e;
        int64_t slot = -1;
        if (pos < 0) {
            atomicOr(&a.status[0], MF_PACK_NEGATIVE_POSITION);
        } else {
            const int64_t blk = pos / a.block_size;
            if (blk >= en[4]) {
                atomicOr(&a.status[0], MF_PACK_TABLE_OVERFLOW);
                atomicMax(&a.status[1], INT_MAX - (int32_t)r);
            } else {
                slot = (int64_t)a.tables[en[3] + blk] * a.block_size + (pos - blk * a.block_size);
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
                              const int32_t* tokens, int block_size, int max_blocks,
                              int64_t total_tokens, int64_t* token_ids, int64_t* positions,
                              int32_t* seq_slot, int64_t* slot_mapping, int32_t* cu_seqlens,
                              int32_t* kv_lens, int32_t* block_tables, uint32_t* slot_bitmap,
                              int64_t num_slots, int32_t* status, mf_stream_t stream) {
    using namespace mf;
    if (num_entries < 0 || num_entries > kMaxEntriesLds || block_size <= 0 || max_blocks < 0 ||
        total_tokens < 0 || total_tokens > INT_MAX || !status || !cu_seqlens)
        return MF_ERR_ARG;
    if (num_entries > 0 && (!entries || !kv_lens)) return MF_ERR_ARG;
    if (total_tokens > 0 && (!tables || !tokens || !token_ids || !positions || !seq_slot || !slot_mapping))
        return MF_ERR_ARG;
    if ((int64_t)num_entries * max_blocks > 0 && !block_tables) return MF_ERR_ARG;
    if (slot_bitmap && num_slots <= 0) return MF_ERR_ARG;
    PackArgs a{entries, num_entries, tables, tokens, block_size, max_blocks, total_tokens,
               token_ids, positions, seq_slot, slot_mapping, cu_seqlens, kv_lens, block_tables,
               slot_bitmap, num_slots, status};
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
