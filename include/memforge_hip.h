/*
 * memforge_hip.h -- C ABI of libmemforge_hip.so, the gfx950 (MI355X) device
 * library behind MemForge's continuous-batching data path.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on `stream` (a hipStream_t, NULL for the default
 * stream) and returns an int status: MF_OK (0) or a negative MF_ERR_* code.
 * Nothing here allocates device memory or synchronises the stream; scratch
 * space is passed in by the caller. Strides are in ELEMENTS, and the last
 * (head_dim) axis of every K/V/Q tensor must be contiguous.
 *
 * Pool addressing (shared by every entry point that touches the KV pool):
 * a slot index s = block * block_size + offset names one token of one
 * physical block, and element (s, head, d) of one layer lives at
 *     layer_base + block * pool_stride_block + offset * pool_stride_slot
 *                + head * pool_stride_head + d.
 * That covers both layouts the reference uses: PagedKVPool's
 * (layers, blocks, slots, kv_heads, head_dim) and PagedKVCache's
 * (blocks, heads, slots, head_dim).
 */
#ifndef MEMFORGE_HIP_H
#define MEMFORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mf_stream_t; /* a hipStream_t */

/* Element types. */
enum { MF_F32 = 0, MF_F16 = 1, MF_BF16 = 2 };

/* Status codes. */
enum {
    MF_OK = 0,
    MF_ERR_ARG = -1,         /* bad size, stride, pointer or dtype */
    MF_ERR_UNSUPPORTED = -2, /* head_dim / dtype combination not built */
    MF_ERR_WORKSPACE = -3,   /* caller-supplied scratch is too small */
    MF_ERR_HIP = -4          /* a HIP launch failed; see mf_last_hip_error */
};

/* Library version string and the last HIP error code seen by this thread. */
const char* mf_version(void);
int mf_last_hip_error(void);
const char* mf_status_string(int status);

/* ------------------------------------------------------------------ KV write
 * Scatter `num_tokens` new key/value rows into one layer of the pool through
 * slot_mapping (int64, one slot per row). A row whose slot is outside
 * [0, num_slots) -- num_slots = blocks * block_size of one pool layer -- is
 * skipped, so a malformed slot can never address memory past the pool.
 * Source row t, head h starts at src + t*src_stride_t + h*src_stride_h (the
 * same strides for k_src and v_src). Converts src_dtype -> pool_dtype with
 * round-to-nearest-even, so the result is bit-identical to torch's
 * `.to(pool dtype)` followed by `index_copy_`.
 * Replaces paged_gather.scatter_kv (memforge_ml/kernels/paged_gather.py:92-117),
 * PagedKVPool.write / write_flat (memforge_ml/runtime/kv_pool.py:134-149,
 * 181-192) and PagedKVCache.write_kv (memforge_ml/models/paged_attention.py:45-67).
 */
int mf_kv_write(const void* k_src, const void* v_src, int src_dtype,
                int64_t src_stride_t, int64_t src_stride_h,
                const int64_t* slot_mapping, int64_t num_tokens,
                void* k_pool, void* v_pool, int pool_dtype,
                int64_t pool_stride_block, int64_t pool_stride_slot,
                int64_t pool_stride_head, int block_size, int64_t num_slots,
                int num_heads, int head_dim, mf_stream_t stream);

/* ----------------------------------------------------------------- KV gather
 * The inverse of mf_kv_write: copy pool slots slot_mapping[0..num_tokens) of
 * one layer into dst rows (dst + t*dst_stride_t + h*dst_stride_h), converting
 * pool_dtype -> dst_dtype. Rows whose slot is outside [0, num_slots) are left
 * unwritten.
 * Replaces paged_gather.gather_kv (memforge_ml/kernels/paged_gather.py:58-89),
 * PagedKVPool.gather / gather_flat (memforge_ml/runtime/kv_pool.py:151-179)
 * and PagedKVCache.read_kv (memforge_ml/models/paged_attention.py:69-97).
 */
int mf_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype,
                 int64_t pool_stride_block, int64_t pool_stride_slot,
                 int64_t pool_stride_head, int block_size, int64_t num_slots,
                 const int64_t* slot_mapping, int64_t num_tokens,
                 void* k_dst, void* v_dst, int dst_dtype,
                 int64_t dst_stride_t, int64_t dst_stride_h, int num_heads,
                 int head_dim, mf_stream_t stream);

/* ---------------------------------------------------------------- block copy
 * The data half of copy-on-write: for each (src, dst) pair in `pairs` (HOST
 * memory, int64, num_pairs x 2), copy physical block src to block dst in every
 * one of `num_layers` layers of both pools. One block of one layer is
 * `block_elems` contiguous elements at layer * pool_stride_layer +
 * block * pool_stride_block (PagedKVPool's (layers, blocks, slots, kv_heads,
 * head_dim) layout: block_elems = slots * kv_heads * head_dim). A pair with
 * src == dst is skipped. MF_ERR_ARG if an index is outside [0, num_blocks),
 * a block is the destination of two pairs, or a destination is also a source
 * (the result would depend on copy order). The pairs go in the kernel
 * arguments (up to 32 per launch), so nothing is allocated or uploaded.
 * Replaces prefix_sharing.copy_block
 * (memforge_ml/runtime/prefix_sharing.py:27-42), which the engine calls when
 * BlockAllocator::prepare_write returns a pair
 * (memforge_ml/runtime/continuous_engine.py:974-1006).
 */
int mf_kv_copy_blocks(void* k_pool, void* v_pool, int pool_dtype, int num_layers,
                      int64_t pool_stride_layer, int64_t pool_stride_block,
                      int64_t block_elems, int64_t num_blocks,
                      const int64_t* pairs, int num_pairs, mf_stream_t stream);

/* --------------------------------------------------------------- ragged pack
 * Build one step's packed token batch on the device from the scheduler's step
 * output. `entries` (device, int32, B rows of MF_ENTRY_INTS) describes each
 * sequence contributing tokens this step, in plan order:
 *   [0] q_len      query tokens this step (chunk length, 1 for a decode,
 *                  k+1 for a speculative verify row)
 *   [1] start_pos  absolute position of the first of them
 *   [2] kv_len     keys attention may read for this entry
 *   [3] table_off  offset of its block table in `tables`
 *   [4] table_len  entries in its block table
 *   [5] token_off  offset of its q_len token ids in `tokens`
 * `tables` holds tables_len int32 block ids and `tokens` tokens_len int32 token
 * ids (device). An entry is malformed (MF_PACK_BAD_ENTRY) when a field is
 * negative, its table run [table_off, table_off + table_len) leaves `tables`,
 * or its token run [token_off, token_off + q_len) leaves `tokens`; the rows of
 * a malformed entry load nothing (token 0, slot -1) and its block-table row is
 * all 0. total_tokens must equal the sum of q_len (MF_PACK_ROW_COUNT
 * otherwise; surplus rows get seq_slot -1 and slot -1).
 * Outputs (device): token_ids[T] and positions[T] (int64, the model's
 * input_ids / position_ids), seq_slot[T] (entry index per row), slot_mapping[T]
 * (int64, table[p / bs] * bs + p % bs), cu_seqlens[B+1], kv_lens[B] and the
 * padded block_tables[B][max_blocks] (unused entries 0). T = sum of q_len.
 * status (device, int32[4], written by this call) reports malformed input:
 *   status[0] bit flags: MF_PACK_TABLE_OVERFLOW, MF_PACK_NEGATIVE_POSITION,
 *             MF_PACK_DUPLICATE_SLOT, MF_PACK_BAD_ENTRY, MF_PACK_ROW_COUNT,
 *             MF_PACK_BLOCK_OUT_OF_POOL
 *   status[1] first row whose slot could not be formed: it needs a block past
 *             its table, or (num_slots > 0) its block lies outside a pool of
 *             num_slots slots (or -1)
 *   status[2] a row whose slot another row also writes (or -1)
 *   status[3] first malformed entry (or -1)
 * With num_slots > 0, slots at or past num_slots are reported and replaced by
 * -1. Duplicate detection runs when slot_bitmap is non-NULL: a device bitmap
 * of num_slots bits that must be all-zero on entry and is all-zero again on
 * exit. num_entries == 0 with total_tokens > 0 is MF_ERR_ARG.
 * Replaces the engine's per-step packing (memforge_ml/runtime/
 * continuous_engine.py:782-905, 1104-1131; batched_speculative.py:696-701) and
 * VarlenPackedCache._build_write_index (memforge_ml/runtime/varlen_cache.py:161-191).
 */
#define MF_ENTRY_INTS 6
#define MF_PACK_TABLE_OVERFLOW 1
#define MF_PACK_NEGATIVE_POSITION 2
#define MF_PACK_DUPLICATE_SLOT 4
#define MF_PACK_BAD_ENTRY 8
#define MF_PACK_ROW_COUNT 16
#define MF_PACK_BLOCK_OUT_OF_POOL 32
int mf_ragged_pack(const int32_t* entries, int num_entries,
                   const int32_t* tables, int64_t tables_len,
                   const int32_t* tokens, int64_t tokens_len,
                   int block_size, int max_blocks, int64_t total_tokens,
                   int64_t* token_ids, int64_t* positions, int32_t* seq_slot,
                   int64_t* slot_mapping, int32_t* cu_seqlens, int32_t* kv_lens,
                   int32_t* block_tables, uint32_t* slot_bitmap,
                   int64_t num_slots, int32_t* status, mf_stream_t stream);

/* ----------------------------------------------------------- paged attention
 * Varlen paged attention: one code path for decode, chunked prefill and the
 * (k+1)-query speculative verify. Packed query rows of sequence s are
 * cu_seqlens[s] .. cu_seqlens[s+1]-1 (through row_map[] when non-NULL, which
 * maps packed index -> physical row of q/out/positions). Row r of sequence s
 * attends, for every query head, to the keys of s at positions
 * 0 .. positions[r] (inclusive) that are < kv_lens[s], with grouped-query
 * heads (query head qh reads kv head qh / (num_q_heads / num_kv_heads)).
 * Keys below pool_lens[s] (all keys when pool_lens is NULL) are read from the
 * pool through block_tables[s][key / block_size]; keys at or above it are the
 * in-flight rows of the same sequence's new tokens (new_k/new_v row
 * cu_seqlens[s] + key - pool_lens[s], through row_map), which is how a verify
 * pass attends to candidates it has not written to the pool. Scores are
 * q.k * scale; any finite scale works (a negative one flips q's sign bits, a
 * zero one gives uniform weights), a NaN or infinite one is MF_ERR_ARG.
 * Softmax accumulates in fp32; out is written in `dtype` (the q/K/V dtype).
 * Work is described by a plan from mf_attention_plan (device copy of its
 * items/merges; num_items_narrow and num_items_wide are multiples of four, as
 * the planner makes them, else MF_ERR_ARG); `partials` is fp32 scratch of at
 * least the planned size.
 * merge_counters (device int32[num_merges], all-zero on entry and again on
 * exit) lets the attention kernel merge split-K partitions itself: the last
 * partition of a group to finish merges it. With merge_counters NULL a
 * separate merge kernel runs after the attention kernel. A plan holding both
 * single-tile (decode) and wide (prefill) items runs them in one launch when
 * block_size is 16 and head_dim is one of the kernel's sizes, 16-bit dtypes
 * only. Passing the plan's
 * items with num_merges = 0, then a second call with no items and only the
 * merges, runs the unfused work in two launches (to time them apart).
 * Concurrent calls must not share partials or merge_counters.
 * Replaces paged_attention_varlen / _materialised (memforge_ml/kernels/
 * varlen_attention.py:78-235, 291-395), paged_attention_blockwise
 * (memforge_ml/kernels/block_attention.py:51-145), PagedAttention.forward
 * (memforge_ml/models/paged_attention.py:108-141) and the Triton
 * paged_decode_attention (memforge_ml/kernels/triton_paged_decode.py:129-176).
 */
int mf_paged_attention(const void* q, int64_t q_stride_row, int64_t q_stride_head,
                       void* out, int64_t out_stride_row, int64_t out_stride_head,
                       int dtype, const void* k_pool, const void* v_pool,
                       int64_t pool_stride_block, int64_t pool_stride_slot,
                       int64_t pool_stride_head, int block_size,
                       const int32_t* block_tables, int64_t block_table_stride,
                       const int32_t* cu_seqlens, const int32_t* kv_lens,
                       const int64_t* positions, const int32_t* row_map,
                       const int32_t* pool_lens, const void* new_k, const void* new_v,
                       int64_t new_stride_row, int64_t new_stride_head,
                       int num_q_heads, int num_kv_heads, int head_dim, float scale,
                       const int32_t* plan_items, int64_t num_items_narrow,
                       int64_t num_items_wide, const int32_t* plan_merges,
                       int64_t num_merges, float* partials, int64_t partials_floats,
                       int32_t* merge_counters, mf_stream_t stream);

/* mf_paged_attention with the work counts read from device memory, for a
 * caller that captures the launch in a HIP graph and replays it with a new
 * plan each step. No counterpart in the reference: it serves callers that
 * capture the decode step (the grid must be fixed at capture time).
 * The grids are sized by the capacities (multiples of four, else MF_ERR_ARG):
 * plan_items holds capacity_narrow
 * narrow items followed by capacity_wide wide items (wide items always start
 * at plan_items + capacity_narrow * MF_PLAN_ITEM_INTS), plan_merges holds
 * capacity_merges records, and device_counts (device, int32[3]) gives the
 * live numbers of narrow items, wide items and merges -- each at most its
 * capacity, both item counts multiples of four as mf_attention_plan makes them;
 * workgroups past them exit at once. Split-K partitions are merged
 * by the separate merge kernel. Everything else is as in mf_paged_attention.
 */
int mf_paged_attention_counted(const void* q, int64_t q_stride_row, int64_t q_stride_head,
                               void* out, int64_t out_stride_row, int64_t out_stride_head,
                               int dtype, const void* k_pool, const void* v_pool,
                               int64_t pool_stride_block, int64_t pool_stride_slot,
                               int64_t pool_stride_head, int block_size,
                               const int32_t* block_tables, int64_t block_table_stride,
                               const int32_t* cu_seqlens, const int32_t* kv_lens,
                               const int64_t* positions, const int32_t* row_map,
                               const int32_t* pool_lens, const void* new_k, const void* new_v,
                               int64_t new_stride_row, int64_t new_stride_head,
                               int num_q_heads, int num_kv_heads, int head_dim, float scale,
                               const int32_t* plan_items, int64_t capacity_narrow,
                               int64_t capacity_wide, const int32_t* plan_merges,
                               int64_t capacity_merges, const int32_t* device_counts,
                               float* partials, int64_t partials_floats, mf_stream_t stream);

/* One packed step's KV write and its attention in one launch. Equivalent to
 * mf_kv_write of new rows [0, num_new_rows) through slot_mapping (a slot < 0
 * or >= num_slots is skipped) followed by mf_paged_attention with pool_lens
 * set to kv_lens[s] - (cu_seqlens[s+1] - cu_seqlens[s]): the pool ends in the
 * same state and the output is the same, bit for bit. Row cu_seqlens[s] + i
 * of q, positions and new_k/new_v must be sequence s's new token at position
 * kv_lens[s] - (cu_seqlens[s+1] - cu_seqlens[s]) + i (how the engine packs a
 * step: every sequence's new tokens, in position order, end its context).
 * The attention reads each sequence's new keys from new_k/new_v instead of
 * the pool, so no workgroup waits on the copy, which runs in workgroups of
 * the same launch. new_k/new_v are (rows, num_kv_heads, head_dim) in `dtype`
 * with element strides new_stride_row / new_stride_head (16-byte aligned
 * rows). With a block_size other than 16 or a head_dim the kernels pad, the
 * call runs as the two launches it replaces. device_counts NULL: num_items_* and num_merges are the
 * plan's counts, as in mf_paged_attention; non-NULL: they are capacities and
 * device_counts holds the live counts, as in mf_paged_attention_counted (for
 * graph capture; padding rows then carry slot -1). Split-K partitions are
 * merged by the separate merge kernel.
 * Replaces VarlenPackedCacheLayer.update's pool.write_flat
 * (memforge_ml/runtime/varlen_cache.py:61-90, memforge_ml/runtime/kv_pool.py:181-192)
 * together with the varlen binding of paged_attention_forward that follows it
 * in every layer (memforge_ml/kernels/attention_backend.py:195-272).
 */
int mf_paged_attention_kv_write(const void* q, int64_t q_stride_row, int64_t q_stride_head,
                                void* out, int64_t out_stride_row, int64_t out_stride_head,
                                int dtype, void* k_pool, void* v_pool,
                                int64_t pool_stride_block, int64_t pool_stride_slot,
                                int64_t pool_stride_head, int block_size,
                                const int32_t* block_tables, int64_t block_table_stride,
                                const int32_t* cu_seqlens, const int32_t* kv_lens,
                                const int64_t* positions, const void* new_k, const void* new_v,
                                int64_t new_stride_row, int64_t new_stride_head,
                                const int64_t* slot_mapping, int64_t num_new_rows, int64_t num_slots,
                                int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                const int32_t* plan_items, int64_t num_items_narrow,
                                int64_t num_items_wide, const int32_t* plan_merges,
                                int64_t num_merges, const int32_t* device_counts,
                                float* partials, int64_t partials_floats, mf_stream_t stream);

/* mf_paged_attention without a partials buffer or merge counters, so that
 * the call allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops or harnesses that forbid hipMalloc). Split-K partials go to
 * a device array the library owns: MF_NOALLOC_PARTIALS_FLOATS fp32 values
 * (32 MiB) per GPU, held from the first call on that GPU until the process
 * ends; partitions are merged by the separate merge kernel. partials_floats
 * is what the plan needs (counts[3] from mf_attention_plan): a plan needing
 * more is MF_ERR_WORKSPACE, returned before anything touches the device.
 * partials_floats must cover every partial slot the plan's items and merge
 * records name (a planner-made plan's counts[3] does): the kernels do not
 * bound slots, so a hand-edited plan naming slots past the array would write
 * past it. The Python binding checks this against the host copy of the plan. The
 * stream must belong to the current device. Every call on one GPU uses the
 * same array, which keeps the last call's contents (no kernel here needs it
 * cleared), so calls that overlap on one GPU race. Everything else is as in
 * mf_paged_attention. */
#define MF_NOALLOC_PARTIALS_FLOATS (8 * 1024 * 1024)
int mf_paged_attention_noalloc(const void* q, int64_t q_stride_row, int64_t q_stride_head,
                               void* out, int64_t out_stride_row, int64_t out_stride_head,
                               int dtype, const void* k_pool, const void* v_pool,
                               int64_t pool_stride_block, int64_t pool_stride_slot,
                               int64_t pool_stride_head, int block_size,
                               const int32_t* block_tables, int64_t block_table_stride,
                               const int32_t* cu_seqlens, const int32_t* kv_lens,
                               const int64_t* positions, const int32_t* row_map,
                               const int32_t* pool_lens, const void* new_k, const void* new_v,
                               int64_t new_stride_row, int64_t new_stride_head,
                               int num_q_heads, int num_kv_heads, int head_dim, float scale,
                               const int32_t* plan_items, int64_t num_items_narrow,
                               int64_t num_items_wide, const int32_t* plan_merges,
                               int64_t num_merges, int64_t partials_floats, mf_stream_t stream);

/* Host-side planner for mf_paged_attention. Inputs are HOST arrays:
 * cu_seqlens[B+1] and kv_lens[B]. Splits every (sequence, kv head, column
 * tile) over key partitions of `partition_tiles` 16-key tiles (0 = chosen
 * from the work: narrow and wide items separately) and writes
 * MF_PLAN_ITEM_INTS ints per work item to items (narrow items -- one
 * 16-column tile -- first, then wide ones) and MF_PLAN_MERGE_INTS ints per
 * split-K merge to merges. Narrow items come in workgroups of four: four
 * single-wave items (ranges of at most P tiles), or one cooperative unit
 * (last int 1) whose four waves take consecutive quarters of a range of at
 * most 4P tiles and combine their softmax states in LDS; only longer ranges
 * are split into several units and merged. Wide items come in workgroups of four: a run of
 * four or more column groups over one (sequence, kv head, key range) fills
 * whole workgroups, which then share each K/V tile through LDS (the last one
 * padded with items that have no column tiles and no partial slot); shorter
 * runs are packed four to a workgroup. With partition_tiles 0 and both item
 * kinds in the plan (one mixed launch), each such workgroup's four column
 * groups (a column quad) take partitions of their own: the tiles the quad's
 * last column can see, cut into equal ranges sized so that the wide
 * workgroups carry about two per compute unit; tiles no column of the quad
 * sees are not planned. The wide workgroups of one key range (in that case,
 * of one sequence and kv head) are placed at grid positions of one residue
 * mod 8, so they run on one XCD and share its L2. counts receives
 * [num_items_narrow, num_items_wide, num_merges, partials_floats].
 * A plan is valid for the dtype and head_dim it was made for and carries the
 * sequences' first rows, row counts and kv lengths: the cu_seqlens / kv_lens
 * later passed to mf_paged_attention must hold the same values.
 * Returns MF_ERR_WORKSPACE if a capacity is too small (counts still holds
 * the required sizes). */
#define MF_PLAN_ITEM_INTS 12
#define MF_PLAN_MERGE_INTS 8
int mf_attention_plan(int num_seqs, const int32_t* cu_seqlens, const int32_t* kv_lens,
                      int num_q_heads, int num_kv_heads, int head_dim, int dtype,
                      int partition_tiles, int32_t* items, int64_t items_capacity,
                      int32_t* merges, int64_t merges_capacity, int64_t* counts);

/* ------------------------------------------------- decode slice plans
 * A second plan form for large decode launches, with the same results as
 * mf_attention_plan + mf_paged_attention (up to fp32 summation order).
 * Replaces, like mf_paged_attention, the decode call of
 * paged_attention_varlen (memforge_ml/kernels/varlen_attention.py:78-235)
 * and the Triton paged_decode_attention (memforge_ml/kernels/
 * triton_paged_decode.py:129-176), for batches large enough to fill the GPU
 * several times over.
 *
 * mf_attention_plan_slices (host) cuts the sequences' 16-key tiles, in
 * sequence order, into slices of equal size: num_cus * MF_SLICE_WAVES_PER_CU
 * / num_kv_heads of them, so that one wave per (slice, kv head) fills the GPU
 * once at one workgroup (one wave per SIMD) per compute unit; num_cus is the
 * device's compute units (hipDeviceProp_t::multiProcessorCount). A workload
 * whose even share exceeds a slice runs whole rounds of such slices. A slice
 * holds at most MF_SLICE_MAX_SEGMENTS sequence pieces and MF_SLICE_MAX_TILES
 * tiles once each piece is padded to a multiple of three. Each sequence cut
 * across slices leaves one fp32 partial per piece and kv head, merged by the
 * records written to merges (MF_PLAN_MERGE_INTS ints each).
 * slices receives MF_SLICE_INTS ints per record: num_slices slice records
 * (first segment, segments, padded tiles, 0...) followed by num_segments
 * segment records (sequence, first tile, end tile, query row, kv length,
 * first partial slot or -1, pieces of the sequence, piece index).
 * counts receives [num_slices, num_segments, num_merges, partials_floats].
 * Only decode steps qualify: every sequence with keys has one query row,
 * num_q_heads / num_kv_heads <= 16, and head_dim is one of the kernel's sizes
 * (32-256 for 16-bit types, 16-128 for fp32, powers of two); otherwise
 * MF_ERR_UNSUPPORTED. A launch whose tiles give each of its waves fewer than
 * min_tiles_per_wave gets no slice plan (MF_OK with counts all zero);
 * MF_SLICE_MIN_TILES is the measured choice (below it mf_attention_plan's
 * items fit the launch in one round), 0 plans every decode step. Returns
 * MF_ERR_WORKSPACE if a capacity is too small (counts holds the required
 * sizes).
 *
 * mf_paged_attention_slices runs such a plan: arguments as in
 * mf_paged_attention without in-flight keys (every key is in the pool),
 * with block_size 16; the plan carries the rows, kv lengths and split
 * pieces, and cu_seqlens / kv_lens must hold the values it was made from.
 * Partials need counts[3] floats. Any other block size is
 * MF_ERR_UNSUPPORTED. */
#define MF_SLICE_INTS 8
#define MF_SLICE_MAX_TILES 512
#define MF_SLICE_MAX_SEGMENTS 64
#define MF_SLICE_MIN_TILES 64
#define MF_SLICE_WAVES_PER_CU 4
int mf_attention_plan_slices(int num_seqs, const int32_t* cu_seqlens, const int32_t* kv_lens,
                             int num_q_heads, int num_kv_heads, int head_dim, int dtype,
                             int num_cus, int min_tiles_per_wave, int32_t* slices,
                             int64_t slices_capacity, int32_t* merges, int64_t merges_capacity,
                             int64_t* counts);
int mf_paged_attention_slices(const void* q, int64_t q_stride_row, int64_t q_stride_head,
                              void* out, int64_t out_stride_row, int64_t out_stride_head,
                              int dtype, const void* k_pool, const void* v_pool,
                              int64_t pool_stride_block, int64_t pool_stride_slot,
                              int64_t pool_stride_head, int block_size,
                              const int32_t* block_tables, int64_t block_table_stride,
                              const int32_t* cu_seqlens, const int32_t* kv_lens,
                              const int64_t* positions, int num_q_heads, int num_kv_heads,
                              int head_dim, float scale, const int32_t* slices,
                              int64_t num_slices, int64_t num_segments,
                              const int32_t* plan_merges, int64_t num_merges, float* partials,
                              int64_t partials_floats, mf_stream_t stream);

/* ----------------------------------------------------- rejection verify
 * Speculative rejection sampling for B rows of K draft candidates, with the
 * randomness supplied by the caller. For row b and i < K: p = target
 * probability and q = draft probability of draft_tokens[b][i]; accept iff
 * (double)u_accept[b][i] <= min(1, p / (q + 1e-9)) in double precision. The
 * first rejection resamples from normalise(max(p_vec - q_vec, 0)) (or from
 * the target distribution when that residual sums to 0) and stops the row;
 * if all K are accepted a bonus token is drawn from target position K. A draw
 * from distribution w is argmax_i(w_i / exp_noise[b][i]) (first index on
 * ties), which is torch.multinomial(w, 1) given the same Exp(1) noise.
 * Target probabilities are softmax(target_logits[b][i][:V] / temperature) in
 * fp32, or a one-hot argmax when temperature <= 0; target logits wider than the
 * draft vocabulary V are clipped to V first. With target_is_probs != 0 the
 * target rows already are probabilities (fp32) and are used as given.
 * Outputs: out_tokens[b][0..out_count[b]) (at most K+1), out_is_draft likewise,
 * out_num_accepted[b] draft tokens accepted.
 * workspace: at least mf_spec_verify_workspace_size(B, K) bytes.
 * Replaces RejectionSampler.verify_tokens / sample_from_probs
 * (memforge_ml/speculative/rejection_sampler.py:12-83) and resolve_round /
 * _probs_from_logits (memforge_ml/runtime/batched_speculative.py:112-124, 731-777).
 */
int64_t mf_spec_verify_workspace_size(int num_rows, int num_draft);
int mf_spec_verify(int num_rows, int num_draft, int vocab,
                   const int32_t* draft_tokens,
                   const float* draft_probs, int64_t dp_stride_row, int64_t dp_stride_pos,
                   const void* target_logits, int target_dtype,
                   int64_t tl_stride_row, int64_t tl_stride_pos,
                   float temperature, int target_is_probs, const float* u_accept,
                   const float* exp_noise, int64_t noise_stride_row,
                   int32_t* out_tokens, uint8_t* out_is_draft, int32_t* out_count,
                   int32_t* out_num_accepted, void* workspace, int64_t workspace_bytes,
                   mf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MEMFORGE_HIP_H */
