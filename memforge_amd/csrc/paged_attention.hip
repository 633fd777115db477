// Varlen paged attention for gfx950: one code path for decode, chunked
// prefill and the (k+1)-query speculative verify.
//
// Work decomposition. A "column" is one (query row, query head) pair; the G
// query heads that share a KV head are adjacent columns, so a decode row of a
// GQA group-5 model is 5 columns and a 5-token verify row of a group-3 model is
// 15. One wave owns a work item = (sequence, kv head, up to NT tiles of 16
// columns, a range of 16-key tiles), reads every K/V tile of that range exactly
// once and shares it across all of its columns.
//
// Per 16-key tile the wave computes S^T = K Q^T with MFMA (A = K rows straight
// from the pool, B = the Q fragment kept in registers), applies the per-column
// causal rule key <= position(row), runs the online softmax with the column
// max reduced across the four 16-lane groups by xor shuffles, and accumulates
// O^T = V^T P^T with a second MFMA whose B operand is the exponentiated S^T
// tile exactly as the first MFMA left it in registers. V arrives with
// fully coalesced 16-token x 16-byte row loads and is transposed into the MFMA
// A layout with byte permutes; no LDS is used at all.
//
// Long contexts are split into key partitions (the plan decides); partial
// (max, sum, unnormalised output) triples go to fp32 scratch and a merge
// kernel combines them with the log-sum-exp rule.
#include <algorithm>
#include <array>
#include <atomic>
#include <climits>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "mf_common.h"

#ifndef MF_MAX_ITEM_TILES
#define MF_MAX_ITEM_TILES 128
#endif
namespace mf {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;

constexpr int kWaves = 4;  // waves per workgroup; each wave runs its own item
constexpr int kMaxItemTiles = MF_MAX_ITEM_TILES;  // key tiles per work item (two block-table entries per lane)
#ifndef MF_NARROW_ITEMS
#define MF_NARROW_ITEMS 4096  // planner: target item count that sets the narrow key partition
#endif
// Stages of the workgroup-shared prefill loop move global -> LDS directly
// (1) or through registers (0).
#ifndef MF_WIDE_DIRECT_LDS
#define MF_WIDE_DIRECT_LDS 1
#endif
// Wave priority (s_setprio) of the workgroup-shared wide loop. In a mixed
// launch a CU holds single-tile (decode) waves beside the wide (prefill) ones;
// at equal priority the decode waves' issue slowed the wide workgroups sharing
// their CU by about 40% (per-workgroup timestamps on the C2 step: 31.4 against
// 22.0 us median life), and the CUs holding a decode workgroup finished last.
// Raised, the wide waves issue first and the decode waves take the slots they
// leave while they wait on memory. Measured on the C2 engine layer: 53.7 us at
// equal priority, 49.3-49.8 us at 1, 49.4-49.8 at 2.
#ifndef MF_WIDE_PRIO
#define MF_WIDE_PRIO 1
#endif
// XCD-local order of the wide workgroups (1). The dispatcher sends
// workgroup b of a launch to XCD b mod 8, so the
// consecutive wide workgroups of one key range (the column groups of one
// sequence, kv head and key partition, which read the same K/V tiles) land on
// eight XCDs whose L2s each fetch the tiles. The planner instead deals whole
// ranges to eight queues (least causal work first) and interleaves them, so
// workgroup 8k + x comes from queue x and a range stays on one XCD; each
// queue runs its workgroups most causal work first. Measured on the C2
// prefill items alone: 38.2-38.8 us -> 35.1-35.5 us between events, PMC
// FETCH 74 MB -> 24 MB (1.4x the K/V and query bytes). In a mixed launch the
// wide workgroups follow the single-tile ones, which only rotates the XCDs
// (a range still shares one). There, at 32-tile wide partitions, the order
// was slower (C2 engine layer 49.2 -> 50.2 us); at 64-tile equal-stride
// partitions it was faster: 45.71-45.75 against 45.85-45.94 us, and the mixed
// plan's prefill items alone 34.7-34.9 against 39.6-39.8 us. Mixed plans now
// cut each column quad on its own (quad partitions, in the planner) and keep
// a (sequence, kv head)'s workgroups on one XCD.
#ifndef MF_WIDE_XCD
#define MF_WIDE_XCD 1
#endif
#ifndef MF_WIDE_ITEMS
#define MF_WIDE_ITEMS 4096  // planner: most wide items before partitions grow
#endif
constexpr float kLazyLog2 = 8.f;  // running-max slack of the online softmax (log2 units)
// Running maximum before any key is seen: finite, so exponent arguments never
// need a -inf guard; 2^(kMinM - x) is 0 for every score x.
constexpr float kMinM = -1e30f;

// 16-column tiles one wave carries for multi-tile (prefill / wide verify)
// items: as many as fit in registers without spilling.
__host__ __device__ constexpr int wide_tiles(int dt, int dp) {
    // measured on MI355X: 2 tiles beat 4 for 16-bit head_dim 64 (more waves
    // per SIMD outweigh the K/V reuse across columns)
    return dt == MF_F32 ? (dp >= 128 ? 2 : 4) : (dp >= 256 ? 1 : (dp == 64 ? 2 : 4));
}

struct AttnArgs {
    const char* q;
    int64_t q_sr, q_sh;
    char* out;
    int64_t o_sr, o_sh;
    const char* k_pool;
    const char* v_pool;
    int64_t p_sb, p_ss, p_sh;
    int block_size;
    const int32_t* block_tables;
    int64_t bt_stride;
    const int32_t* cu_seqlens;
    const int32_t* kv_lens;
    const int64_t* positions;
    const int32_t* row_map;
    const int32_t* pool_lens;
    const char* new_k;
    const char* new_v;
    int64_t n_sr, n_sh;
    int G;
    int head_dim;
    float scale_log2;    // |scale| * log2(e), > 0
    float inv_scale_log2;
    uint32_t q_sign;     // xor applied to every Q word: flips the sign for a negative scale
    const int32_t* items;
    int num_items;
    const int32_t* dev_count;  // when set, the live item / merge count (the grid is a capacity)
    float* partials;
    int part_dstride;  // floats per column of a partial slot's output block
    const int32_t* merges;  // plan merge records (fused split-K merge)
    int32_t* counters;      // per-group arrival counters; null = separate merge kernel
    // Written-in-flight launch (mf_paged_attention_kv_write; the kernels'
    // TAIL instances): a sequence's keys at or above kv_len - rows are its own
    // new rows, read from new_k/new_v (row cu_seqlens[s] + key - (kv_len -
    // rows)), and the launch's first w_blocks workgroups copy new rows
    // [0, w_rows) into the pool through w_slots (a slot < 0 or >= w_num_slots
    // is skipped). No item reads a slot that this launch writes, so nothing
    // waits on the copy.
    int num_kv_heads;
    const int64_t* w_slots;
    int w_rows;
    int w_blocks;
    int64_t w_num_slots;
};

// The copy of a written-in-flight launch: workgroup `wblock` of the leading
// w_blocks. Every new row's K and V, head by head, go to the pool slot of
// w_slots in 16-byte pieces: consecutive lanes take consecutive pieces of one
// row (its heads are adjacent), so loads and stores coalesce.
template <int DT>
__device__ __forceinline__ void write_new_rows(const AttnArgs& a, int wblock) {
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    const int cpr = a.head_dim * ES / 16;  // 16-byte pieces of one head's row
    const int per_row = 2 * a.num_kv_heads * cpr;
    const int total = a.w_rows * per_row;
    for (int u = wblock * 256 + (int)threadIdx.x; u < total; u += a.w_blocks * 256) {
        const int row = u / per_row;
        int rest = u - row * per_row;
        const int isv = rest >= a.num_kv_heads * cpr;
        rest -= isv * a.num_kv_heads * cpr;
        const int head = rest / cpr;
        const int piece = rest - head * cpr;
        const int64_t slot = a.w_slots[row];
        if (slot < 0 || slot >= a.w_num_slots) continue;
        const int64_t blk = slot / a.block_size;
        const int64_t off = slot - blk * a.block_size;
        const char* src = (isv ? a.new_v : a.new_k) + ((int64_t)row * a.n_sr + (int64_t)head * a.n_sh) * ES + piece * 16;
        char* dst = const_cast<char*>(isv ? a.v_pool : a.k_pool) +
                    (blk * a.p_sb + off * a.p_ss + (int64_t)head * a.p_sh) * ES + piece * 16;
        *(uint4*)dst = *(const uint4*)src;
    }
}

// ------------------------------------------------------------- MFMA wrappers
// S^T tile: 16 keys x 16 columns, contraction over one 16-byte chunk of
// head_dim per lane (8 x 16-bit or 4 x fp32 elements).
template <int DT>
__device__ __forceinline__ f32x4 mfma_qk(uint4 a, uint4 b, f32x4 c) {
    if constexpr (DT == MF_BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else if constexpr (DT == MF_F16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    } else {
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
        return c;
    }
}

// O^T tile: 16 head_dim rows x 16 columns, contraction over 16 keys
// (4 per lane) for 16-bit types.
template <int DT>
__device__ __forceinline__ f32x4 mfma_pv16(uint2 a, uint2 b, f32x4 c) {
    if constexpr (DT == MF_BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                         __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                     __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
    }
}

// ---------------------------------------------------------- memory helpers

template <int N>
__device__ __forceinline__ void ld_words(const char* p, uint32_t* w) {
    if constexpr (N == 4) {
        w[0] = *(const uint32_t*)p;
    } else if constexpr (N == 8) {
        const uint2 v = *(const uint2*)p;
        w[0] = v.x; w[1] = v.y;
    } else {
        static_assert(N % 16 == 0, "chunk");
#pragma unroll
        for (int k = 0; k < N / 16; ++k) {
            const uint4 v = *(const uint4*)(p + 16 * k);
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    }
}

// The same loads marked non-temporal (streamed, not kept in cache): pool
// tiles of single-column-tile items are read by exactly one wave.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt16(const char* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// 16 bytes per lane from global memory straight into LDS (gfx950's
// global_load_lds_dwordx4): lane i's bytes land at lds_addr + 16 i, lds_addr
// being the same for the whole wave. Written as inline assembly because the
// builtin makes the compiler wait for the transfer before every later LDS
// read; the caller waits for it (vmcnt) before the barrier that publishes it.
// The LDS address is bound to m0 by the operand constraint, so the compiler
// writes m0 itself and knows what it holds (a clobber of the reserved m0
// would not be honoured); the s_nop gives the write its one wait state before
// the load reads it.
__device__ __forceinline__ void ld_lds16(const void* gsrc, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"{m0}"(lds_addr), "v"(gsrc) : "memory");
}

template <int N>
__device__ __forceinline__ void ld_words_nt(const char* p, uint32_t* w) {
    if constexpr (N == 4) {
        w[0] = __builtin_nontemporal_load((const uint32_t*)p);
    } else if constexpr (N == 8) {
        const u32x2 v = __builtin_nontemporal_load((const u32x2*)p);
        w[0] = v.x; w[1] = v.y;
    } else {
        static_assert(N % 16 == 0, "chunk");
#pragma unroll
        for (int k = 0; k < N / 16; ++k) {
            const uint4 v = ld_nt16(p + 16 * k);
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    }
}

template <int N>
__device__ __forceinline__ void st_words(char* p, const uint32_t* w) {
    if constexpr (N == 4) {
        *(uint32_t*)p = w[0];
    } else if constexpr (N == 8) {
        *(uint2*)p = make_uint2(w[0], w[1]);
    } else {
        static_assert(N % 16 == 0, "chunk");
#pragma unroll
        for (int k = 0; k < N / 16; ++k)
            *(uint4*)(p + 16 * k) = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
    }
}

// Writes NE contiguous output elements (value e is vals[e]) in dtype DT.
template <int DT, int NE>
__device__ __forceinline__ void store_elems(char* p, const float* vals) {
    if constexpr (DT == MF_F32) {
        uint32_t w[NE];
#pragma unroll
        for (int e = 0; e < NE; ++e) w[e] = __float_as_uint(vals[e]);
        st_words<NE * 4>(p, w);
    } else {
        uint32_t w[NE / 2];
#pragma unroll
        for (int e = 0; e < NE / 2; ++e)
            w[e] = f32_to_bits<DT>(vals[2 * e]) | (f32_to_bits<DT>(vals[2 * e + 1]) << 16);
        st_words<NE * 2>(p, w);
    }
}

// Writes the lane's contiguous chunk of 4*VCH output elements.
template <int DT, int VCH>
__device__ __forceinline__ void store_out_chunk(char* p, const float* vals) {
    store_elems<DT, 4 * VCH>(p, vals);
}

// ------------------------------------------------------------- split-K merge
// Partials of one 16-column tile (merge record `mg`) live in slots
// slot0 + p*sstride, p < np. A slot holds, per column, the partition's
// normalised output o_p / l_p in the launch's element type (column c at
// element c*part_dstride), then 16 running maxima m_p and 16 sums l_p (fp32,
// at float 16*part_dstride). The merged output is
// sum_p w_p l_p (o_p / l_p) / sum_p w_p l_p with w_p = 2^(m_p - max_p m_p).
// A normalised output is a convex combination of V rows, so it keeps the
// output type's range; 16-bit partials halve the bytes written and merged
// against fp32 ones, for one more rounding to that type.
template <int DT>
__device__ __forceinline__ char* partial_out(const AttnArgs& a, int64_t slot, int col, int elem) {
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    return (char*)(a.partials + slot * (16 * (int64_t)(a.part_dstride + 2))) +
           ((int64_t)col * a.part_dstride + elem) * ES;
}
__device__ __forceinline__ float* partial_ml(const AttnArgs& a, int64_t slot) {
    return a.partials + slot * (16 * (int64_t)(a.part_dstride + 2)) + 16 * a.part_dstride;
}

// merge_range accumulates partitions p0, p0+pinc, ... relative to their own
// maximum `mx` (lane (g, j): column j, head_dim range [4g*VCH, 4g*VCH+4*VCH)).
// Partitions go four at a time with every load of a batch issued before any
// is used (a batch past the last partition loads only what exists; the
// condition is wave-uniform), and the running maximum moves batch to batch:
// a merge of n partitions per wave costs ceil(n/4) memory round trips.
template <int DT, int DP>
__device__ __forceinline__ void merge_range(const AttnArgs& a, const int32_t* mg, int p0, int pinc, int j,
                                            int dbase, float& mx, float& L, float (&o)[DP / 4]) {
    constexpr int VCH = DP / 16;
    constexpr int B = 4;
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    constexpr int NW = 4 * VCH * ES / 4;  // words of the lane's chunk
    const int np = mg[3], slot0 = mg[4], sstride = mg[5];
    mx = kMinM;
    L = 0.f;
#pragma unroll
    for (int e = 0; e < 4 * VCH; ++e) o[e] = 0.f;
    for (int p = p0; p < np; p += B * pinc) {
        uint32_t raw[B][NW];
        float mb[B], lb[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if (p + b * pinc < np) {
                const int64_t slot = slot0 + (int64_t)(p + b * pinc) * sstride;
                ld_words<4 * VCH * ES>(partial_out<DT>(a, slot, j, dbase), raw[b]);
                const float* ml = partial_ml(a, slot);
                mb[b] = ml[j];
                lb[b] = ml[16 + j];
            } else {
#pragma unroll
                for (int e = 0; e < NW; ++e) raw[b][e] = 0u;
                mb[b] = kMinM;
                lb[b] = 0.f;
            }
        }
        float bm = mx;
#pragma unroll
        for (int b = 0; b < B; ++b) bm = fmaxf(bm, mb[b]);
        const float keep = __builtin_amdgcn_exp2f(mx - bm);
        L *= keep;
#pragma unroll
        for (int e = 0; e < 4 * VCH; ++e) o[e] *= keep;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float wl = __builtin_amdgcn_exp2f(mb[b] - bm) * lb[b];
            L += wl;
#pragma unroll
            for (int e = 0; e < 4 * VCH; ++e) {
                float v;
                if constexpr (DT == MF_F32) v = __uint_as_float(raw[b][e]);
                else v = bits_to_f32<DT>((raw[b][e >> 1] >> (16 * (e & 1))) & 0xffffu);
                o[e] += wl * v;
            }
        }
        mx = bm;
    }
}

// Output row/head of column tile ct's column j, or false for a padding column.
// mg: a merge record (s, h, column tile, parts, slot0, slot stride, first row,
// rows)
__device__ __forceinline__ bool merge_column(const AttnArgs& a, const int32_t* mg, int j, int& prow, int& qhead) {
    const int h = mg[1], ct = mg[2];
    const int row0 = mg[6];
    const int ncols = mg[7] * a.G;
    const int cidx = ct * 16 + j;
    if (cidx >= ncols) return false;
    const int r = cidx / a.G;
    prow = row0 + r;
    if (a.row_map) prow = a.row_map[prow];
    qhead = h * a.G + (cidx - r * a.G);
    return true;
}

// Single-wave merge of one record (used by the fused in-kernel merge).
template <int DT, int DP>
__device__ __forceinline__ void merge_tile(const AttnArgs& a, const int32_t* mg, int g, int j) {
    constexpr int VCH = DP / 16;
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    int prow, qhead;
    const int dbase = 4 * g * VCH;
    if (!merge_column(a, mg, j, prow, qhead) || dbase >= a.head_dim) return;
    float mx, L, o[4 * VCH];
    merge_range<DT, DP>(a, mg, 0, 1, j, dbase, mx, L, o);
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int e = 0; e < 4 * VCH; ++e) o[e] *= inv;
    store_out_chunk<DT, VCH>(a.out + ((int64_t)prow * a.o_sr + (int64_t)qhead * a.o_sh + dbase) * ES, o);
}

// -------------------------------------------------------------- main kernel
// Waves per SIMD the register allocator must leave room for: two where the
// kernel fits in 256 registers without spilling (key rows up to 128 bytes,
// or up to 256 bytes for single-tile items), else one.
template <int DT, int DP, int NT>
constexpr int attn_waves_per_eu() {
    constexpr int row_bytes = DP * (DT == MF_F32 ? 4 : 2);
    return (row_bytes <= 128 || (row_bytes <= 256 && NT == 1)) ? 2 : 1;
}

// Register buffers of the single-column-tile key pipeline: the tile being
// processed plus the two in flight. Measured on MI355X for 128-byte rows
// (bf16 D 64): four and six buffers were no faster than three, and eight
// slower (they cost waves per SIMD); a 256-byte row's buffer is 32 registers,
// and three fit the two-waves-per-SIMD budget.
// One launch for plans holding both single-tile and wide items (see
// attn_mixed_kernel); 0 launches them one after the other.
#ifndef MF_MIXED_LAUNCH
#define MF_MIXED_LAUNCH 1
#endif

// Tiles of extra work the planner charges to the last wave of a cooperative
// unit that holds a multi-row sequence's last tile. Measured on C3's verify
// layer (graph replays): 0 13.2 us, 2 12.96-12.99, 4 12.93-12.94, 6
// 12.36-12.37, 8 12.34-12.37, 10 13.22-13.24, 12 13.18-13.19, 16 13.0. In an
// instrumented build's timeline those waves started their key loop 1.1 us
// after the unit's other waves and ran the boundary and in-flight tiles after
// it, while the others waited at the combine.
#ifndef MF_TAIL_WAVE_TILES
#define MF_TAIL_WAVE_TILES 6
#endif

#ifndef MF_NARROW_DEPTH
#define MF_NARROW_DEPTH 3
#endif

// LDS of the attention kernels: one dynamically sized arena per workgroup.
// A workgroup uses at most one of its two layouts -- the wide items'
// double-buffered K/V stages (workgroup-shared key loop) or the cooperative
// units' softmax states (narrow items) -- so a launch that runs both kinds of
// workgroup (attn_mixed_kernel) sizes the arena for the larger, not for both.
extern __shared__ __attribute__((aligned(16))) char attn_lds[];

// Workgroup-shared prefill loop: tiles per LDS stage, and stage buffers (the
// stage being computed plus the ones in flight) for 128-byte rows. Measured
// on the C2 engine layer (and the prefill items alone, between events):
// 2 x 4 tiles 48.8-49.0 us (35.4-35.8), 4 x 2 50.3 (36.3-36.5), 3 x 3
// 49.1-49.4 (36.2-36.4), 3 x 2 49.6-50.1 (36.2-36.5), 3 x 4 55.4-55.6 (48 KB
// of LDS: three workgroups per CU). More tiles in flight do not help: the
// loop does not wait on memory.
#ifndef MF_WIDE_TPS128
#define MF_WIDE_TPS128 4
#endif
#ifndef MF_WIDE_NBUF128
#define MF_WIDE_NBUF128 2
#endif
constexpr int wide_tps(int rb) { return rb == 128 ? MF_WIDE_TPS128 : 2; }
constexpr int wide_nbuf(int rb) { return rb == 128 ? MF_WIDE_NBUF128 : 2; }
template <int DT, int DP>
constexpr int wide_lds_bytes() {
    constexpr int rb = DP * (DT == MF_F32 ? 4 : 2);
    if constexpr (DT == MF_F32) return 0;  // the workgroup-shared loop is 16-bit only
    else return wide_nbuf(rb) * wide_tps(rb) * 32 * rb + 16;
}
template <int DP>
constexpr int coop_lds_bytes() {
    return (kWaves * 4 * (DP / 16) * 64 + 2 * kWaves * 16) * 4;
}
template <int DT, int DP, int NT, bool FAST>
constexpr int attn_lds_bytes() {
    if constexpr (NT == 1) return coop_lds_bytes<DP>();
    else return FAST ? wide_lds_bytes<DT, DP>() : 0;
}

// The body of one workgroup of the attention kernel: `block` is its index
// among the workgroups that run items of this column-tile width.
// TAIL: a written-in-flight launch (compiled apart, so the other launches
// keep their register budget).
template <int DT, int DP, int NT, bool FAST, bool TAIL = false>
__device__ __forceinline__ void attn_body(const AttnArgs& a, const int block) {
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    constexpr int EPL = 16 / ES;      // elements per 16-byte chunk
    constexpr int NL = DP * ES / 64;  // 16-byte K/Q chunks per lane
    constexpr int VCH = DP / 16;      // V elements per lane per key (= d tiles)
    constexpr int VB = VCH * ES;      // bytes of one lane's V chunk
    constexpr int VWD = VB / 4;       // 32-bit words of one lane's V chunk
    static_assert(NL >= 1 && VWD >= 1, "head_dim too small for this dtype");
    constexpr float kNegInf = -__builtin_huge_valf();

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = block * kWaves + wave;
    // The item carries its sequence's first row, row count and kv length (the
    // planner's copies of cu_seqlens / kv_lens), so nothing waits on loading
    // them before the row positions and block table are fetched.
    const int32_t* it = a.items + (int64_t)item * MF_PLAN_ITEM_INTS;
    int4 iv0, iv1, iv2;
    if constexpr (NT == 1) {
        // Single-tile items load their item before the count check, together
        // with the argument block that the check reads (the item list's
        // address needs no argument load when it is preloaded), instead of
        // one round trip after it. The item is in bounds past the live count:
        // plans fill whole workgroups and counted launches size the list by
        // its capacity. The empty asm keeps the loads ahead of the check.
        // Wide items keep the order below: their setup issues the item with
        // the workgroup's other items' keys in one batch after the check.
        iv0 = *(const int4*)it;
        iv1 = *(const int4*)(it + 4);
        iv2 = *(const int4*)(it + 8);
        asm volatile("" ::"s"(iv0.x), "s"(iv0.y), "s"(iv0.z), "s"(iv0.w), "s"(iv1.x), "s"(iv1.y), "s"(iv1.z),
                     "s"(iv1.w), "s"(iv2.x), "s"(iv2.y), "s"(iv2.z), "s"(iv2.w));
        // ... and so do the argument fields the next batch of loads (block
        // table, row positions, Q) is addressed from, which otherwise come
        // from argument cache lines fetched after the check
        asm volatile("" ::"s"(a.block_tables), "s"(a.bt_stride), "s"(a.positions), "s"(a.pool_lens), "s"(a.q),
                     "s"(a.q_sr), "s"(a.q_sh), "s"(a.G), "s"(a.row_map), "s"(a.q_sign));
    }
    const int num_items = a.dev_count ? *a.dev_count : a.num_items;
    if (item >= num_items) return;
    if constexpr (NT != 1) {
        iv0 = make_int4(it[0], it[1], it[2], it[3]);
        iv1 = make_int4(it[4], it[5], it[6], it[7]);
        iv2 = make_int4(it[8], it[9], it[10], it[11]);
    }
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;  // 16-lane group: MFMA k-group / output row group
    const int j = lane & 15;  // MFMA column (query column) and A-row (key) index

    const int s = iv0.x, h = iv0.y, c0 = iv0.z, nct = iv0.w;
    const int kt0 = iv1.x, kt1 = iv1.y, pslot = iv1.z;
    const int row0 = iv2.x;
    const int ncols = iv2.y * a.G;
    const int kv_len = iv2.z;
    // Keys below pool_len are in the pool; the rest are in-flight rows of the
    // sequence's own new tokens (a verify pass: pool_lens; a written-in-flight
    // step: everything past the keys before the sequence's rows).
    const bool inflight = TAIL || a.pool_lens != nullptr;
    const int pool_len = TAIL ? kv_len - iv2.y : (a.pool_lens != nullptr ? a.pool_lens[s] : kv_len);
    const int D = a.head_dim;

    // The loads that need nothing but the item go out together -- block-table
    // entries first (loads retire in issue order, and the first K/V tiles
    // wait only on them), then row positions, then Q -- so the setup costs
    // one round trip before the K/V stream starts, not three.
    //
    // ---- block-table entries of the item's tiles, two per lane (tile kt0+l
    // and kt0+64+l; fast path, at most kMaxItemTiles), read back with
    // readlane. On a verify pass
    // that is every tile holding a pool key (the boundary tile included);
    // pool_end is the end of the tiles lying wholly in the pool.
    const int tbl_end = inflight ? max(kt0, min(kt1, (pool_len + 15) >> 4)) : kt1;
    const int pool_end = inflight ? max(kt0, min(kt1, pool_len >> 4)) : kt1;
    int tbl = 0, tbl_hi = 0;
    const int tbl_base = kt0;
    if constexpr (FAST) {
        // Every lane loads (a clamped entry past the item's tiles, entry 0 of
        // the row for an item without tiles; only entries of the item's own
        // tiles are ever read back), so no branch skips a load and nothing
        // consumes the values before the other setup loads are issued: the
        // count of loads in flight is the same on every path and later waits
        // stay exact.
        const int idx = kt0 + lane;
        const int32_t* row = a.block_tables + (int64_t)s * a.bt_stride;
        const bool any = tbl_end > kt0;
        tbl = row[any ? min(idx, tbl_end - 1) : 0];
        if constexpr (kMaxItemTiles > 64) tbl_hi = row[any ? min(idx + 64, tbl_end - 1) : 0];
    }
    // physical block of the item's tile i (wave-uniform i)
    auto tbl_at = [&](int i) -> int {
        const int lo = __builtin_amdgcn_readlane(tbl, i & 63);
        if constexpr (kMaxItemTiles > 64) return i < 64 ? lo : __builtin_amdgcn_readlane(tbl_hi, i & 63);
        return lo;
    };

    // ---- columns owned by this lane (one per tile)
    int prow[NT], qhead[NT], qpos[NT];
    bool qvalid[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        // padding columns read row0's position and query (unconditional
        // loads, results discarded)
        const int cidx = (c0 + nt) * 16 + j;
        const bool valid = nt < nct && cidx < ncols;
        const int r = valid ? cidx / a.G : 0;
        const int gq = valid ? cidx - r * a.G : 0;
        int pr = row0 + r;
        if (a.row_map) pr = a.row_map[pr];
        // the low word of the little-endian int64 position (what the int
        // conversion keeps): a 64-bit load's unused high register would be
        // reused as a temporary, and that write waits for the load
        const int pos = reinterpret_cast<const int32_t*>(a.positions)[2 * (int64_t)pr];
        prow[nt] = pr;
        qhead[nt] = h * a.G + gq;
        qpos[nt] = valid ? pos : -1;
        qvalid[nt] = valid;
    }

    // ---- Q fragments (MFMA B operand of S^T = K Q^T): lane (g, j) holds
    // column j's head_dim chunk (c*4 + g) for c < NL.
    uint4 qf[NT][NL];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int d0 = (c * 4 + g) * EPL;
            // A padding column holds row0's query (its scores are computed
            // and never stored; every column has its own softmax state).
            uint4 v = make_uint4(0, 0, 0, 0);
            if (FAST || d0 < D)  // the fast path has head_dim == DP: every chunk exists
                v = *(const uint4*)(a.q + ((int64_t)prow[nt] * a.q_sr + (int64_t)qhead[nt] * a.q_sh + d0) * ES);
            qf[nt][c] = make_uint4(v.x ^ a.q_sign, v.y ^ a.q_sign, v.z ^ a.q_sign, v.w ^ a.q_sign);
        }
    }

    // General path: address of key `key`'s row for this kv head, or null.
    auto key_row = [&](const char* pool, const char* inflight, int key) -> const char* {
        if (key >= kv_len) return nullptr;
        if (key < pool_len) {
            const int blk = key / a.block_size;
            const int off = key - blk * a.block_size;
            const int phys = a.block_tables[(int64_t)s * a.bt_stride + blk];
            return pool + ((int64_t)phys * a.p_sb + (int64_t)off * a.p_ss + (int64_t)h * a.p_sh) * ES;
        }
        int nr = row0 + (key - pool_len);
        if (a.row_map) nr = a.row_map[nr];
        return inflight + ((int64_t)nr * a.n_sr + (int64_t)h * a.n_sh) * ES;
    };

    // byte offsets of this lane's K chunk (key j, chunk g) and V chunk (keys
    // 4g.., head_dim j*VCH..) inside one block of one kv head
    const uint32_t k_lane_off = (uint32_t)(((int64_t)j * a.p_ss + g * EPL) * ES);
    const uint32_t v_row_bytes = (uint32_t)(a.p_ss * ES);
    const uint32_t v_lane_off = (uint32_t)(((int64_t)(4 * g) * a.p_ss + j * VCH) * ES);
    // Per-key loads of tile kt (the verify boundary and in-flight tiles, and
    // every tile off the fast path). On the fast path a tile's pool keys all
    // lie in one block, whose entry is already in tbl.
    // has_map: the launch has a row map (a compile-time copy of each case:
    // with the map read behind a runtime test, the five row lookups below
    // each ended in a wait for every load in flight, row map or not -- on a
    // verify pass the boundary tile's wave then started its key loop 2.3 us
    // after the others and held up its cooperative unit)
    auto load_general_m = [&](int kt, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD], auto has_map) {
        int phys = 0;
        if constexpr (FAST) phys = kt < tbl_end ? tbl_at(kt - tbl_base) : 0;
        auto row = [&](const char* pool, const char* inflight, int key) -> const char* {
            if constexpr (FAST) {
                if (key >= kv_len) return nullptr;
                if (key < pool_len)
                    return pool + ((int64_t)phys * a.p_sb + (int64_t)(key & 15) * a.p_ss + (int64_t)h * a.p_sh) * ES;
                int nr = row0 + (key - pool_len);
                if constexpr (decltype(has_map)::value) nr = a.row_map[nr];
                return inflight + ((int64_t)nr * a.n_sr + (int64_t)h * a.n_sh) * ES;
            } else {
                return key_row(pool, inflight, key);
            }
        };
        const char* kp = row(a.k_pool, a.new_k, kt * 16 + j);
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int d0 = (c * 4 + g) * EPL;
            kf[c] = (kp && d0 < D) ? *(const uint4*)(kp + (int64_t)d0 * ES) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const char* vp = row(a.v_pool, a.new_v, kt * 16 + 4 * g + r);
            if (vp && j * VCH < D) {
                ld_words<VB>(vp + (int64_t)j * VCH * ES, vf[r]);
            } else {
#pragma unroll
                for (int w = 0; w < VWD; ++w) vf[r][w] = 0;
            }
        }
    };
    auto load_general = [&](int kt, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD]) {
        if (FAST && a.row_map) load_general_m(kt, kf, vf, std::true_type{});
        else load_general_m(kt, kf, vf, std::false_type{});
    };
    // Lane byte offsets of the V rows 4g..4g+3 inside a block, computed once.
    uint32_t v_off[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v_off[r] = v_lane_off + (uint32_t)r * v_row_bytes;
    // A dummy load (a prefetch slot past the item's last tile) keeps the
    // chunk offsets but drops the lane offsets: the wave reads the block's
    // first few lines instead of the whole tile again. `none` (wave-uniform):
    // the item has no pool tile at all, and the dummy reads the start of Q,
    // which every call has.
    auto load_tile = [&](int kt, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD], bool dummy = false, bool none = false) {
        if constexpr (FAST) {
            // block base is wave-uniform (scalar registers); the lane's byte
            // offsets inside a block never change
            const int phys = tbl_at(kt - tbl_base);
            const int64_t boff = ((int64_t)phys * a.p_sb + (int64_t)h * a.p_sh) * ES;
            const char* kb = none ? a.q : a.k_pool + boff;
            const char* vb = none ? a.q : a.v_pool + boff;
            const uint32_t sel = (dummy || none) ? 0u : 0xffffffffu;
            const uint32_t ko = k_lane_off & sel;
            if constexpr (NT == 1 && DP * ES >= 256) {
                // non-temporal only for rows of 256 bytes or more: measured
                // faster there (bf16 D 128) and slower for 128-byte rows
#pragma unroll
                for (int c = 0; c < NL; ++c) kf[c] = ld_nt16(kb + ko + c * 4 * 16);
#pragma unroll
                for (int r = 0; r < 4; ++r) ld_words_nt<VB>(vb + (v_off[r] & sel), vf[r]);
            } else {
#pragma unroll
                for (int c = 0; c < NL; ++c) kf[c] = *(const uint4*)(kb + ko + c * 4 * 16);
#pragma unroll
                for (int r = 0; r < 4; ++r) ld_words<VB>(vb + (v_off[r] & sel), vf[r]);
            }
        } else {
            load_general(kt, kf, vf);
        }
    };

    // The first NB-1 tiles of a single-column-tile (decode) item go out with
    // the setup loads: positions only trim the item's key range, and these
    // tiles lie in it whenever the item has any. Slots past the item's tiles
    // take a one-line dummy load.
    // The loads are unconditional -- an item without pool tiles issues dummy
    // ones -- so the count of loads in flight is the same on every path and
    // the first use of Q waits for Q alone, not for these tiles too.
    constexpr int NB = NT == 1 ? MF_NARROW_DEPTH : 2;
    uint4 kR[NB][NL];
    uint32_t vR[NB][4][VWD];
    if constexpr (FAST && NT == 1) {
        const bool none = kt0 >= pool_end;
#pragma unroll
        for (int i = 0; i < NB - 1; ++i)
            load_tile(max(kt0, min(kt0 + i, pool_end - 1)), kR[i], vR[i], kt0 + i > pool_end - 1, none);
    }

    // ---- workgroup-shared key loop, first part. Wide items whose workgroup
    // shares one key range (the planner packs wide items that way, one column
    // group per wave) stage each 16-key K/V tile in LDS for all four waves
    // (the loop itself follows below). Its first stage needs only the item and
    // the block table, so it is fetched here, before the row positions are
    // waited for: the setup then costs the block table's round trip and the
    // stage's, overlapped with the positions', instead of three in a row
    // (the positions only trim how far the range is read; the first stage is
    // bounded by the item's range instead). On a written-in-flight step the
    // loop also takes the tiles holding new rows, reading each lane's key from
    // the pool or from the new rows.
    constexpr int RB = DP * ES;             // bytes of one key row
    constexpr int NCH = RB / 16;            // 16-byte chunks per row
    constexpr int STAGE = 32 * RB;          // K tile, then V tile
    constexpr int NI = (STAGE + kWaves * 1024 - 1) / (kWaves * 1024);  // 16-byte loads per lane per tile
    // Tiles per LDS stage: each barrier and each refill covers TPS
    // tiles, so a refill has TPS tiles of compute to arrive in.
    // Measured on the C2 prefill items (bf16, D 64): 1 tile 42.0 us,
    // 2 tiles 40.3 us, 4 tiles 39.2 us. Four would take the D 32
    // kernel past 128 registers (three waves per SIMD), so other row
    // sizes use two.
    constexpr int TPS = wide_tps(RB);
    constexpr int NBUF = wide_nbuf(RB);
    static_assert(NBUF >= 2 && NBUF <= 5 && (MF_WIDE_DIRECT_LDS || NBUF == 2), "stage buffers");
    // this lane's 16 bytes of each tile: LDS byte base + lane*16 of
    // piece (i*4 + wave) mod STAGE, and the matching pool offset inside
    // the block (vector types rather than arrays keep them in registers)
    typedef uint32_t offs_t __attribute__((ext_vector_type(NI)));
    typedef uint32_t regs_t __attribute__((ext_vector_type(4 * NI * TPS)));
    bool wg_shared = false;
    if constexpr (FAST && DT != MF_F32 && NT > 1) {
        if ((block + 1) * kWaves <= num_items) {
            // The four items' (sequence, kv head, key range) are loaded
            // together and compared without short-circuit: chained && made
            // the compiler issue one load per comparison, each behind a full
            // wait -- twelve round trips before the first K/V fetch, which
            // beside a decode workgroup's streams took 12.7 us of a prefill
            // workgroup's setup (4.0 us alone).
            const int32_t* i0 = a.items + (int64_t)block * kWaves * MF_PLAN_ITEM_INTS;
            int32_t key[kWaves][4];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const int32_t* iw = i0 + w * MF_PLAN_ITEM_INTS;
                key[w][0] = iw[0];
                key[w][1] = iw[1];
                key[w][2] = iw[4];
                key[w][3] = iw[5];
            }
            bool same = true;
#pragma unroll
            for (int w = 1; w < kWaves; ++w)
                same = same & (key[w][0] == key[0][0]) & (key[w][1] == key[0][1]) & (key[w][2] == key[0][2]) &
                       (key[w][3] == key[0][3]);
            wg_shared = same;
        }
    }
    const bool shared_inflight = TAIL && wg_shared;
    offs_t src_off, key_of, piece_of;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int base = ((i * kWaves + wave) * 1024) % STAGE;
        const bool isv = base >= 16 * RB;
        const int p2 = (isv ? base - 16 * RB : base) + lane * 16;
        const int key = p2 / RB, slot = (p2 % RB) >> 4;
        const int q = isv ? slot : (slot ^ (key & (NCH - 1)));
        src_off[i] = (uint32_t)key * v_row_bytes + (uint32_t)q * 16;
        key_of[i] = (uint32_t)key;
        piece_of[i] = (uint32_t)q * 16;
    }
    // in-flight key k of this kv head: K row at ibase + k * irow_bytes,
    // its V row iv_off bytes on (so the loop holds three numbers, not
    // both tensors and their strides)
    const char* ibase = a.new_k;
    int64_t irow_bytes = 0, iv_off = 0;
    if (shared_inflight) {
        irow_bytes = a.n_sr * ES;
        ibase = a.new_k + ((int64_t)(row0 - pool_len) * a.n_sr + (int64_t)h * a.n_sh) * ES;
        iv_off = a.new_v - a.new_k;
    }
    // Tiles the fetches clamp to: the item's range for the first stage, the
    // workgroup's last read tile once the positions are in.
    int fetch_end = kt1;
    // Loads are unconditional (a wave without a piece of a small tile
    // re-reads another wave's piece and does not store it; tiles past
    // the range re-read the last one): a conditional load would make
    // every later wait drain all loads.
    auto fetch = [&](int t0, regs_t& r) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < TPS; ++u) {
            const int t = min(t0 + u, fetch_end - 1);
            const int phys = tbl_at(t - kt0);
            const int64_t boff = ((int64_t)phys * a.p_sb + (int64_t)h * a.p_sh) * ES;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int base = ((i * kWaves + wave) * 1024) % STAGE;
                const bool isv = base >= 16 * RB;
                const char* src = (isv ? a.v_pool : a.k_pool) + boff + src_off[i];
                if (shared_inflight) {
                    // this lane's key is a new row of the sequence
                    // (clamped to its last row past the context; those
                    // keys are masked and their V cleared)
                    const int key = t * 16 + (int)key_of[i];
                    const char* isrc = ibase + (isv ? iv_off : 0) +
                                       (int64_t)min(key, kv_len - 1) * irow_bytes + piece_of[i];
                    src = key >= pool_len ? isrc : src;
                }
                const uint4 v = *(const uint4*)src;
                const int w = 4 * (u * NI + i);
                r[w] = v.x;
                r[w + 1] = v.y;
                r[w + 2] = v.z;
                r[w + 3] = v.w;
            }
        }
    };
    // The same stage straight into LDS buffer `buf` (direct form): each wave
    // writes its 1 KB pieces of each tile; a wave without a piece of a small
    // tile loads nothing.
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)attn_lds;
    auto dfetch = [&](int t0, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < TPS; ++u) {
            const int t = min(t0 + u, fetch_end - 1);
            const int phys = tbl_at(t - kt0);
            const int64_t boff = ((int64_t)phys * a.p_sb + (int64_t)h * a.p_sh) * ES;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int base = (i * kWaves + wave) * 1024;
                if (base >= STAGE) continue;
                const bool isv = base >= 16 * RB;
                const char* src = (isv ? a.v_pool : a.k_pool) + boff + src_off[i];
                if (shared_inflight) {
                    const int key = t * 16 + (int)key_of[i];
                    const char* isrc = ibase + (isv ? iv_off : 0) +
                                       (int64_t)min(key, kv_len - 1) * irow_bytes + piece_of[i];
                    src = key >= pool_len ? isrc : src;
                }
                ld_lds16(src, lds_base + (uint32_t)((buf * TPS + u) * STAGE + base));
            }
        }
    };
    regs_t rs;
    if constexpr (FAST && DT != MF_F32 && NT > 1) {
        if (wg_shared) {
            if constexpr (MF_WIDE_PRIO > 0) __builtin_amdgcn_s_setprio(MF_WIDE_PRIO);
            if (kt1 > kt0) {
                if constexpr (MF_WIDE_DIRECT_LDS) dfetch(kt0, 0);
                else fetch(kt0, rs);
            }
        }
    }

    int maxpos = -1;
    int minpos = INT_MAX;  // over the item's real columns
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        maxpos = max(maxpos, qpos[nt]);
        if (qvalid[nt]) minpos = min(minpos, qpos[nt]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        maxpos = max(maxpos, __shfl_xor(maxpos, off, 64));
        minpos = min(minpos, __shfl_xor(minpos, off, 64));
    }
    minpos = __builtin_amdgcn_readfirstlane(minpos);
    // last key each lane's column may see (-1 for padding columns)
    int lim[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) lim[nt] = qpos[nt] >= 0 ? min(qpos[nt], kv_len - 1) : -1;
    // Tiles past the last key any column may see are never read.
    int kt_end = min(kt1, (min(maxpos, kv_len - 1) >> 4) + 1);
    if (maxpos < 0 || kv_len <= 0) kt_end = kt0;
    kt_end = __builtin_amdgcn_readfirstlane(kt_end);

    // m: running max of the scaled scores (log2 units); thr: the raw score
    // above which a column's running max must move, (m + kLazyLog2) / scale.
    float m[NT], l[NT], thr[NT];
    f32x4 acc[NT][VCH];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m[nt] = kMinM;
        thr[nt] = (kMinM + kLazyLog2) * a.inv_scale_log2;
        l[nt] = 0.f;
#pragma unroll
        for (int c = 0; c < VCH; ++c) acc[nt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // K: lane (g, j) loads key j's head_dim chunks (c*4 + g).
    // V: lane (g, j) loads keys 4g..4g+3, head_dim elements [j*VCH, j*VCH+VCH).
    // FAST path (16-token blocks, head_dim == DP): every
    // load is unconditional, so the compiler can keep the next tile's loads in
    // flight while the current tile is processed.
    // Tiles [kt0, fast_end) run through the pipelined loop. On the fast path
    // with in-flight keys (a verify pass) that is only the tiles lying wholly
    // in the pool; the one or two tiles holding the boundary and the in-flight
    // candidates follow through the general per-key loads.
    int fast_end = kt_end;
    if constexpr (FAST) {
        if (inflight && !shared_inflight) fast_end = max(kt0, min(kt_end, pool_len >> 4));
    }
    // Per-tile work is branch-free apart from wave-uniform decisions: every
    // column tile's MFMAs run (tiles past nct hold zero queries and are never
    // stored), and masking is a select, so the scheduler sees one straight
    // block per tile, in four parts: scores, the lazy rescale, exponentials
    // and the PV product.
    //
    // Slots past the context in the last block may hold anything, NaN
    // included; p = 0 there, but 0 * NaN is NaN, so clear them.
    auto clear_v_tail = [&](int kt, uint32_t (&vf)[4][VWD]) {
        if constexpr (FAST) {
            if ((kt + 1) * 16 > kv_len) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool live = kt * 16 + 4 * g + r < kv_len;
#pragma unroll
                    for (int w = 0; w < VWD; ++w) vf[r][w] = live ? vf[r][w] : 0u;
                }
            }
        }
    };
    // S^T = K Q^T for every column tile (lane (g, j): keys 4g..4g+3 of
    // column j), masked. Scores stay raw; the scale is applied inside the
    // exponent, p = 2^(s * scale - m), one fma.
    auto scores = [&](int kt, const uint4 (&kf)[NL], float (&sv)[NT][4]) {
        f32x4 st[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            st[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NL; ++c) st[nt] = mfma_qk<DT>(kf[c], qf[nt][c], st[nt]);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[nt][r] = st[nt][r];
        // Every key of a tile wholly inside the context and at or before every
        // column's position is visible to all columns: no mask to apply.
        if (!(kt * 16 + 15 <= minpos && (kt + 1) * 16 <= kv_len)) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sv[nt][r] = kt * 16 + 4 * g + r <= lim[nt] ? sv[nt][r] : kNegInf;
        }
    };
    // Lazy rescaling: a column's running max m moves (and l, acc are
    // rescaled) only when one of its scores exceeds m by more than
    // kLazyLog2, so p = 2^(s - m) stays below 2^kLazyLog2; l and acc always
    // share the m they were built with, so the result is the same softmax.
    // Each lane tests its own four scores; the max across the column's
    // four lane groups is only formed when some lane asks for a move.
    auto needs_rescale = [&](const float (&sv)[NT][4], float (&lmax)[NT]) -> bool {
        bool grow = false;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            lmax[nt] = fmax_prop(fmax_prop(sv[nt][0], sv[nt][1]), fmax_prop(sv[nt][2], sv[nt][3]));
            grow |= lmax[nt] > thr[nt];
        }
        return __builtin_amdgcn_ballot_w64(grow) != 0;
    };
    auto rescale = [&](const float (&lmax)[NT]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float mn = fmaxf(m[nt], group_max4(lmax[nt]) * a.scale_log2);
            const float alpha = __builtin_amdgcn_exp2f(m[nt] - mn);
            l[nt] *= alpha;
#pragma unroll
            for (int c = 0; c < VCH; ++c) acc[nt][c] *= alpha;
            m[nt] = mn;
            thr[nt] = (mn + kLazyLog2) * a.inv_scale_log2;
        }
    };
    // p = 2^(s * scale - m) against the current running max, l += row sums;
    // packed to the 16-bit dtype for the PV MFMA (fp32 kept as is).
    auto exps = [&](const float (&sv)[NT][4], uint2 (&p16)[NT], float (&p32)[NT][4]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[nt][r], a.scale_log2, -m[nt]));
            l[nt] += (p[0] + p[1]) + (p[2] + p[3]);
            if constexpr (DT == MF_F32) {
#pragma unroll
                for (int r = 0; r < 4; ++r) p32[nt][r] = p[r];
            } else if constexpr (DT == MF_BF16) {
                // hardware round-to-nearest-even pack (v_cvt_pk_bf16_f32)
                p16[nt] = make_uint2(
                    __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){p[0], p[1]}, bf16x2)),
                    __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){p[2], p[3]}, bf16x2)));
            } else {
                p16[nt] = make_uint2(f32_to_bits<DT>(p[0]) | (f32_to_bits<DT>(p[1]) << 16),
                                     f32_to_bits<DT>(p[2]) | (f32_to_bits<DT>(p[3]) << 16));
            }
        }
    };
    // MFMA A operand (16-bit) of head_dim tile c: element c of keys
    // 4g..4g+3, the low (c even) or high halves of word c/2, paired by byte
    // permutes. Row i of tile c is head_dim element i*VCH + c.
    auto va16 = [&](const uint32_t (&vf)[4][VWD], int c) -> uint2 {
        const int wd = c >> 1;
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        return make_uint2(__builtin_amdgcn_perm(vf[1][wd], vf[0][wd], sel),
                          __builtin_amdgcn_perm(vf[3][wd], vf[2][wd], sel));
    };
    // O^T += V^T P^T for one tile, one MFMA per 16-row head_dim tile c.
    auto pv = [&](const uint32_t (&vf)[4][VWD], const uint2 (&p16)[NT], const float (&p32)[NT][4]) {
#pragma unroll
        for (int c = 0; c < VCH; ++c) {
            if constexpr (DT == MF_F32) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float va = __uint_as_float(vf[r][c]);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[nt][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, p32[nt][r], acc[nt][c], 0, 0, 0);
                }
            } else {
                const uint2 va = va16(vf, c);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[nt][c] = mfma_pv16<DT>(va, p16[nt], acc[nt][c]);
            }
        }
    };
    auto process = [&](int kt, const uint4 (&kf)[NL], uint32_t (&vf)[4][VWD]) {
        clear_v_tail(kt, vf);
        float sv[NT][4];
        scores(kt, kf, sv);
        float lmax[NT];
        if (needs_rescale(sv, lmax)) rescale(lmax);
        uint2 p16[NT];
        float p32[NT][4];
        exps(sv, p16, p32);
        pv(vf, p16, p32);
    };

    // ---- key loops. Single-column-tile items (decode, verify) stream their
    // own tiles through the NB-buffer register ring below; wide items either
    // share each tile through LDS (next) or, pooled four to a workgroup with
    // unrelated items, stream their own tiles through two buffers. Every
    // prefetch is unconditional (past the end it is a dummy or a clamped
    // re-read) because a conditional load makes the compiler drain every
    // outstanding load at the join and serialises the pipeline.
    // ---- workgroup-shared key loop (16-bit wide items on the fast path).
    // When the workgroup's four items cover one (sequence, kv head, key
    // range) -- the planner packs wide items that way, one column group per
    // wave -- every 16-key K/V tile is fetched once for the workgroup (a
    // quarter per wave, 16 bytes per lane) and staged in LDS, and each wave
    // reads its MFMA fragments from LDS. That takes the four-fold re-reads of
    // each tile off the texture path, which is what limits the per-wave loop
    // on prefill. Tiles move in stages of TPS: loads run one stage ahead in
    // registers; LDS holds two stages (a stage is written after the barrier
    // that retires the previous reads of its buffer). Each K row's 16-byte
    // chunks are stored xor-swizzled by key, so the fragment reads (16 keys x
    // one chunk) hit distinct banks; V rows are read 16 lanes to a row,
    // conflict-free. One barrier per stage.
    if constexpr (FAST && DT != MF_F32 && NT > 1) {
        if (wg_shared) {
            static_assert(wide_lds_bytes<DT, DP>() == NBUF * TPS * STAGE + 16, "LDS arena layout");
            char* smem = attn_lds;
            int* s_end = reinterpret_cast<int*>(attn_lds + NBUF * TPS * STAGE);
            if (lane == 0) s_end[wave] = fast_end;
            __syncthreads();
            const int wg_end = __builtin_amdgcn_readfirstlane(
                max(max(s_end[0], s_end[1]), max(s_end[2], s_end[3])));
            const int n = wg_end - kt0;
            fetch_end = wg_end;
            auto stash = [&](const regs_t& r, int buf) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < TPS; ++u) {
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
                        const int base = (i * kWaves + wave) * 1024;
                        const int w = 4 * (u * NI + i);
                        if (base < STAGE)
                            *(uint4*)(smem + (buf * TPS + u) * STAGE + base + lane * 16) =
                                make_uint4(r[w], r[w + 1], r[w + 2], r[w + 3]);
                    }
                }
            };
            auto sync = [&]() {
                // this wave's LDS reads and writes are done, then all waves'
                __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            };
            auto wait_stages = [&](int pending) {
                // this wave's direct loads done, but for the last `pending` stages
                if (pending <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                else if (pending == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(TPS * NI) : "memory");
                else if (pending == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * TPS * NI) : "memory");
                else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * TPS * NI) : "memory");
            };
            if (n > 0 && MF_WIDE_DIRECT_LDS) {
                // NBUF buffers: stage u is computed while stages u+1 ..
                // u+NBUF-1 arrive; after the barrier that ends stage u (every
                // wave is done reading its buffer, and has waited for its own
                // pieces of stage u+1), stage u+NBUF is issued into it.
                const int nst = (n + TPS - 1) / TPS;
                // the first stage went out with the setup loads
                for (int s = 1; s < NBUF; ++s)
                    if (s < nst) dfetch(kt0 + s * TPS, s);
                wait_stages(min(NBUF - 1, nst - 1));
                sync();
                int buf = 0;
                for (int u = 0; u < nst; ++u) {
                    // fragments of staged tile v (K rows swizzled, V rows plain)
                    auto frags = [&](int v, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD]) {
                        const char* stg = smem + (buf * TPS + v) * STAGE;
#pragma unroll
                        for (int c = 0; c < NL; ++c)
                            kf[c] = *(const uint4*)(stg + j * RB + (((c * 4 + g) ^ (j & (NCH - 1))) << 4));
#pragma unroll
                        for (int r = 0; r < 4; ++r) ld_words<VB>(stg + 16 * RB + (4 * g + r) * RB + j * VB, vf[r]);
                    };
#pragma unroll
                    for (int v = 0; v < TPS; ++v) {
                        const int t = kt0 + u * TPS + v;
                        if (t < fast_end) {
                            uint4 kf[NL];
                            uint32_t vf[4][VWD];
                            frags(v, kf, vf);
                            process(t, kf, vf);
                        }
                    }
                    wait_stages(min(NBUF - 2, nst - 2 - u));
                    sync();
                    if (u + NBUF < nst) dfetch(kt0 + (u + NBUF) * TPS, buf);
                    buf = buf + 1 == NBUF ? 0 : buf + 1;
                }
            } else if (n > 0) {
                // Register form (two LDS buffers): one register set in
                // flight; stage u+1 (TPS tiles) arrives during stage u's
                // compute, is stored to the other LDS buffer, and the set is
                // refilled with stage u+2.
                const int nst = (n + TPS - 1) / TPS;
                stash(rs, 0);  // the first stage, fetched with the setup loads
                fetch(kt0 + TPS, rs);
                sync();
                for (int u = 0; u < nst; ++u) {
                    // fragments of staged tile v (K rows swizzled, V rows plain)
                    auto frags = [&](int v, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD]) {
                        const char* stg = smem + ((u & 1) * TPS + v) * STAGE;
#pragma unroll
                        for (int c = 0; c < NL; ++c)
                            kf[c] = *(const uint4*)(stg + j * RB + (((c * 4 + g) ^ (j & (NCH - 1))) << 4));
#pragma unroll
                        for (int r = 0; r < 4; ++r) ld_words<VB>(stg + 16 * RB + (4 * g + r) * RB + j * VB, vf[r]);
                    };
#pragma unroll
                    for (int v = 0; v < TPS; ++v) {
                        const int t = kt0 + u * TPS + v;
                        if (t < fast_end) {
                            uint4 kf[NL];
                            uint32_t vf[4][VWD];
                            frags(v, kf, vf);
                            process(t, kf, vf);
                        }
                    }
                    if (u + 1 < nst) {
                        stash(rs, (u + 1) & 1);
                        fetch(kt0 + (u + 2) * TPS, rs);
                    }
                    sync();
                }
            }
        }
    }
    // The first tile past the pipelined range (a verify pass's boundary or
    // candidate tile) is fetched before the loop, so its per-key loads
    // overlap the pool tiles instead of following them.
    uint4 kT[NL];
    uint32_t vT[4][VWD];
    if constexpr (FAST && NT == 1) {
        if (fast_end < kt_end) load_general(fast_end, kT, vT);
    }
    if (kt0 < fast_end && !wg_shared) {
        // Ring of NB register buffers: each step issues the tile NB-1 ahead
        // into the slot freed last and processes the oldest. The loop runs
        // whole rounds of NB steps and the last n % NB tiles (already in
        // slots 0..) follow after it: an exit from inside a round would give
        // the loop a latch that some paths reach with a slot's loads still
        // in flight, and the compiler then drains every load at the top of
        // each round. Prefetches past the last tile still issue (a
        // conditional load would drain the pipeline as well), but as a
        // single line: for 256-byte rows these loads bypass L2, so a full
        // re-read would cost HBM.
        const int last = fast_end - 1;
        int kt = kt0;
        if constexpr (NT == 1) {
            if constexpr (!FAST) {
                // (fast items issued these with the setup loads)
#pragma unroll
                for (int i = 0; i < NB - 1; ++i) load_tile(min(kt0 + i, last), kR[i], vR[i]);
            }
            for (int r = (fast_end - kt0) / NB; r > 0; --r) {
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    const int nx = kt + NB - 1;
                    load_tile(min(nx, last), kR[(u + NB - 1) % NB], vR[(u + NB - 1) % NB], nx > last);
                    process(kt, kR[u], vR[u]);
                    ++kt;
                }
            }
            // The last (n mod NB) tiles, as nested tests: the flat form (one
            // test per slot) keeps every slot live through the tail and
            // spills at 256-byte rows.
            auto tail = [&](auto self, auto U) {
                constexpr int u = decltype(U)::value;
                if constexpr (u < NB - 1) {
                    if (kt + u <= last) {
                        process(kt + u, kR[u], vR[u]);
                        self(self, std::integral_constant<int, u + 1>{});
                    }
                }
            };
            tail(tail, std::integral_constant<int, 0>{});
        } else {
            // wide items without LDS sharing (a few pooled workgroups): two
            // buffers, which keeps the D 64 kernel at four waves per SIMD
            load_tile(kt, kR[0], vR[0]);
            for (;;) {
                load_tile(min(kt + 1, last), kR[1], vR[1]);
                process(kt, kR[0], vR[0]);
                if (++kt > last) break;
                load_tile(min(kt + 1, last), kR[0], vR[0]);
                process(kt, kR[1], vR[1]);
                if (++kt > last) break;
            }
        }
    }

    if constexpr (FAST) {
        int kt = fast_end;
        if constexpr (NT == 1) {
            if (kt < kt_end) process(kt++, kT, vT);
        }
        for (; kt < kt_end; ++kt) {
            load_general(kt, kR[0], vR[0]);
            process(kt, kR[0], vR[0]);
        }
    }

    // ---- cooperative items: the workgroup's four waves took consecutive key
    // ranges of one (sequence, kv head, column tile) and combine their
    // softmax states through LDS. Every lane (g, j) of every wave holds the
    // same column j and head_dim elements (4g + r)*VCH + c; wave w combines
    // the elements with r == w across the four waves and stores them -- the
    // normalised output, or one partial of a longer split.
    if constexpr (NT == 1) {
        if (iv2.w != 0) {  // the planner flags all four items of a cooperative workgroup
            static_assert(coop_lds_bytes<DP>() == (kWaves * 4 * VCH * 64 + 2 * kWaves * 16) * 4, "LDS arena layout");
            auto s_acc = reinterpret_cast<float (*)[4 * VCH][64]>(attn_lds);
            auto s_m = reinterpret_cast<float (*)[16]>(attn_lds + kWaves * 4 * VCH * 64 * 4);
            auto s_l = reinterpret_cast<float (*)[16]>(attn_lds + (kWaves * 4 * VCH * 64 + kWaves * 16) * 4);
            const float lt = group_sum4(l[0]);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < VCH; ++c) s_acc[wave][r * VCH + c][lane] = acc[0][c][r];
            if (g == 0) {
                s_m[wave][j] = m[0];
                s_l[wave][j] = lt;
            }
            __syncthreads();
            float mw[kWaves], M = kMinM;
#pragma unroll
            for (int u = 0; u < kWaves; ++u) {
                mw[u] = s_m[u][j];
                M = fmaxf(M, mw[u]);
            }
            float L = 0.f, o[VCH];
#pragma unroll
            for (int c = 0; c < VCH; ++c) o[c] = 0.f;
#pragma unroll
            for (int u = 0; u < kWaves; ++u) {
                const float w = __builtin_amdgcn_exp2f(mw[u] - M);
                L += s_l[u][j] * w;
#pragma unroll
                for (int c = 0; c < VCH; ++c) o[c] += w * s_acc[u][wave * VCH + c][lane];
            }
            const int d0 = (4 * g + wave) * VCH;
            if (nct > 0 && qpos[0] >= 0) {
                if (pslot < 0) {
                    if (d0 < D) {
                        const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
                        for (int c = 0; c < VCH; ++c) o[c] *= inv;
                        store_elems<DT, VCH>(a.out + ((int64_t)prow[0] * a.o_sr + (int64_t)qhead[0] * a.o_sh + d0) * ES, o);
                    }
                } else {
                    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
                    for (int c = 0; c < VCH; ++c) o[c] *= inv;
                    store_elems<DT, VCH>(partial_out<DT>(a, pslot, j, d0), o);
                    if (g == 0 && wave == 0) {
                        float* ml = partial_ml(a, pslot);
                        ml[j] = M;
                        ml[16 + j] = L;
                    }
                }
            }
            // fused split-K merge: every wave releases its part of the
            // partial, then wave 0 counts the workgroup's arrival
            if (pslot >= 0 && a.counters != nullptr) {
                __threadfence();
                __syncthreads();
                if (wave == 0) {
                    const int m0 = iv1.w;
                    int prev = 0;
                    if (lane == 0) prev = atomicAdd(a.counters + m0, 1);
                    prev = __shfl(prev, 0, 64);
                    const int32_t* mg0 = a.merges + (int64_t)m0 * MF_PLAN_MERGE_INTS;
                    if (prev == mg0[3] - 1) {
                        __threadfence();
                        if (lane == 0) a.counters[m0] = 0;
                        merge_tile<DT, DP>(a, mg0, g, j);
                    }
                }
            }
            return;
        }
    }

    // ---- finish: the lane holds O^T[d = (4g + r)*VCH + c][column j], i.e. the
    // contiguous head_dim range [4g*VCH, 4g*VCH + 4*VCH) of its column.
    const int dbase = 4 * g * VCH;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float lt = group_sum4(l[nt]);
        if (nt >= nct || qpos[nt] < 0) continue;
        if (pslot < 0) {
            if (dbase < D) {
                const float inv = lt > 0.f ? 1.f / lt : 0.f;
                float vals[4 * VCH];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < VCH; ++c) vals[r * VCH + c] = acc[nt][c][r] * inv;
                char* op = a.out + ((int64_t)prow[nt] * a.o_sr + (int64_t)qhead[nt] * a.o_sh + dbase) * ES;
                store_out_chunk<DT, VCH>(op, vals);
            }
        } else {
            const float inv = lt > 0.f ? 1.f / lt : 0.f;
            float vals[4 * VCH];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < VCH; ++c) vals[r * VCH + c] = acc[nt][c][r] * inv;
            store_out_chunk<DT, VCH>(partial_out<DT>(a, pslot + nt, j, dbase), vals);
            if (g == 0) {
                float* ml = partial_ml(a, pslot + nt);
                ml[j] = m[nt];
                ml[16 + j] = lt;
            }
        }
    }

    // ---- fused split-K merge: the last partition of a group to arrive merges
    // the group. Release the partials (agent-scope fence: the L2s of the XCDs
    // are not coherent with each other), count the arrival, and on the last
    // arrival acquire everyone else's partials and reset the counter for the
    // next call. Every wave runs to the end; nothing waits on another wave.
    if (pslot >= 0 && a.counters != nullptr) {
        const int m0 = iv1.w;
        __threadfence();
        int prev = 0;
        if (lane == 0) prev = atomicAdd(a.counters + m0, 1);
        prev = __shfl(prev, 0, 64);
        const int32_t* mg0 = a.merges + (int64_t)m0 * MF_PLAN_MERGE_INTS;
        if (prev == mg0[3] - 1) {
            __threadfence();
            if (lane == 0) a.counters[m0] = 0;
            for (int o = 0; o < nct; ++o) merge_tile<DT, DP>(a, mg0 + o * MF_PLAN_MERGE_INTS, g, j);
        }
    }
}

// The item list comes as a separate first argument, which the build has the
// hardware preload into scalar registers: a wave's first item load then
// needs no load of the argument block (see attn_body).
template <int DT, int DP, int NT, bool FAST, bool TAIL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(attn_waves_per_eu<DT, DP, NT>())))
void attn_kernel(const int32_t* items, AttnArgs a) {
    a.items = items;
    if constexpr (TAIL) {
        // the copy workgroups first (measured on the C2 step: 53.7 us per
        // layer against 55.7 with them last)
        const int b = blockIdx.x;
        if (b < a.w_blocks) write_new_rows<DT>(a, b);
        else attn_body<DT, DP, NT, FAST, true>(a, b - a.w_blocks);
    } else {
        attn_body<DT, DP, NT, FAST>(a, blockIdx.x);
    }
}

// In a mixed launch the single-tile (decode) waves start their loads after a
// short sleep, about the time the dispatcher takes to hand out the launch's
// workgroups. Per-workgroup timestamps of the C2 launch showed a prefill
// workgroup beside a decode workgroup spend 14.6 us (median) from its start
// to its first staged tile, against 6.1 us on a CU without one: its setup
// loads (block table, Q, the first K/V stages) queued behind the decode
// waves' streams, while the decode workgroups themselves finished at 14 us
// and the prefill ones at 34-41 us. With the decode waves held back by one
// s_sleep(32) (2,048 cycles) the prefill setup loads go out first: C2 engine
// layer 43.0-43.6 us against 44.6-45.1 (graph replays, alternating builds);
// two to four sleeps gave 43.3-44.1, six 44.9-45.1, nine 46.0-46.4.
#ifndef MF_MIXED_NARROW_SLEEPS
#define MF_MIXED_NARROW_SLEEPS 1
#endif
__device__ __forceinline__ void narrow_start_delay() {
#pragma unroll
    for (int i = 0; i < MF_MIXED_NARROW_SLEEPS; ++i) __builtin_amdgcn_s_sleep(32);
}

// Single-tile and wide items of one plan in one launch: the first
// workgroups run the single-tile items (decode rows: chains of dependent
// loads, latency-bound), the last `wide_blocks` the wide ones (prefill rows:
// MFMA and softmax work), which fill the slots the single-tile workgroups
// leave and overlap their load latency. Two back-to-back launches would leave
// the chip half idle for the length of the shorter one. Measured on the C2
// step (bf16, D 64, 382 single-tile and 900 wide workgroups): 67.9 us per
// layer as two launches, 62.7 us with the wide workgroups first, 58.6 us with
// the single-tile ones first. Each workgroup is entirely one kind, so the
// barriers of either body stay workgroup-uniform.
//
// Occupancy: with 16-bit rows of 128 bytes (D 64) the launch asks
// for four waves per SIMD. Its LDS is one arena sized for the larger of the
// two bodies (32.8 KB at D 64, so four workgroups fit a CU), and the compiler
// then keeps it to 128 registers with a few spills; three waves per SIMD, the
// single-tile body's own need (140 registers), left the C2 step's 1,104
// workgroups in more than one round of three per CU. Measured on the C2
// engine layer as graph replays: 55.1-56.3 us at four, 56.0-57.3 at three.
template <int DT, int DP, int NTW>
constexpr int mixed_waves_per_eu() {
    if constexpr (DT != MF_F32 && DP == 64) return 4;
    else return attn_waves_per_eu<DT, DP, NTW>() < attn_waves_per_eu<DT, DP, 1>() ? attn_waves_per_eu<DT, DP, NTW>()
                                                                                 : attn_waves_per_eu<DT, DP, 1>();
}
template <int DT, int DP, int NTW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(mixed_waves_per_eu<DT, DP, NTW>())))
void attn_mixed_kernel(AttnArgs narrow, AttnArgs wide, int wide_blocks) {
    const int b = blockIdx.x;
    const int narrow_blocks = (int)gridDim.x - wide_blocks;
    if (b < narrow_blocks) {
        narrow_start_delay();
        attn_body<DT, DP, 1, true>(narrow, b);
    } else {
        attn_body<DT, DP, NTW, true>(wide, b - narrow_blocks);
    }
}

// The written-in-flight form: the copy workgroups first, then the narrow and
// wide ones. One argument block (the wide items differ only in their list):
// the larger body needs the scalar registers a second block would take.
template <int DT, int DP, int NTW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(mixed_waves_per_eu<DT, DP, NTW>())))
void attn_mixed_tail_kernel(AttnArgs a, const int32_t* wide_items, int wide_num_items,
                            const int32_t* wide_dev_count, int wide_blocks) {
    const int b = blockIdx.x - a.w_blocks;
    const int narrow_blocks = (int)gridDim.x - a.w_blocks - wide_blocks;
    if (b < 0) {
        write_new_rows<DT>(a, blockIdx.x);
    } else if (b < narrow_blocks) {
        narrow_start_delay();
        attn_body<DT, DP, 1, true, true>(a, b);
    } else {
        AttnArgs w = a;
        w.items = wide_items;
        w.num_items = wide_num_items;
        w.dev_count = wide_dev_count;
        attn_body<DT, DP, NTW, true, true>(w, b - narrow_blocks);
    }
}

// ------------------------------------------------------------ decode slices
// A large decode launch as one resident round of waves (mf_attention_plan_slices).
// The plan cuts the concatenated (sequence, 16-key tile) order into equal
// slices; one wave per (slice, kv head) streams the slice's tiles for its head
// and the waves of a slice sit next to each other in the grid (four to a
// workgroup), so every block's rows are read for all kv heads at about the
// same time and no workgroup waits for another to leave. Measured on MI355X
// with a load-only kernel over the C5 block tables: the per-range plan
// (cooperative units: one CU reading one head's quarters, several rounds of
// workgroups) streams at 5.9 TB/s, the same tiles in one round with a
// workgroup per four heads of a range at 6.5-6.8 TB/s. The plan counts one
// workgroup per CU (one wave per SIMD, MF_SLICE_WAVES_PER_CU): with two per
// CU the C5 layer took 521 us against 505, fewer streams keeping the HBM
// busier (three per CU at head_dim 64: 303 against 287 us).
//
// A slice is a list of segments, each one sequence's tiles [kt0, kt1) (a
// whole range or a piece of one; pieces leave split-K partials for the merge
// kernel). Each lane holds eight of the slice's block-table entries (tile
// lane + 64k), so the register ring below runs across segment boundaries
// without a drain: every segment is padded to a multiple of the ring depth
// with dummy tiles (entry stored as ~block: a one-line load, every key
// masked), which keeps the ring's slot of a tile fixed at tile % depth. Lane
// i holds segment i's record and query position, and each segment start
// loads the next segment's query.
constexpr int kSliceRecordInts = MF_SLICE_INTS;
constexpr int kSliceMaxTiles = MF_SLICE_MAX_TILES;        // table entries per lane: tiles / 64
constexpr int kSliceTableRegs = kSliceMaxTiles / 64;
constexpr int kSliceMaxSegments = MF_SLICE_MAX_SEGMENTS;  // one record per lane at set-up
static_assert(kSliceMaxTiles % 64 == 0 && kSliceMaxSegments <= 64, "slice limits");

template <int DT, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(attn_waves_per_eu<DT, DP, 1>())))
void attn_slice_kernel(AttnArgs a, int num_slices, int hkv) {
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    constexpr int EPL = 16 / ES;
    constexpr int NL = DP * ES / 64;
    constexpr int VCH = DP / 16;
    constexpr int VB = VCH * ES;
    constexpr int VWD = VB / 4;
    constexpr int NB = MF_NARROW_DEPTH;
    constexpr float kNegInf = -__builtin_huge_valf();

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int w = blockIdx.x * kWaves + wave;
    if (w >= num_slices * hkv) return;
    const int sl = w / hkv;
    const int h = w - sl * hkv;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int j = lane & 15;

    // ---- set-up: the slice's segment records, one per lane, then its
    // block-table entries (4 per lane) and the first ring tiles
    const int32_t* hdr = a.items + (int64_t)sl * kSliceRecordInts;
    const int seg0 = hdr[0], nseg = hdr[1], ntiles = hdr[2];
    if (nseg <= 0 || ntiles <= 0) return;  // (the planner makes no empty slice)
    const int32_t* segs = a.items + ((int64_t)num_slices + seg0) * kSliceRecordInts;
    // Lane i keeps segment i's record (and its query position) for the whole
    // slice: a segment start reads it with readlane, no memory wait.
    const int32_t* rec = segs + (int64_t)min(lane, nseg - 1) * kSliceRecordInts;
    const int4 r0 = *(const int4*)rec;        // s, kt0, kt1, row
    const int4 r1 = *(const int4*)(rec + 4);  // kv_len, slot0, pieces, piece
    int tbl[kSliceTableRegs];
    {
        const int len = lane < nseg ? r0.z - r0.y : 0;
        const int plen = (len + NB - 1) / NB * NB;
        int pend = plen;  // inclusive scan of the padded lengths
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(pend, off, 64);
            if (lane >= off) pend += v;
        }
        const int pstart = pend - plen;
#pragma unroll
        for (int k = 0; k < kSliceTableRegs; ++k) {
            const int t = min(lane + 64 * k, ntiles - 1);
            int idx = 0;  // last segment starting at or before t
#pragma unroll
            for (int step = 32; step >= 1; step >>= 1) {
                const int c = idx + step;
                const int ps = __shfl(pstart, min(c, 63), 64);
                if (c < nseg && ps <= t) idx = c;
            }
            const int ts = __shfl(r0.x, idx, 64);
            const int tk0 = __shfl(r0.y, idx, 64);
            const int tlen = __shfl(len, idx, 64);
            const int o = t - __shfl(pstart, idx, 64);
            const bool real = o < tlen;
            const int e = a.block_tables[(int64_t)ts * a.bt_stride + tk0 + (real ? o : tlen - 1)];
            tbl[k] = real ? e : ~e;
        }
    }
    auto tbl_at = [&](int i) -> int {  // wave-uniform i
        const int k = i >> 6;
        const int l = i & 63;
        int e = __builtin_amdgcn_readlane(tbl[0], l);
#pragma unroll
        for (int q = 1; q < kSliceTableRegs; ++q) e = k == q ? __builtin_amdgcn_readlane(tbl[q], l) : e;
        return e;
    };

    const uint32_t k_lane_off = (uint32_t)(((int64_t)j * a.p_ss + g * EPL) * ES);
    const uint32_t v_row_bytes = (uint32_t)(a.p_ss * ES);
    const uint32_t v_lane_off = (uint32_t)(((int64_t)(4 * g) * a.p_ss + j * VCH) * ES);
    uint32_t v_off[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v_off[r] = v_lane_off + (uint32_t)r * v_row_bytes;
    // Tile i of the slice; `past` (wave-uniform): a prefetch slot beyond the
    // slice's last tile. Dummy and past tiles load one line per chunk.
    auto load_tile = [&](int i, uint4 (&kf)[NL], uint32_t (&vf)[4][VWD], bool past) {
        const int e = tbl_at(i);
        const int phys = e < 0 ? ~e : e;
        const int64_t boff = ((int64_t)phys * a.p_sb + (int64_t)h * a.p_sh) * ES;
        const char* kb = a.k_pool + boff;
        const char* vb = a.v_pool + boff;
        const uint32_t sel = (past || e < 0) ? 0u : 0xffffffffu;
        const uint32_t ko = k_lane_off & sel;
        if constexpr (DP * ES >= 256) {
#pragma unroll
            for (int c = 0; c < NL; ++c) kf[c] = ld_nt16(kb + ko + c * 4 * 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) ld_words_nt<VB>(vb + (v_off[r] & sel), vf[r]);
        } else {
#pragma unroll
            for (int c = 0; c < NL; ++c) kf[c] = *(const uint4*)(kb + ko + c * 4 * 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) ld_words<VB>(vb + (v_off[r] & sel), vf[r]);
        }
    };

    // Query position of lane i's segment; then the first segment's query
    // (MFMA B operand: lane (g, j) holds column j's head_dim chunks c*4 + g;
    // padding columns j >= G read column 0's, whose scores are never stored)
    // and the first ring tiles. A segment loads the next one's query when it
    // starts, so no segment start waits on memory.
    const int lpos = reinterpret_cast<const int32_t*>(a.positions)[2 * (int64_t)r0.w];
    const bool colv = j < a.G;  // decode: one row, columns 0..G-1 are its heads
    const int qhead = h * a.G + (colv ? j : 0);
    uint4 qn[NL];
    auto load_q = [&](int row) {
#pragma unroll
        for (int c = 0; c < NL; ++c)
            qn[c] = *(const uint4*)(a.q + ((int64_t)row * a.q_sr + (int64_t)qhead * a.q_sh + (c * 4 + g) * EPL) * ES);
    };
    load_q(__builtin_amdgcn_readlane(r0.w, 0));
    uint4 kR[NB][NL];
    uint32_t vR[NB][4][VWD];
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) load_tile(min(i, ntiles - 1), kR[i], vR[i], i > ntiles - 1);

    // ---- per-segment state (the lambdas below read it by reference)
    uint4 qf[NL];
    float m, l, thr;
    f32x4 acc[VCH];
    int lim = -1, minpos = -1, key_end = 0;

    auto process = [&](int kt, const uint4 (&kf)[NL], uint32_t (&vf)[4][VWD]) {
        if ((kt + 1) * 16 > key_end) {
            // keys past the segment (padding, or slots past the context,
            // which may hold anything): p = 0 there, and 0 * NaN is NaN
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool live = kt * 16 + 4 * g + r < key_end;
#pragma unroll
                for (int x = 0; x < VWD; ++x) vf[r][x] = live ? vf[r][x] : 0u;
            }
        }
        f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NL; ++c) st = mfma_qk<DT>(kf[c], qf[c], st);
        float sv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[r] = st[r];
        if (!(kt * 16 + 15 <= minpos && (kt + 1) * 16 <= key_end)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[r] = kt * 16 + 4 * g + r <= lim ? sv[r] : kNegInf;
        }
        // lazy rescale, exactly as the per-range kernel does it
        const float lmax = fmax_prop(fmax_prop(sv[0], sv[1]), fmax_prop(sv[2], sv[3]));
        if (__builtin_amdgcn_ballot_w64(lmax > thr) != 0) {
            const float mn = fmaxf(m, group_max4(lmax) * a.scale_log2);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            l *= alpha;
#pragma unroll
            for (int c = 0; c < VCH; ++c) acc[c] *= alpha;
            m = mn;
            thr = (mn + kLazyLog2) * a.inv_scale_log2;
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], a.scale_log2, -m));
        l += (p[0] + p[1]) + (p[2] + p[3]);
        if constexpr (DT == MF_F32) {
#pragma unroll
            for (int c = 0; c < VCH; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vf[r][c]), p[r], acc[c], 0, 0, 0);
        } else {
            uint2 p16;
            if constexpr (DT == MF_BF16) {
                p16 = make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){p[0], p[1]}, bf16x2)),
                                 __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){p[2], p[3]}, bf16x2)));
            } else {
                p16 = make_uint2(f32_to_bits<DT>(p[0]) | (f32_to_bits<DT>(p[1]) << 16),
                                 f32_to_bits<DT>(p[2]) | (f32_to_bits<DT>(p[3]) << 16));
            }
#pragma unroll
            for (int c = 0; c < VCH; ++c) {
                const int wd = c >> 1;
                const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                const uint2 va = make_uint2(__builtin_amdgcn_perm(vf[1][wd], vf[0][wd], sel),
                                            __builtin_amdgcn_perm(vf[3][wd], vf[2][wd], sel));
                acc[c] = mfma_pv16<DT>(va, p16, acc[c]);
            }
        }
    };

    const int dbase = 4 * g * VCH;
    int t = 0;  // slice index of the next tile to process
    for (int si = 0; si < nseg; ++si) {
        const int kt0 = __builtin_amdgcn_readlane(r0.y, si);
        const int kt1 = __builtin_amdgcn_readlane(r0.z, si);
        const int row = __builtin_amdgcn_readlane(r0.w, si);
        const int kv_len = __builtin_amdgcn_readlane(r1.x, si);
        const int pos = __builtin_amdgcn_readlane(lpos, si);
#pragma unroll
        for (int c = 0; c < NL; ++c)
            qf[c] = make_uint4(qn[c].x ^ a.q_sign, qn[c].y ^ a.q_sign, qn[c].z ^ a.q_sign, qn[c].w ^ a.q_sign);
        // the next segment's query (the last segment re-reads its own, so
        // every segment issues the same loads)
        load_q(__builtin_amdgcn_readlane(r0.w, min(si + 1, nseg - 1)));
        key_end = min(kv_len, kt1 * 16);
        lim = colv && pos >= 0 ? min(pos, key_end - 1) : -1;
        minpos = pos;
        m = kMinM;
        thr = (kMinM + kLazyLog2) * a.inv_scale_log2;
        l = 0.f;
#pragma unroll
        for (int c = 0; c < VCH; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

        const int seg_start = t;
        const int rounds = (kt1 - kt0 + NB - 1) / NB;
        for (int r = rounds; r > 0; --r) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int nx = t + NB - 1;
                load_tile(min(nx, ntiles - 1), kR[(u + NB - 1) % NB], vR[(u + NB - 1) % NB], nx > ntiles - 1);
                process(kt0 + (t - seg_start), kR[u], vR[u]);
                ++t;
            }
        }

        // ---- finish the segment: the normalised output, or its partial
        const float lt = group_sum4(l);
        if (colv && pos >= 0) {
            const int slot0 = __builtin_amdgcn_readlane(r1.y, si);
            if (slot0 < 0) {
                const float inv = lt > 0.f ? 1.f / lt : 0.f;
                float vals[4 * VCH];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < VCH; ++c) vals[r * VCH + c] = acc[c][r] * inv;
                store_out_chunk<DT, VCH>(a.out + ((int64_t)row * a.o_sr + (int64_t)qhead * a.o_sh + dbase) * ES, vals);
            } else {
                const int pslot = slot0 + h * __builtin_amdgcn_readlane(r1.z, si) + __builtin_amdgcn_readlane(r1.w, si);
                const float inv = lt > 0.f ? 1.f / lt : 0.f;
                float vals[4 * VCH];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < VCH; ++c) vals[r * VCH + c] = acc[c][r] * inv;
                store_out_chunk<DT, VCH>(partial_out<DT>(a, pslot, j, dbase), vals);
                if (g == 0) {
                    float* ml = partial_ml(a, pslot);
                    ml[j] = m;
                    ml[16 + j] = lt;
                }
            }
        }
    }
}

// --------------------------------------------------------------- merge kernel
// A merge launch's record mi, loaded before its count check (record
// min(mi, num_merges - 1): in bounds for every workgroup of the grid), so the
// load goes out with the argument block's instead of one round trip after it;
// the record list's address and num_merges are the preloaded first arguments.
// The argument fields the merge addresses its partials, row map and output
// from are loaded in the same batch. The empty asm keeps the loads ahead of
// the check.
__device__ __forceinline__ void load_merge_record(const AttnArgs& a, const int32_t* merges, int mi, int num_merges,
                                                  int32_t (&mg)[MF_PLAN_MERGE_INTS]) {
    const int32_t* rec = merges + (int64_t)min(mi, num_merges - 1) * MF_PLAN_MERGE_INTS;
    const int4 r0 = *(const int4*)rec, r1 = *(const int4*)(rec + 4);
    asm volatile("" ::"s"(r0.x), "s"(r0.y), "s"(r0.z), "s"(r0.w), "s"(r1.x), "s"(r1.y), "s"(r1.z), "s"(r1.w));
    asm volatile("" ::"s"(a.G), "s"(a.out), "s"(a.o_sr), "s"(a.o_sh), "s"(a.row_map), "s"(a.partials),
                 "s"(a.part_dstride), "s"(a.head_dim));
    mg[0] = r0.x; mg[1] = r0.y; mg[2] = r0.z; mg[3] = r0.w;
    mg[4] = r1.x; mg[5] = r1.y; mg[6] = r1.z; mg[7] = r1.w;
}

// One wave per merge record, each record a workgroup of its own: the wave
// loads its record's partitions four at a time (merge_range) and writes the
// output directly, with no LDS combine or barrier. Measured on MI355X against
// the two earlier forms (four waves per record splitting its partitions and
// combining them in LDS below 128 records, four records per workgroup above):
// C3's verify layer (75 records) 11.36-11.38 us against 12.29-12.40, the C2
// layer (1,955 records) 37.9-38.1 against 38.2-38.3, C5 (824) the same.
template <int DT, int DP>
__global__ __launch_bounds__(64) void merge_kernel(const int32_t* merges, int num_merges, AttnArgs a) {
    const int mi = blockIdx.x;
    int32_t mg[MF_PLAN_MERGE_INTS];
    load_merge_record(a, merges, mi, num_merges, mg);
    if (mi >= (a.dev_count ? *a.dev_count : num_merges)) return;
    const int lane = threadIdx.x & 63;
    merge_tile<DT, DP>(a, mg, lane >> 4, lane & 15);
}

// The split-K merge launch: one single-wave workgroup per record.
template <int DT, int DP>
int launch_merge(const AttnArgs& a, const int32_t* merges, int64_t n_merges, hipStream_t stream) {
    hipLaunchKernelGGL((merge_kernel<DT, DP>), dim3((unsigned)n_merges), dim3(64), 0, stream, merges, (int)n_merges,
                       a);
    return check_launch();
}

// TAIL: a written-in-flight launch (16-token blocks and unpadded head_dim
// only: `fast`); its copy workgroups ride in the first launch, or in a
// copy-only launch when there are no items.
template <int DT, int DP, bool TAIL = false>
int launch_attention(AttnArgs a, const int32_t* items, int64_t n_narrow, int64_t n_wide,
                     const int32_t* merges, int64_t n_merges, bool fast, const int32_t* dev_counts,
                     hipStream_t stream) {
    // With arrival counters the attention kernel merges its own partitions;
    // a merges-only call (no items) still runs the separate merge kernel.
    const bool fused = a.counters != nullptr && (n_narrow + n_wide) > 0;
    constexpr int NTW = wide_tiles(DT, DP);
    if constexpr (TAIL) {
        if (!fast) return MF_ERR_UNSUPPORTED;
        if (a.w_blocks > 0 && n_narrow + n_wide == 0) {
            AttnArgs aw = a;
            aw.items = items;
            aw.num_items = 0;
            aw.dev_count = nullptr;
            hipLaunchKernelGGL((attn_kernel<DT, DP, 1, true, true>), dim3((unsigned)a.w_blocks), dim3(256),
                               (attn_lds_bytes<DT, DP, 1, true>()), stream, aw.items, aw);
            if (int st = check_launch()) return st;
        }
    } else {
        a.w_blocks = 0;
    }
#if MF_MIXED_LAUNCH
    if constexpr (NTW > 1 && DT != MF_F32) {
        if (fast && n_narrow > 0 && n_wide > 0) {
            AttnArgs an = a, aw = a;
            an.items = items;
            an.num_items = (int)n_narrow;
            an.dev_count = dev_counts ? dev_counts + 0 : nullptr;
            aw.items = items + n_narrow * MF_PLAN_ITEM_INTS;
            aw.num_items = (int)n_wide;
            aw.dev_count = dev_counts ? dev_counts + 1 : nullptr;
            const int64_t wide_blocks = (n_wide + kWaves - 1) / kWaves;
            const dim3 grid((unsigned)(a.w_blocks + wide_blocks + (n_narrow + kWaves - 1) / kWaves));
            constexpr int lds = attn_lds_bytes<DT, DP, 1, true>() > attn_lds_bytes<DT, DP, NTW, true>()
                                    ? attn_lds_bytes<DT, DP, 1, true>() : attn_lds_bytes<DT, DP, NTW, true>();
            if constexpr (TAIL)
                hipLaunchKernelGGL((attn_mixed_tail_kernel<DT, DP, NTW>), grid, dim3(256), lds, stream, an,
                                   aw.items, aw.num_items, aw.dev_count, (int)wide_blocks);
            else
                hipLaunchKernelGGL((attn_mixed_kernel<DT, DP, NTW>), grid, dim3(256), lds, stream, an, aw,
                                   (int)wide_blocks);
            if (int st = check_launch()) return st;
            n_narrow = n_wide = 0;
            a.w_blocks = 0;
        }
    }
#endif
    if (n_narrow > 0) {
        a.items = items;
        a.num_items = (int)n_narrow;
        a.dev_count = dev_counts ? dev_counts + 0 : nullptr;
        const dim3 grid((unsigned)(a.w_blocks + (n_narrow + kWaves - 1) / kWaves));
        if (fast)
            hipLaunchKernelGGL((attn_kernel<DT, DP, 1, true, TAIL>), grid, dim3(256),
                               (attn_lds_bytes<DT, DP, 1, true>()), stream, a.items, a);
        else if constexpr (!TAIL)
            hipLaunchKernelGGL((attn_kernel<DT, DP, 1, false>), grid, dim3(256), (attn_lds_bytes<DT, DP, 1, false>()),
                               stream, a.items, a);
        if (int st = check_launch()) return st;
        a.w_blocks = 0;
    }
    if constexpr (NTW > 1) {
        if (n_wide > 0) {
            a.items = items + n_narrow * MF_PLAN_ITEM_INTS;
            a.num_items = (int)n_wide;
            a.dev_count = dev_counts ? dev_counts + 1 : nullptr;
            const dim3 grid((unsigned)(a.w_blocks + (n_wide + kWaves - 1) / kWaves));
            if (fast)
                hipLaunchKernelGGL((attn_kernel<DT, DP, NTW, true, TAIL>), grid, dim3(256),
                                   (attn_lds_bytes<DT, DP, NTW, true>()), stream, a.items, a);
            else if constexpr (!TAIL)
                hipLaunchKernelGGL((attn_kernel<DT, DP, NTW, false>), grid, dim3(256),
                                   (attn_lds_bytes<DT, DP, NTW, false>()), stream, a.items, a);
            if (int st = check_launch()) return st;
        }
    } else {
        if (n_wide > 0) return MF_ERR_ARG;  // the plan was made for another dtype
    }
    if (n_merges > 0 && !fused) {
        a.dev_count = dev_counts ? dev_counts + 2 : nullptr;
        if (int st = launch_merge<DT, DP>(a, merges, n_merges, stream)) return st;
    }
    return MF_OK;
}

// A slice plan (mf_attention_plan_slices): one wave per (slice, kv head),
// then the merge of the sequences split across slices.
template <int DT, int DP>
int launch_slices(AttnArgs a, const int32_t* slices, int64_t n_slices, int hkv, const int32_t* merges,
                  int64_t n_merges, hipStream_t stream) {
    if (n_slices > 0) {
        a.items = slices;
        const int64_t waves = n_slices * hkv;
        const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves));
        hipLaunchKernelGGL((attn_slice_kernel<DT, DP>), grid, dim3(256), 0, stream, a, (int)n_slices, hkv);
        if (int st = check_launch()) return st;
    }
    if (n_merges > 0) {
        if (int st = launch_merge<DT, DP>(a, merges, n_merges, stream)) return st;
    }
    return MF_OK;
}

// Padded head_dim the kernels are built for, or 0 if unsupported.
int padded_head_dim(int dtype, int d) {
    if (d <= 0 || (d & (d - 1)) != 0) return 0;  // powers of two only
    if (dtype == MF_F32) {
        if (d > 128) return 0;
        return d < 16 ? 16 : d;
    }
    if (d > 256) return 0;
    return d < 32 ? 32 : d;
}

inline int part_dstride_for(int head_dim) { return head_dim < 32 ? 32 : head_dim; }

}  // namespace
}  // namespace mf

extern "C" int mf_attention_plan(int num_seqs, const int32_t* cu_seqlens, const int32_t* kv_lens,
                                 int num_q_heads, int num_kv_heads, int head_dim, int dtype,
                                 int partition_tiles, int32_t* items, int64_t items_capacity,
                                 int32_t* merges, int64_t merges_capacity, int64_t* counts) {
    if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || !counts)
        return MF_ERR_ARG;
    if (num_q_heads % num_kv_heads) return MF_ERR_ARG;
    if (num_seqs > 0 && (!cu_seqlens || !kv_lens)) return MF_ERR_ARG;
    const int DP = mf::padded_head_dim(dtype, head_dim);
    if (!mf::dtype_ok(dtype) || !DP) return MF_ERR_UNSUPPORTED;
    const int WT = mf::wide_tiles(dtype, DP);
    const int G = num_q_heads / num_kv_heads;
    const int Hkv = num_kv_heads;

    auto col_tiles = [&](int s) -> int {
        const int qlen = cu_seqlens[s + 1] - cu_seqlens[s];
        if (qlen <= 0 || kv_lens[s] <= 0) return 0;
        return (qlen * G + 15) / 16;
    };

    // Key partition sizes, per item class. Single-column-tile (narrow)
    // items get their parallelism from splitting keys: about MF_NARROW_ITEMS
    // items (two to four waves per SIMD), few enough that partials stay
    // small. (Measured on C5: 128-tile partitions, 4,192 items, beat 64-tile
    // ones, 7,320 items: 539 vs 548 us and a merge of 13.5 vs 20 us.) Wide items already
    // come as many column groups, and each split of one costs a 16-column fp32
    // partial per tile written and merged again, so they are split only as far
    // as it takes to reach kWideItems items.
    // Narrow partition: the candidate (a power of two from 4 to
    // kMaxItemTiles tiles per wave) with the least estimated time, where a
    // launch takes the longer of its bandwidth time and its longest wave's
    // chain of tiles, plus the merge launch if any range is split. A range of
    // T > q tiles runs as ceil(T / 4q) units of four waves. Ties go to the
    // longer partition. The constants are fitted to partition sweeps on
    // MI355X (bf16, D 64) timed as HIP-graph replays, i.e. without host
    // submission time: a lone wave's chain costs about 0.53 us per 16-key
    // tile, decode items stream near 5 TB/s, and a split costs about 9 us of
    // merge. Picks: merge-free 32-tile waves for a 64-sequence decode step of
    // 96-1152 keys (17.0 us against 18.5 at 4 tiles), 8 for C3's verify (16.8
    // against 18.5 merge-free at 32), 16 for C2's decodes, 128 on C5.
    auto narrow_partition = [&](int fallback) {
        constexpr double kChainUs = 0.53, kMergeUs = 9.0, kBytesPerUs = 5.0e6;
        const double tile_us = 16.0 * DP * mf::dtype_size(dtype) * 2 / kBytesPerUs;
        int64_t tiles_all = 0;
        for (int s = 0; s < num_seqs; ++s) {
            const int nct = col_tiles(s);
            if (nct && (nct == 1 || WT == 1)) tiles_all += (int64_t)Hkv * nct * ((kv_lens[s] + 15) / 16);
        }
        if (!tiles_all) return fallback;
        int best_q = fallback;
        double best = 1e300;
        for (int q = 4; q <= mf::kMaxItemTiles; q *= 2) {
            int longest = 0;
            bool split = false;
            for (int s = 0; s < num_seqs; ++s) {
                const int nct = col_tiles(s);
                if (!nct || !(nct == 1 || WT == 1)) continue;
                const int T = (kv_lens[s] + 15) / 16;
                if (T <= q) {
                    longest = std::max(longest, T);
                    continue;
                }
                const int units = (T + 4 * q - 1) / (4 * q);
                const int unit = (T + units - 1) / units;
                longest = std::max(longest, (unit + 3) / 4);
                split = split || units > 1;
            }
            const double est = std::max(tiles_all * tile_us, longest * kChainUs) + (split ? kMergeUs : 0.0);
            if (est <= best) {
                best = est;
                best_q = q;
            }
        }
        return best_q;
    };
    int64_t work = 0, wide_units = 0, narrow_units = 0;
    int wide_max_tiles = 0;
    for (int s = 0; s < num_seqs; ++s) {
        const int nct = col_tiles(s);
        if (!nct) continue;
        const bool narrow = nct == 1 || WT == 1;
        const int groups = narrow ? nct : (nct + WT - 1) / WT;
        const int tiles = (kv_lens[s] + 15) / 16;
        work += (int64_t)Hkv * groups * tiles;
        if (narrow) narrow_units += (int64_t)Hkv * groups;
        if (!narrow) {
            wide_units += (int64_t)Hkv * groups;
            wide_max_tiles = std::max(wide_max_tiles, tiles);
        }
    }
    int P = std::min(partition_tiles, mf::kMaxItemTiles);
    int PW = P;
    bool mixed = false;  // a shared launch of narrow and wide items (quad partitions below)
    if (P <= 0) {
        const int64_t target_items = MF_NARROW_ITEMS;
        int64_t want = (work + target_items - 1) / target_items;
        int PA = 4;
        while (PA < want && PA < mf::kMaxItemTiles) PA *= 2;
        P = narrow_partition(PA);
        // wide: the smallest partition (a power of two, at least PA) whose
        // item count stays within the target
        PW = PA;
        if (wide_units > 0) {
            auto wide_items = [&](int q) {
                int64_t n = 0;
                for (int s = 0; s < num_seqs; ++s) {
                    const int nct = col_tiles(s);
                    if (!nct || nct == 1 || WT == 1) continue;
                    n += (int64_t)Hkv * ((nct + WT - 1) / WT) * (((kv_lens[s] + 15) / 16 + q - 1) / q);
                }
                return n;
            };
            while (PW < mf::kMaxItemTiles && PW < wide_max_tiles && wide_items(PW) > MF_WIDE_ITEMS) PW *= 2;
            // Beside wide items the narrow ones run in the same launch
            // (attn_mixed_kernel), where a narrow chain as long as a wide
            // wave's key range is hidden behind the wide waves; longer
            // narrow partitions then only save items and merges. Measured
            // on the C2 step (PW 32): narrow P 16 (the estimate's pick)
            // 58.1-58.9 us per layer, P 32 56.6-56.8, P 64 60.3-60.5;
            // again with the KV write in the launch and the raised prefill
            // priority: P 16 57.0-57.3, P 32 48.9-49.3, P 64 58.1-58.3.
            // The planner does not see the pool's block size: the shared
            // launch needs 16-key blocks, and with other block sizes the two
            // classes run as separate launches, where the raised partition
            // only lengthens the narrow launch's chains (no effect on
            // results, which do not depend on the partition).
            if (MF_MIXED_LAUNCH && WT > 1 && dtype != MF_F32 && head_dim == DP && narrow_units > 0) {
                P = std::max(P, PW);
                mixed = true;
            }
        }
    }

    // Narrow items (one 16-column tile): a (sequence, kv head, column tile)
    // of at most P key tiles is one single-wave item, packed four to a
    // workgroup with other single items. A longer one is cut into balanced
    // units of at most 4P tiles; a unit is a cooperative workgroup whose four
    // waves take consecutive quarters of its tiles and combine their softmax
    // states through LDS, so only ranges of more than 4P tiles leave split-K
    // partials for the merge kernel.
    //
    // Wide items are launched in workgroups of kWaves (one item per wave).
    // A (sequence, kv head, partition) run of at least kWaves column groups
    // fills whole workgroups of its own -- consecutive column groups, the last
    // one padded with empty items (no column tiles) -- so the workgroup shares
    // each K/V tile through LDS. Shorter runs are pooled and packed kWaves to
    // a workgroup, each wave on its own keys.
    const int U = mf::kWaves;
    auto round_up = [&](int64_t n) { return (n + U - 1) / U * U; };
    // key partitions of sequence s: count, and the start of partition p
    // (narrow cooperative ranges are balanced; the rest are Q-tile strides).
    // A wide range takes as many partitions as PW-tile strides would give,
    // in strides of equal length: the C2 chunks planned prefill-only
    // 34.9-35.3 us against 36.3-36.6 with PW strides (a short last
    // partition).
    auto partitions = [&](int s, bool narrow, int& Q, bool& coop) {
        const int tiles = (kv_lens[s] + 15) / 16;
        coop = narrow && tiles > P;
        Q = narrow ? (coop ? U * P : P) : PW;
        if (!narrow && tiles > PW) {
            const int np = (tiles + PW - 1) / PW;
            Q = (tiles + np - 1) / np;
        }
        return (tiles + Q - 1) / Q;
    };
    auto part_begin = [&](int tiles, int nparts, int Q, bool coop, int p) {
        return coop ? (int)((int64_t)p * tiles / nparts) : std::min(tiles, p * Q);
    };
    // Quad partitions (mixed plans). A sequence whose wide items fill whole
    // workgroups runs as column quads: the kWaves column groups one
    // workgroup holds, over one key range. In a mixed plan each quad takes
    // its own partitions: the tiles its last column sees, cut into
    // round(visible / W) equal ranges, W chosen so that the launch's wide
    // workgroups carry about two rounds' worth per compute unit (the total
    // visible work over 2 x 256 CUs, at least PW). Every wide workgroup then
    // holds about the same work, and each compute unit about two of them
    // beside the narrow ones, all in one resident round. C2 step, engine
    // layer as graph replays: 44.1-44.2 us against 45.8-46.0 with the ranges'
    // partitions (PW 64 strides); 1.5 workgroups per CU 49.3-49.6, 2.5
    // 47.1-47.4, 3 47.5-48.0, 4 53.3-53.5. Plans of wide items only keep the
    // ranges' partitions (there two per CU took the prefill items from 35.1
    // to 37.9 us). The XCD queues below take a (sequence, kv head)'s quads
    // as one run: the launch fetches 1.09x its algorithmic reads, against
    // 1.65x with each (quad, kv head) dealt alone (0.3 us faster).
    constexpr int kPlanCUs = 256;  // compute units of an MI355X
    auto quads = [&](int s) -> int {  // column quads of s, 0 if s is not a shared wide sequence
        const int nct = col_tiles(s);
        if (!mixed || !nct || nct == 1 || WT == 1) return 0;
        const int ngroups = (nct + WT - 1) / WT;
        return ngroups >= U ? (int)(round_up(ngroups) / U) : 0;
    };
    auto quad_visible = [&](int s, int qd) -> int {
        const int rows = cu_seqlens[s + 1] - cu_seqlens[s];
        const int end_ct = std::min(col_tiles(s), (qd + 1) * U * WT);
        const int last_col = std::min(end_ct * 16, rows * G) - 1;
        const int last_pos = kv_lens[s] - rows + last_col / G;
        return std::max(1, std::min((kv_lens[s] + 15) / 16, last_pos / 16 + 1));
    };
    double quad_w = 1.0;
    if (mixed) {
        int64_t visible = 0;
        for (int s = 0; s < num_seqs; ++s)
            for (int qd = 0, nq = quads(s); qd < nq; ++qd) visible += (int64_t)Hkv * quad_visible(s, qd);
        quad_w = std::max((double)std::max(PW, 1), (double)visible / (2.0 * kPlanCUs));
    }
    // Partition counts per (sequence, quad), then at most two wide
    // workgroups per CU: rounding can leave a few more, and with every CU
    // holding two, those few land as a third on some CU, which then finishes
    // last. Partitions are merged, one at a time, in the quad whose ranges
    // grow the least. C2: 530 -> 510 workgroups, engine layer 42.1-42.3 us
    // against 42.7-42.9.
    std::vector<std::vector<int>> qparts(num_seqs);
    if (mixed) {
        int64_t total = 0;
        for (int s = 0; s < num_seqs; ++s) {
            const int nq = quads(s);
            qparts[s].resize(nq);
            for (int qd = 0; qd < nq; ++qd) {
                const int v = quad_visible(s, qd);
                const int n = std::max(1, (int)std::lround(v / quad_w));
                qparts[s][qd] = std::max(n, (v + mf::kMaxItemTiles - 1) / mf::kMaxItemTiles);
                total += (int64_t)Hkv * qparts[s][qd];
            }
        }
        while (total > 2 * kPlanCUs) {
            int bs = -1, bq = -1;
            double best = 1e300;
            for (int s = 0; s < num_seqs; ++s)
                for (int qd = 0; qd < (int)qparts[s].size(); ++qd) {
                    const int n = qparts[s][qd], v = quad_visible(s, qd);
                    if (n <= 1 || (v + n - 2) / (n - 1) > mf::kMaxItemTiles) continue;
                    const double grown = (double)v / (n - 1);
                    if (grown < best) {
                        best = grown;
                        bs = s;
                        bq = qd;
                    }
                }
            if (bs < 0) break;  // every quad is down to one range (or at the item limit)
            --qparts[bs][bq];
            total -= Hkv;
        }
    }
    auto quad_parts = [&](int s, int qd) { return qparts[s][qd]; };

    // First walk: sizes only.
    int64_t n_single = 0, n_coop = 0, n_wide = 0, n_loose = 0, n_merges = 0, n_slots = 0;
    for (int s = 0; s < num_seqs; ++s) {
        const int nct = col_tiles(s);
        if (!nct) continue;
        const bool narrow = nct == 1 || WT == 1;
        int Q;
        bool coop;
        const int nparts = partitions(s, narrow, Q, coop);
        const int width = narrow ? 1 : WT;
        const int ngroups = (nct + width - 1) / width;
        if (narrow) {
            if (coop) n_coop += (int64_t)U * nparts * Hkv * ngroups;
            else n_single += (int64_t)nparts * Hkv * ngroups;
        } else if (const int nq = quads(s)) {
            for (int qd = 0; qd < nq; ++qd) {
                const int n = quad_parts(s, qd);
                const int cols = std::min(nct, (qd + 1) * U * WT) - qd * U * WT;
                n_wide += (int64_t)Hkv * n * U;
                if (n > 1) {
                    n_slots += (int64_t)Hkv * n * cols;
                    n_merges += (int64_t)Hkv * cols;
                }
            }
            continue;
        } else if (ngroups >= U) {
            n_wide += (int64_t)nparts * Hkv * round_up(ngroups);
        } else {
            n_loose += (int64_t)nparts * Hkv * ngroups;
        }
        if (nparts > 1) {
            n_slots += (int64_t)Hkv * nparts * nct;
            n_merges += (int64_t)Hkv * nct;
        }
    }
    const int64_t n_narrow = round_up(n_single) + n_coop;
    n_wide += round_up(n_loose);
    const int64_t pstride = 16 * (int64_t)(mf::part_dstride_for(head_dim) + 2);
    counts[0] = n_narrow;
    counts[1] = n_wide;
    counts[2] = n_merges;
    counts[3] = n_slots * pstride;
    if (n_narrow + n_wide > items_capacity || n_merges > merges_capacity) return MF_ERR_WORKSPACE;
    if ((n_narrow + n_wide) > 0 && !items) return MF_ERR_ARG;
    if (n_merges > 0 && !merges) return MF_ERR_ARG;

    // Second walk: stage the items and write the merges. Column group gi of
    // a sequence owns partial slots from slot0 + gi*Hkv*nparts*width
    // (head-major, then partition, then its w tiles) and merge records from
    // merge0 + gi*Hkv*width.
    typedef std::array<int32_t, MF_PLAN_ITEM_INTS> Item;
    std::vector<Item> singles, coop_items, shared_items, loose_items;
    int64_t wm = 0, slots = 0;
    for (int s = 0; s < num_seqs; ++s) {
        const int nct = col_tiles(s);
        if (!nct) continue;
        const bool narrow = nct == 1 || WT == 1;
        const int tiles = (kv_lens[s] + 15) / 16;
        int Q;
        bool coop;
        const int nparts = partitions(s, narrow, Q, coop);
        const int width = narrow ? 1 : WT;
        const int ngroups = (nct + width - 1) / width;
        if (const int nq = narrow ? 0 : quads(s)) {
            // quad partitions: per (kv head, quad), each column group owns
            // n * w consecutive slots (partition-major) and w merge records;
            // a kv head's workgroups are consecutive (one XCD run)
            for (int h = 0; h < Hkv; ++h) {
                for (int qd = 0; qd < nq; ++qd) {
                    const int n = quad_parts(s, qd);
                    const int v = quad_visible(s, qd);
                    int64_t gslot[mf::kWaves], grec[mf::kWaves];
                    for (int k = 0; k < U; ++k) {
                        const int gi = qd * U + k;
                        gslot[k] = grec[k] = -1;
                        if (gi >= ngroups || n <= 1) continue;
                        const int w = std::min(WT, nct - gi * WT);
                        gslot[k] = slots;
                        slots += (int64_t)n * w;
                        grec[k] = wm;
                        for (int o2 = 0; o2 < w; ++o2, ++wm) {
                            int32_t* o = merges + wm * MF_PLAN_MERGE_INTS;
                            o[0] = s;
                            o[1] = h;
                            o[2] = gi * WT + o2;
                            o[3] = n;
                            o[4] = (int32_t)(gslot[k] + o2);
                            o[5] = w;
                            o[6] = cu_seqlens[s];
                            o[7] = cu_seqlens[s + 1] - cu_seqlens[s];
                        }
                    }
                    for (int p = 0; p < n; ++p) {
                        const int k0 = (int)((int64_t)p * v / n), k1 = (int)((int64_t)(p + 1) * v / n);
                        for (int k = 0; k < U; ++k) {
                            const int gi = qd * U + k;
                            Item o{};
                            o[0] = s;
                            o[1] = h;
                            o[4] = k0;
                            o[5] = k1;
                            o[8] = cu_seqlens[s];
                            o[9] = cu_seqlens[s + 1] - cu_seqlens[s];
                            o[10] = kv_lens[s];
                            if (gi < ngroups) {
                                const int w = std::min(WT, nct - gi * WT);
                                o[2] = gi * WT;
                                o[3] = w;
                                o[6] = n > 1 ? (int32_t)(gslot[k] + (int64_t)p * w) : -1;
                                o[7] = n > 1 ? (int32_t)grec[k] : -1;
                            } else {  // padding: same keys, no columns, no partial slot
                                o[2] = (ngroups - 1) * WT;
                                o[6] = -1;
                                o[7] = -1;
                            }
                            shared_items.push_back(o);
                        }
                    }
                }
            }
            continue;
        }
        const int64_t slot0 = slots, merge0 = wm;
        auto make = [&](int gi, int p, int h, int k0, int k1) {
            const int cg0 = gi * width;
            const int w = std::min(width, nct - cg0);
            Item o;
            o[0] = s;
            o[1] = h;
            o[2] = cg0;
            o[3] = w;
            o[4] = k0;
            o[5] = k1;
            o[6] = nparts > 1 ? (int32_t)(slot0 + (int64_t)gi * Hkv * nparts * width + ((int64_t)h * nparts + p) * w)
                              : -1;
            o[7] = nparts > 1 ? (int32_t)(merge0 + (int64_t)gi * Hkv * width + (int64_t)h * w) : -1;
            o[8] = cu_seqlens[s];
            o[9] = cu_seqlens[s + 1] - cu_seqlens[s];
            o[10] = kv_lens[s];
            o[11] = 0;
            return o;
        };
        for (int p = 0; p < nparts; ++p) {
            const int k0 = part_begin(tiles, nparts, Q, coop, p);
            const int k1 = part_begin(tiles, nparts, Q, coop, p + 1);
            for (int h = 0; h < Hkv; ++h) {
                if (narrow) {
                    for (int gi = 0; gi < ngroups; ++gi) {
                        if (!coop) {
                            singles.push_back(make(gi, p, h, k0, k1));
                            continue;
                        }
                        // four waves on consecutive quarters of [k0, k1). In
                        // the unit holding a multi-row sequence's last tile (a
                        // verify pass: the boundary tile and the in-flight
                        // candidates, loaded key by key), the last wave counts
                        // MF_TAIL_WAVE_TILES more tiles than it has, so the
                        // others take them and the unit's waves reach its
                        // LDS combine together.
                        const int n = k1 - k0;
                        const int rows = cu_seqlens[s + 1] - cu_seqlens[s];
                        const int extra = (k1 == tiles && rows > 1) ? MF_TAIL_WAVE_TILES : 0;
                        auto cut = [&](int w) {
                            return w >= U ? k1 : std::min(k1, k0 + (int)((int64_t)w * (n + extra) / U));
                        };
                        for (int w = 0; w < U; ++w) {
                            Item o = make(gi, p, h, cut(w), cut(w + 1));
                            o[11] = 1;
                            coop_items.push_back(o);
                        }
                    }
                } else if (ngroups >= U) {
                    for (int gi = 0; gi < round_up(ngroups); ++gi) {
                        Item o = make(std::min(gi, ngroups - 1), p, h, k0, k1);
                        if (gi >= ngroups) {  // padding: same keys, no columns, no partial slot
                            o[3] = 0;
                            o[6] = -1;
                            o[7] = -1;
                        }
                        shared_items.push_back(o);
                    }
                } else {
                    for (int gi = 0; gi < ngroups; ++gi) loose_items.push_back(make(gi, p, h, k0, k1));
                }
            }
        }
        if (nparts > 1) {
            for (int gi = 0; gi < ngroups; ++gi) {
                const int cg0 = gi * width;
                const int w = std::min(width, nct - cg0);
                const int64_t group_base = slot0 + (int64_t)gi * Hkv * nparts * width;
                for (int h = 0; h < Hkv; ++h) {
                    for (int o2 = 0; o2 < w; ++o2) {
                        int32_t* o = merges + wm * MF_PLAN_MERGE_INTS;
                        o[0] = s;
                        o[1] = h;
                        o[2] = cg0 + o2;
                        o[3] = nparts;
                        o[4] = (int32_t)(group_base + (int64_t)h * nparts * w + o2);
                        o[5] = w;
                        o[6] = cu_seqlens[s];
                        o[7] = cu_seqlens[s + 1] - cu_seqlens[s];
                        ++wm;
                    }
                }
            }
            slots += (int64_t)Hkv * nparts * nct;
        }
    }
    // Longest first: the hardware hands out workgroups in order as slots free
    // up, so the last round of the grid is made of the short remainder
    // partitions instead of a few long ones. Items that run alone are sorted
    // and then cut into workgroups (the last padded with empty items); all
    // workgroups are ordered by their longest item. Stable, so equal lengths
    // keep their heads-adjacent order.
    auto len = [](const Item& o) { return o[5] - o[4]; };
    auto longer = [&](const Item& x, const Item& y) { return len(x) > len(y); };
    auto pad_to_workgroups = [&](std::vector<Item>& v) {
        std::stable_sort(v.begin(), v.end(), longer);
        while (v.size() % U) {
            Item o{};
            o[6] = -1;
            o[7] = -1;
            v.push_back(o);
        }
    };
    auto unit_len = [&](const Item* u) {
        int l = 0;
        for (int w = 0; w < U; ++w) l = std::max(l, len(u[w]));
        return l;
    };
    auto emit = [&](std::vector<const Item*>& units, int64_t wi) {
        std::stable_sort(units.begin(), units.end(),
                         [&](const Item* x, const Item* y) { return unit_len(x) > unit_len(y); });
        for (const Item* u : units)
            for (int w = 0; w < U; ++w, ++wi) std::copy(u[w].begin(), u[w].end(), items + wi * MF_PLAN_ITEM_INTS);
    };
    pad_to_workgroups(singles);
    pad_to_workgroups(loose_items);
    std::vector<const Item*> nunits, wunits;
    for (size_t i = 0; i < coop_items.size(); i += U) nunits.push_back(&coop_items[i]);
    for (size_t i = 0; i < singles.size(); i += U) nunits.push_back(&singles[i]);
    for (size_t i = 0; i < shared_items.size(); i += U) wunits.push_back(&shared_items[i]);
    for (size_t i = 0; i < loose_items.size(); i += U) wunits.push_back(&loose_items[i]);
    emit(nunits, 0);
    // A wide item's work: its tiles up to the last one its last column sees
    // (causal), a workgroup's the most of its four.
    auto item_work = [&](const Item& o) -> int64_t {
        const int ncols = o[9] * G;
        const int last_col = std::min((o[2] + o[3]) * 16, ncols) - 1;
        if (o[3] <= 0 || last_col < 0) return 0;
        const int last_pos = o[10] - o[9] + last_col / G;
        return std::max(0, std::min(o[5], last_pos / 16 + 1) - o[4]);
    };
    auto unit_work = [&](const Item* u) {
        int64_t l = 0;
        for (int w = 0; w < U; ++w) l = std::max(l, item_work(u[w]));
        return l;
    };
    if (MF_WIDE_XCD) {
        // Runs of workgroups on one key range, most work first, are dealt
        // to the queue with the least work so far; each queue then runs its
        // workgroups most work first, and the queues are interleaved.
        constexpr int X = 8;
        const size_t nu = wunits.size();
        std::vector<int64_t> work(nu);
        for (size_t i = 0; i < nu; ++i) work[i] = unit_work(wunits[i]);
        auto same_range = [&](size_t x, size_t y) {
            const Item& a = wunits[x][0];
            const Item& b = wunits[y][0];
            // one key range; in a mixed plan one (sequence, kv head), whose
            // quads' ranges overlap
            return a[0] == b[0] && a[1] == b[1] && (mixed || (a[4] == b[4] && a[5] == b[5]));
        };
        // run r holds units [run_begin[r], run_begin[r + 1])
        std::vector<size_t> run_begin;
        std::vector<int64_t> run_work;
        for (size_t i = 0; i < nu; ++i) {
            if (i >= shared_items.size() / U || run_begin.empty() || !same_range(i - 1, i)) {
                run_begin.push_back(i);
                run_work.push_back(0);
            }
            run_work.back() += work[i];
        }
        const size_t nruns = run_begin.size();
        run_begin.push_back(nu);
        std::vector<size_t> order(nruns);
        for (size_t i = 0; i < nruns; ++i) order[i] = i;
        std::stable_sort(order.begin(), order.end(), [&](size_t x, size_t y) { return run_work[x] > run_work[y]; });
        // queue x holds exactly the workgroups at wide positions x mod 8; a
        // run that no queue has room for is split over the roomiest ones
        std::vector<size_t> queue[X];
        int64_t load[X] = {};
        for (auto& q : queue) q.reserve(nu / X + 1);
        auto room = [&](int x) { return (int64_t)(nu / X + (x < (int)(nu % X) ? 1 : 0)) - (int64_t)queue[x].size(); };
        for (size_t ri : order) {
            size_t i = run_begin[ri];
            const size_t end = run_begin[ri + 1];
            while (i < end) {
                int best = -1;
                for (int x = 0; x < X; ++x)
                    if (room(x) >= (int64_t)(end - i) && (best < 0 || load[x] < load[best])) best = x;
                if (best < 0) {
                    for (int x = 0; x < X; ++x)
                        if (best < 0 || room(x) > room(best)) best = x;
                }
                const size_t take = std::min<size_t>(end - i, (size_t)room(best));
                for (size_t t = 0; t < take; ++t, ++i) {
                    queue[best].push_back(i);
                    load[best] += work[i];
                }
            }
        }
        for (auto& q : queue)
            std::stable_sort(q.begin(), q.end(), [&](size_t x, size_t y) { return work[x] > work[y]; });
        int64_t wi = n_narrow;
        for (size_t k = 0;; ++k) {
            bool any = false;
            for (int x = 0; x < X; ++x) {
                if (k >= queue[x].size()) continue;
                any = true;
                const Item* u = wunits[queue[x][k]];
                for (int w = 0; w < U; ++w, ++wi) std::copy(u[w].begin(), u[w].end(), items + wi * MF_PLAN_ITEM_INTS);
            }
            if (!any) break;
        }
    } else {
        emit(wunits, n_narrow);
    }
    return MF_OK;
}

// Slice plan for a large decode launch (attn_slice_kernel). The sequences'
// 16-key tiles, in sequence order, are cut into slices of about
// total / (num_cus * MF_SLICE_WAVES_PER_CU / Hkv) tiles, so one wave per
// (slice, kv head) fills the GPU exactly once at one workgroup per CU. A slice holds at most MF_SLICE_MAX_SEGMENTS
// segments and MF_SLICE_MAX_TILES tiles once each segment is padded to a
// multiple of the kernel's ring depth; a workload whose even share would
// exceed that gets more slices (a second round). A sequence cut across
// slices leaves one partial per piece and kv head, merged afterwards.
extern "C" int mf_attention_plan_slices(int num_seqs, const int32_t* cu_seqlens, const int32_t* kv_lens,
                                        int num_q_heads, int num_kv_heads, int head_dim, int dtype,
                                        int num_cus, int min_tiles_per_wave, int32_t* slices,
                                        int64_t slices_capacity, int32_t* merges, int64_t merges_capacity,
                                        int64_t* counts) {
    if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || !counts || num_cus <= 0 ||
        min_tiles_per_wave < 0)
        return MF_ERR_ARG;
    const int64_t resident_waves = (int64_t)num_cus * MF_SLICE_WAVES_PER_CU;
    if (num_q_heads % num_kv_heads) return MF_ERR_ARG;
    if (num_seqs > 0 && (!cu_seqlens || !kv_lens)) return MF_ERR_ARG;
    const int DP = mf::padded_head_dim(dtype, head_dim);
    if (!mf::dtype_ok(dtype) || !DP) return MF_ERR_UNSUPPORTED;
    const int G = num_q_heads / num_kv_heads;
    const int Hkv = num_kv_heads;
    counts[0] = counts[1] = counts[2] = counts[3] = 0;
    // Decode only: one query row per sequence, whose heads fit one column
    // tile, and head_dim at one of the kernel's sizes.
    if (DP != head_dim || G > 16) return MF_ERR_UNSUPPORTED;
    int64_t total = 0;
    for (int s = 0; s < num_seqs; ++s) {
        const int qlen = cu_seqlens[s + 1] - cu_seqlens[s];
        if (qlen < 0) return MF_ERR_ARG;
        if (kv_lens[s] <= 0 || qlen == 0) continue;
        if (qlen != 1) return MF_ERR_UNSUPPORTED;
        total += (kv_lens[s] + 15) / 16;
    }
    // Launches whose tiles give each resident wave fewer than
    // min_tiles_per_wave get no slice plan (counts stay zero): at
    // MF_SLICE_MIN_TILES and below, per-range items fit them in one round.
    if (total == 0 || total * Hkv < (int64_t)min_tiles_per_wave * resident_waves) return MF_OK;

    // Slices per round fill the GPU once; a workload whose even share would
    // not fit one slice runs whole rounds of equal slices (a round with only
    // a few slices would leave the GPU idle for its whole length). A slice's
    // real tiles stay below MF_SLICE_MAX_TILES by enough for the padding of
    // sixteen segments, so padding rarely closes a slice early.
    constexpr int NB = MF_NARROW_DEPTH;
    const int64_t base_slices = std::max<int64_t>(1, resident_waves / Hkv);
    const int64_t fill_cap = mf::kSliceMaxTiles - 16 * (NB - 1);
    const int64_t rounds = (total + base_slices * fill_cap - 1) / (base_slices * fill_cap);
    const int64_t want = rounds * base_slices;
    // slice i carries total / want tiles, one more for the first total % want
    const int64_t share = total / want, extra = total % want;

    // First walk: cut the slices (segment = sequence, kt0, kt1).
    struct Seg { int s, kt0, kt1; };
    std::vector<Seg> segs;
    std::vector<int64_t> begins;  // first segment of each slice
    std::vector<int> padded;      // padded tiles of each slice
    int64_t cur_real = 0, target = 0;
    int cur_pad = 0, cur_n = 0;
    auto open_slice = [&]() {
        target = std::max<int64_t>(1, share + ((int64_t)begins.size() < extra ? 1 : 0));
        begins.push_back((int64_t)segs.size());
        padded.push_back(0);
        cur_real = 0;
        cur_pad = 0;
        cur_n = 0;
    };
    open_slice();
    for (int s = 0; s < num_seqs; ++s) {
        const int qlen = cu_seqlens[s + 1] - cu_seqlens[s];
        if (kv_lens[s] <= 0 || qlen == 0) continue;
        const int T = (kv_lens[s] + 15) / 16;
        int kt = 0;
        while (kt < T) {
            const int64_t room_pad = mf::kSliceMaxTiles - cur_pad;
            if (cur_n == mf::kSliceMaxSegments || cur_real >= target || room_pad < NB) {
                open_slice();
                continue;
            }
            const int64_t take = std::min<int64_t>({(int64_t)(T - kt), target - cur_real, room_pad / NB * NB});
            segs.push_back({s, kt, (int)(kt + take)});
            cur_real += take;
            cur_pad += (int)((take + NB - 1) / NB * NB);
            padded.back() = cur_pad;
            ++cur_n;
            kt += (int)take;
        }
    }
    if (padded.back() == 0) {  // a slice opened after the last segment
        begins.pop_back();
        padded.pop_back();
    }
    const int64_t n_slices = (int64_t)begins.size();
    const int64_t n_segs = (int64_t)segs.size();

    // Pieces per sequence: slot ranges and merge records for split ones.
    std::vector<int> pieces(num_seqs, 0);
    for (const Seg& g : segs) ++pieces[g.s];
    int64_t n_merges = 0, n_slots = 0;
    for (int s = 0; s < num_seqs; ++s)
        if (pieces[s] > 1) {
            n_merges += Hkv;
            n_slots += (int64_t)Hkv * pieces[s];
        }
    counts[0] = n_slices;
    counts[1] = n_segs;
    counts[2] = n_merges;
    counts[3] = n_slots * 16 * (int64_t)(mf::part_dstride_for(head_dim) + 2);
    if (n_slices + n_segs > slices_capacity || n_merges > merges_capacity) return MF_ERR_WORKSPACE;
    if (!slices || (n_merges > 0 && !merges)) return MF_ERR_ARG;

    constexpr int R = MF_SLICE_INTS;
    for (int64_t i = 0; i < n_slices; ++i) {
        int32_t* o = slices + i * R;
        const int64_t end = i + 1 < n_slices ? begins[i + 1] : n_segs;
        std::fill(o, o + R, 0);
        o[0] = (int32_t)begins[i];
        o[1] = (int32_t)(end - begins[i]);
        o[2] = padded[i];
    }
    std::vector<int64_t> slot0(num_seqs, -1);
    int64_t slots = 0, wm = 0;
    for (int s = 0; s < num_seqs; ++s) {
        if (pieces[s] <= 1) continue;
        slot0[s] = slots;
        for (int h = 0; h < Hkv; ++h) {
            int32_t* o = merges + (wm++) * MF_PLAN_MERGE_INTS;
            o[0] = s;
            o[1] = h;
            o[2] = 0;
            o[3] = pieces[s];
            o[4] = (int32_t)(slots + (int64_t)h * pieces[s]);
            o[5] = 1;
            o[6] = cu_seqlens[s];
            o[7] = 1;
        }
        slots += (int64_t)Hkv * pieces[s];
    }
    std::vector<int> part(num_seqs, 0);
    for (int64_t i = 0; i < n_segs; ++i) {
        const Seg& g = segs[i];
        int32_t* o = slices + (n_slices + i) * R;
        o[0] = g.s;
        o[1] = g.kt0;
        o[2] = g.kt1;
        o[3] = cu_seqlens[g.s];
        o[4] = kv_lens[g.s];
        o[5] = (int32_t)slot0[g.s];
        o[6] = pieces[g.s];
        o[7] = part[g.s]++;
    }
    return MF_OK;
}

namespace {
int paged_attention_impl(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* cu_seqlens,
    const int32_t* kv_lens, const int64_t* positions, const int32_t* row_map,
    const int32_t* pool_lens, const void* new_k, const void* new_v, int64_t new_stride_row,
    int64_t new_stride_head, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    const int32_t* plan_items, int64_t num_items_narrow, int64_t num_items_wide,
    const int32_t* plan_merges, int64_t num_merges, float* partials, int64_t partials_floats,
    int32_t* merge_counters, const int32_t* device_counts, mf_stream_t stream, bool sliced = false,
    const int64_t* write_slots = nullptr, int64_t write_rows = 0, int64_t write_num_slots = 0,
    bool tail_inflight = false) {
    using namespace mf;
    if (!(std::fabs(scale) < INFINITY)) return MF_ERR_ARG;  // NaN or infinite
    if (!dtype_ok(dtype) || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads ||
        block_size <= 0 || num_items_narrow < 0 || num_items_wide < 0 || num_merges < 0)
        return MF_ERR_ARG;
    const int DP = padded_head_dim(dtype, head_dim);
    if (!DP) return MF_ERR_UNSUPPORTED;
    // A call may carry only items (partials left for a later merge-only call)
    // or only merges; both are how a caller times the two kernels apart.
    if (num_items_narrow + num_items_wide == 0 && num_merges == 0 && write_rows == 0) return MF_OK;
    if (!q || !out || !k_pool || !v_pool || !block_tables || !cu_seqlens || !kv_lens || !positions)
        return MF_ERR_ARG;
    if (num_items_narrow + num_items_wide > 0 && !plan_items) return MF_ERR_ARG;
    // Range-plan items run in workgroups of four and a wave loads its item
    // before its count check: both counts are whole workgroups, as plans make
    // them (a slice plan's counts are slices and segments).
    if (!sliced && ((num_items_narrow % kWaves) || (num_items_wide % kWaves))) return MF_ERR_ARG;
    if (pool_lens && (!new_k || !new_v)) return MF_ERR_ARG;
    if (num_merges > 0 && (!plan_merges || !partials || partials_floats <= 0)) return MF_ERR_WORKSPACE;
    // 16-byte row loads need 16-byte aligned rows.
    const int es = dtype_size(dtype);
    const int64_t epl = 16 / es;
    const int64_t strides[] = {q_stride_row, q_stride_head, pool_stride_block, pool_stride_slot,
                               pool_stride_head};
    for (int64_t st : strides)
        if (st % epl) return MF_ERR_ARG;
    if (((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool) & 15) return MF_ERR_ARG;
    if (pool_lens && ((new_stride_row % epl) || (new_stride_head % epl) ||
                      (((uintptr_t)new_k | (uintptr_t)new_v) & 15)))
        return MF_ERR_ARG;
    const int out_align = std::min(16, 4 * (DP / 16) * es);
    if ((out_stride_row * es) % out_align || (out_stride_head * es) % out_align ||
        ((uintptr_t)out % out_align))
        return MF_ERR_ARG;

    AttnArgs a{};
    a.q = (const char*)q;
    a.q_sr = q_stride_row;
    a.q_sh = q_stride_head;
    a.out = (char*)out;
    a.o_sr = out_stride_row;
    a.o_sh = out_stride_head;
    a.k_pool = (const char*)k_pool;
    a.v_pool = (const char*)v_pool;
    a.p_sb = pool_stride_block;
    a.p_ss = pool_stride_slot;
    a.p_sh = pool_stride_head;
    a.block_size = block_size;
    a.block_tables = block_tables;
    a.bt_stride = block_table_stride;
    a.cu_seqlens = cu_seqlens;
    a.kv_lens = kv_lens;
    a.positions = positions;
    a.row_map = row_map;
    a.pool_lens = pool_lens;
    a.new_k = (const char*)new_k;
    a.new_v = (const char*)new_v;
    a.n_sr = new_stride_row;
    a.n_sh = new_stride_head;
    a.G = num_q_heads / num_kv_heads;
    a.head_dim = head_dim;
    // Scores are scaled inside the exponent, which needs a positive factor:
    // a negative scale flips the sign of Q instead (exact), and a zero scale
    // becomes 2^-100, for which every 2^(s * scale - m) rounds to exactly 1,
    // the uniform weights a zero scale gives.
    a.q_sign = scale < 0.f ? (es == 4 ? 0x80000000u : 0x80008000u) : 0u;
    a.scale_log2 = scale == 0.f ? 0x1p-100f : std::fabs(scale) * 1.4426950408889634f;
    a.inv_scale_log2 = 1.f / a.scale_log2;
    a.partials = partials;
    a.part_dstride = part_dstride_for(head_dim);
    a.merges = plan_merges;
    a.counters = num_merges > 0 ? merge_counters : nullptr;
    a.num_kv_heads = num_kv_heads;
    const bool fast = block_size == 16 && head_dim == DP;
    hipStream_t st = (hipStream_t)stream;
    if (tail_inflight) {
        if (!new_k || !new_v || row_map || pool_lens || write_rows < 0 || write_num_slots < 0) return MF_ERR_ARG;
        if (write_rows > 0 && !write_slots) return MF_ERR_ARG;
        if ((new_stride_row % epl) || (new_stride_head % epl) || (((uintptr_t)new_k | (uintptr_t)new_v) & 15))
            return MF_ERR_ARG;
        if (!fast) {
            // other block sizes and padded head_dims: the write, then the
            // attention reading every key from the pool (same result, two launches)
            if (write_rows > 0) {
                if (int sw = mf_kv_write(new_k, new_v, dtype, new_stride_row, new_stride_head, write_slots,
                                         write_rows, const_cast<void*>(k_pool), const_cast<void*>(v_pool), dtype,
                                         pool_stride_block, pool_stride_slot, pool_stride_head, block_size,
                                         write_num_slots, num_kv_heads, head_dim, stream))
                    return sw;
            }
            tail_inflight = false;
        } else {
            // the copy: 16-byte pieces of every new row's K and V, about four
            // per thread of the copy workgroups
            const int64_t pieces = write_rows * 2 * num_kv_heads * (head_dim * es / 16);
            if (pieces > INT_MAX / 2) return MF_ERR_ARG;
            a.w_slots = write_slots;
            a.w_rows = (int)write_rows;
            a.w_num_slots = write_num_slots;
            a.w_blocks = pieces > 0 ? (int)std::min<int64_t>(1024, (pieces + 1023) / 1024) : 0;
        }
    }

    if (sliced && (!fast || row_map || pool_lens || merge_counters || device_counts || tail_inflight))
        return MF_ERR_UNSUPPORTED;
#define MF_ATTN_CASE(DT, DPV)                                                                  \
    if (dtype == DT && DP == DPV)                                                              \
        return sliced ? launch_slices<DT, DPV>(a, plan_items, num_items_narrow, num_kv_heads,  \
                                               plan_merges, num_merges, st)                    \
                      : (tail_inflight ? launch_attention<DT, DPV, true>(a, plan_items, num_items_narrow, \
                                                                         num_items_wide, plan_merges, num_merges, \
                                                                         fast, device_counts, st) \
                                       : launch_attention<DT, DPV>(a, plan_items, num_items_narrow, num_items_wide, \
                                                                   plan_merges, num_merges, fast, device_counts, st));
    MF_ATTN_CASE(MF_F32, 16)
    MF_ATTN_CASE(MF_F32, 32)
    MF_ATTN_CASE(MF_F32, 64)
    MF_ATTN_CASE(MF_F32, 128)
    MF_ATTN_CASE(MF_BF16, 32)
    MF_ATTN_CASE(MF_BF16, 64)
    MF_ATTN_CASE(MF_BF16, 128)
    MF_ATTN_CASE(MF_BF16, 256)
    MF_ATTN_CASE(MF_F16, 32)
    MF_ATTN_CASE(MF_F16, 64)
    MF_ATTN_CASE(MF_F16, 128)
    MF_ATTN_CASE(MF_F16, 256)
#undef MF_ATTN_CASE
    return MF_ERR_UNSUPPORTED;
}
}  // namespace

extern "C" int mf_paged_attention(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* cu_seqlens,
    const int32_t* kv_lens, const int64_t* positions, const int32_t* row_map,
    const int32_t* pool_lens, const void* new_k, const void* new_v, int64_t new_stride_row,
    int64_t new_stride_head, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    const int32_t* plan_items, int64_t num_items_narrow, int64_t num_items_wide,
    const int32_t* plan_merges, int64_t num_merges, float* partials, int64_t partials_floats,
    int32_t* merge_counters, mf_stream_t stream) {
    return paged_attention_impl(q, q_stride_row, q_stride_head, out, out_stride_row, out_stride_head, dtype,
                                k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                                block_size, block_tables, block_table_stride, cu_seqlens, kv_lens, positions,
                                row_map, pool_lens, new_k, new_v, new_stride_row, new_stride_head, num_q_heads,
                                num_kv_heads, head_dim, scale, plan_items, num_items_narrow, num_items_wide,
                                plan_merges, num_merges, partials, partials_floats, merge_counters, nullptr,
                                stream);
}

extern "C" int mf_paged_attention_slices(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* cu_seqlens,
    const int32_t* kv_lens, const int64_t* positions, int num_q_heads, int num_kv_heads, int head_dim,
    float scale, const int32_t* slices, int64_t num_slices, int64_t num_segments,
    const int32_t* plan_merges, int64_t num_merges, float* partials, int64_t partials_floats,
    mf_stream_t stream) {
    return paged_attention_impl(q, q_stride_row, q_stride_head, out, out_stride_row, out_stride_head, dtype,
                                k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                                block_size, block_tables, block_table_stride, cu_seqlens, kv_lens, positions,
                                nullptr, nullptr, nullptr, nullptr, 0, 0, num_q_heads, num_kv_heads, head_dim,
                                scale, slices, num_slices, num_segments, plan_merges, num_merges, partials,
                                partials_floats, nullptr, nullptr, stream, /*sliced=*/true);
}

extern "C" int mf_paged_attention_counted(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* cu_seqlens,
    const int32_t* kv_lens, const int64_t* positions, const int32_t* row_map,
    const int32_t* pool_lens, const void* new_k, const void* new_v, int64_t new_stride_row,
    int64_t new_stride_head, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    const int32_t* plan_items, int64_t capacity_narrow, int64_t capacity_wide,
    const int32_t* plan_merges, int64_t capacity_merges, const int32_t* device_counts, float* partials,
    int64_t partials_floats, mf_stream_t stream) {
    if (!device_counts) return MF_ERR_ARG;
    return paged_attention_impl(q, q_stride_row, q_stride_head, out, out_stride_row, out_stride_head, dtype,
                                k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                                block_size, block_tables, block_table_stride, cu_seqlens, kv_lens, positions,
                                row_map, pool_lens, new_k, new_v, new_stride_row, new_stride_head, num_q_heads,
                                num_kv_heads, head_dim, scale, plan_items, capacity_narrow, capacity_wide,
                                plan_merges, capacity_merges, partials, partials_floats, nullptr,
                                device_counts, stream);
}

extern "C" int mf_paged_attention_kv_write(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, void* k_pool, void* v_pool, int64_t pool_stride_block,
    int64_t pool_stride_slot, int64_t pool_stride_head, int block_size, const int32_t* block_tables,
    int64_t block_table_stride, const int32_t* cu_seqlens, const int32_t* kv_lens, const int64_t* positions,
    const void* new_k, const void* new_v, int64_t new_stride_row, int64_t new_stride_head,
    const int64_t* slot_mapping, int64_t num_new_rows, int64_t num_slots, int num_q_heads, int num_kv_heads,
    int head_dim, float scale, const int32_t* plan_items, int64_t num_items_narrow, int64_t num_items_wide,
    const int32_t* plan_merges, int64_t num_merges, const int32_t* device_counts, float* partials,
    int64_t partials_floats, mf_stream_t stream) {
    return paged_attention_impl(q, q_stride_row, q_stride_head, out, out_stride_row, out_stride_head, dtype,
                                k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                                block_size, block_tables, block_table_stride, cu_seqlens, kv_lens, positions,
                                nullptr, nullptr, new_k, new_v, new_stride_row, new_stride_head, num_q_heads,
                                num_kv_heads, head_dim, scale, plan_items, num_items_narrow, num_items_wide,
                                plan_merges, num_merges, partials, partials_floats, nullptr, device_counts,
                                stream, /*sliced=*/false, slot_mapping, num_new_rows, num_slots,
                                /*tail_inflight=*/true);
}

// ------------------------------------------------------- no-allocation entry
//
// mf_paged_attention for callers that cannot allocate device memory: the
// split-K partials go to `scratch`, a library-owned device array that every
// GPU holding this code object keeps until the process ends. In host code the
// array's name is only a stand-in for the symbol; its device address, which
// differs per GPU, comes from hipGetSymbolAddress on the first call on each
// device and is the only form host code ever passes to a kernel. Nothing in
// it needs clearing between calls (every partial slot is written before the
// merge reads it), and calls that overlap on one GPU race on it.
static __device__ __align__(256) float scratch[MF_NOALLOC_PARTIALS_FLOATS];

namespace {
constexpr int kMaxScratchDevices = 64;
std::atomic<float*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of the current device's `scratch`, looked up once per device.
int scratch_for_current_device(float** out) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {
        mf::set_last_hip_error((int)err);
        return MF_ERR_HIP;
    }
    if (dev < 0 || dev >= kMaxScratchDevices) return MF_ERR_UNSUPPORTED;
    float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* addr = nullptr;
            err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (err != hipSuccess || !addr) {
                mf::set_last_hip_error((int)err);
                return MF_ERR_HIP;
            }
            p = (float*)addr;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MF_OK;
}
}  // namespace

extern "C" int mf_paged_attention_noalloc(
    const void* q, int64_t q_stride_row, int64_t q_stride_head, void* out, int64_t out_stride_row,
    int64_t out_stride_head, int dtype, const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* cu_seqlens,
    const int32_t* kv_lens, const int64_t* positions, const int32_t* row_map,
    const int32_t* pool_lens, const void* new_k, const void* new_v, int64_t new_stride_row,
    int64_t new_stride_head, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    const int32_t* plan_items, int64_t num_items_narrow, int64_t num_items_wide,
    const int32_t* plan_merges, int64_t num_merges, int64_t partials_floats, mf_stream_t stream) {
    // sizes first: a plan that needs more than the array is refused before
    // anything touches the device
    if (partials_floats < 0) return MF_ERR_ARG;
    if (partials_floats > MF_NOALLOC_PARTIALS_FLOATS) return MF_ERR_WORKSPACE;
    float* partials = nullptr;
    if (int st = scratch_for_current_device(&partials)) return st;
    return paged_attention_impl(q, q_stride_row, q_stride_head, out, out_stride_row, out_stride_head, dtype,
                                k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                                block_size, block_tables, block_table_stride, cu_seqlens, kv_lens, positions,
                                row_map, pool_lens, new_k, new_v, new_stride_row, new_stride_head, num_q_heads,
                                num_kv_heads, head_dim, scale, plan_items, num_items_narrow, num_items_wide,
                                plan_merges, num_merges, partials, MF_NOALLOC_PARTIALS_FLOATS, nullptr,
                                nullptr, stream);
}
