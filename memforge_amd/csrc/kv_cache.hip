// KV write (slot_mapping scatter) and KV gather for the paged pool.
//
// One thread moves one chunk of VW consecutive head_dim elements of one
// (token, head) pair for both K and V, so a wave covers whole 16-byte runs of
// the pool row and the HBM traffic is exactly the bytes moved. The copy is a
// pure permutation plus an optional dtype conversion (round to nearest even),
// which makes it bit-identical to torch's index_copy_ / index_select of the
// same data (memforge_ml/kernels/paged_gather.py:58-117).
#include "mf_common.h"

namespace mf {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads N bytes (N in {2,4,8,16,32}) into 32-bit words; NT marks the loads
// non-temporal (measured slower for the 128-byte pool rows of a gather, so
// the gather does not use it).
template <int N, bool NT = false>
__device__ __forceinline__ void load_words(const char* p, uint32_t* w) {
    if constexpr (N == 2) {
        w[0] = NT ? __builtin_nontemporal_load((const uint16_t*)p) : *(const uint16_t*)p;
    } else if constexpr (N == 4) {
        w[0] = NT ? __builtin_nontemporal_load((const uint32_t*)p) : *(const uint32_t*)p;
    } else if constexpr (N == 8) {
        const u32x2 v = NT ? __builtin_nontemporal_load((const u32x2*)p) : *(const u32x2*)p;
        w[0] = v.x; w[1] = v.y;
    } else {
        static_assert(N == 16 || N == 32, "chunk size");
#pragma unroll
        for (int k = 0; k < N / 16; ++k) {
            const u32x4 v = NT ? __builtin_nontemporal_load((const u32x4*)(p + 16 * k)) : *(const u32x4*)(p + 16 * k);
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    }
}

// Stores 32-bit words as N bytes; NT marks the stores non-temporal (measured
// slower for the pool side of a write on MI355X, so the write path does not
// use it).
template <int N, bool NT = false>
__device__ __forceinline__ void store_words(char* p, const uint32_t* w) {
    if constexpr (N == 2) {
        if (NT) __builtin_nontemporal_store((uint16_t)w[0], (uint16_t*)p);
        else *(uint16_t*)p = (uint16_t)w[0];
    } else if constexpr (N == 4) {
        if (NT) __builtin_nontemporal_store(w[0], (uint32_t*)p);
        else *(uint32_t*)p = w[0];
    } else if constexpr (N == 8) {
        const u32x2 v = {w[0], w[1]};
        if (NT) __builtin_nontemporal_store(v, (u32x2*)p);
        else *(u32x2*)p = v;
    } else {
        static_assert(N == 16 || N == 32, "chunk size");
#pragma unroll
        for (int k = 0; k < N / 16; ++k) {
            const u32x4 v = {w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
            if (NT) __builtin_nontemporal_store(v, (u32x4*)(p + 16 * k));
            else *(u32x4*)(p + 16 * k) = v;
        }
    }
}

template <int ES>
__device__ __forceinline__ uint32_t get_elem(const uint32_t* w, int e) {
    if constexpr (ES == 4) return w[e];
    else return (w[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
}
template <int ES>
__device__ __forceinline__ void set_elem(uint32_t* w, int e, uint32_t v) {
    if constexpr (ES == 4) {
        w[e] = v;
    } else {
        const int sh = (e & 1) * 16;
        w[e >> 1] = (w[e >> 1] & ~(0xffffu << sh)) | (v << sh);
    }
}

// Copies VW elements from `src` (dtype SDT) to `dst` (dtype DDT); NT_LOAD /
// NT_STORE mark the pool side non-temporal.
template <int SDT, int DDT, int VW, bool NT_LOAD, bool NT_STORE>
__device__ __forceinline__ void copy_chunk(const char* src, char* dst) {
    constexpr int SES = SDT == MF_F32 ? 4 : 2;
    constexpr int DES = DDT == MF_F32 ? 4 : 2;
    uint32_t in[(VW * SES + 3) / 4];
    load_words<VW * SES, NT_LOAD>(src, in);
    if constexpr (SDT == DDT) {
        store_words<VW * DES, NT_STORE>(dst, in);
    } else {
        uint32_t out[(VW * DES + 3) / 4] = {};
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            const float f = bits_to_f32<SDT>(get_elem<SES>(in, e));
            set_elem<DES>(out, e, f32_to_bits<DDT>(f));
        }
        store_words<VW * DES, NT_STORE>(dst, out);
    }
}

struct CopyArgs {
    const char* row_k;   // contiguous-row side (source of a write, dest of a gather)
    const char* row_v;
    int64_t row_st, row_sh;  // elements
    char* pool_k;
    char* pool_v;
    int64_t p_sb, p_ss, p_sh;  // elements
    const int64_t* slots;
    int64_t num_tokens;
    int64_t num_slots;  // slots of one pool layer; rows outside [0, num_slots) are skipped
    int block_size, num_heads, head_dim;
};

// GATHER=false: rows -> pool (write). GATHER=true: pool -> rows (gather).
template <int RDT, int PDT, int VW, bool GATHER>
__global__ __launch_bounds__(256) void kv_copy_kernel(CopyArgs a) {
    constexpr int RES = RDT == MF_F32 ? 4 : 2;
    constexpr int PES = PDT == MF_F32 ? 4 : 2;
    const int chunks = a.head_dim / VW;
    const int64_t per_tok = (int64_t)a.num_heads * chunks;
    const int64_t total = a.num_tokens * per_tok;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / per_tok;
        const int rem = (int)(idx - t * per_tok);
        const int h = rem / chunks;
        const int c = rem - h * chunks;
        const int64_t slot = a.slots[t];
        if (slot < 0 || slot >= a.num_slots) continue;
        const int64_t blk = slot / a.block_size;
        const int64_t off = slot - blk * a.block_size;
        const int64_t pe = blk * a.p_sb + off * a.p_ss + (int64_t)h * a.p_sh + (int64_t)c * VW;
        const int64_t re = t * a.row_st + (int64_t)h * a.row_sh + (int64_t)c * VW;
        if constexpr (!GATHER) {
            copy_chunk<RDT, PDT, VW, false, false>(a.row_k + re * RES, a.pool_k + pe * PES);
            copy_chunk<RDT, PDT, VW, false, false>(a.row_v + re * RES, a.pool_v + pe * PES);
        } else {
            copy_chunk<PDT, RDT, VW, false, false>(a.pool_k + pe * PES, (char*)a.row_k + re * RES);
            copy_chunk<PDT, RDT, VW, false, false>(a.pool_v + pe * PES, (char*)a.row_v + re * RES);
        }
    }
}

template <int RDT, int PDT, bool GATHER>
int launch_copy(const CopyArgs& a, hipStream_t stream) {
    // Widest chunk that keeps every access aligned: all strides and both base
    // pointers must be multiples of the chunk.
    auto aligned = [&](int vw) {
        if (a.head_dim % vw) return false;
        const int64_t strides[] = {a.row_st, a.row_sh, a.p_sb, a.p_ss, a.p_sh};
        for (int64_t s : strides)
            if (s % vw) return false;
        const uintptr_t rb = (uintptr_t)vw * (RDT == MF_F32 ? 4 : 2);
        const uintptr_t pb = (uintptr_t)vw * (PDT == MF_F32 ? 4 : 2);
        return ((uintptr_t)a.row_k % rb == 0) && ((uintptr_t)a.row_v % rb == 0) &&
               ((uintptr_t)a.pool_k % pb == 0) && ((uintptr_t)a.pool_v % pb == 0);
    };
    const int64_t total_base = a.num_tokens * a.num_heads;
    auto grid_for = [&](int vw) {
        const int64_t threads = total_base * (a.head_dim / vw);
        int64_t blocks = (threads + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        if (blocks < 1) blocks = 1;
        return (unsigned)blocks;
    };
    if (aligned(8)) {
        hipLaunchKernelGGL((kv_copy_kernel<RDT, PDT, 8, GATHER>), dim3(grid_for(8)), dim3(256), 0, stream, a);
    } else if (aligned(4)) {
        hipLaunchKernelGGL((kv_copy_kernel<RDT, PDT, 4, GATHER>), dim3(grid_for(4)), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((kv_copy_kernel<RDT, PDT, 1, GATHER>), dim3(grid_for(1)), dim3(256), 0, stream, a);
    }
    return check_launch();
}

template <bool GATHER>
int dispatch_copy(int rdt, int pdt, const CopyArgs& a, hipStream_t stream) {
#define MF_COPY_CASE(R, P) \
    if (rdt == R && pdt == P) return launch_copy<R, P, GATHER>(a, stream);
    MF_COPY_CASE(MF_F32, MF_F32)
    MF_COPY_CASE(MF_F32, MF_F16)
    MF_COPY_CASE(MF_F32, MF_BF16)
    MF_COPY_CASE(MF_F16, MF_F32)
    MF_COPY_CASE(MF_F16, MF_F16)
    MF_COPY_CASE(MF_F16, MF_BF16)
    MF_COPY_CASE(MF_BF16, MF_F32)
    MF_COPY_CASE(MF_BF16, MF_F16)
    MF_COPY_CASE(MF_BF16, MF_BF16)
#undef MF_COPY_CASE
    return MF_ERR_ARG;
}

bool copy_args_ok(const CopyArgs& a, int rdt, int pdt) {
    if (!dtype_ok(rdt) || !dtype_ok(pdt)) return false;
    if (a.num_tokens < 0 || a.num_slots < 0 || a.block_size <= 0 || a.num_heads <= 0 || a.head_dim <= 0)
        return false;
    if (a.num_tokens > 0 && (!a.row_k || !a.row_v || !a.pool_k || !a.pool_v || !a.slots)) return false;
    return true;
}

}  // namespace
}  // namespace mf

extern "C" int mf_kv_write(const void* k_src, const void* v_src, int src_dtype,
                           int64_t src_stride_t, int64_t src_stride_h,
                           const int64_t* slot_mapping, int64_t num_tokens, void* k_pool,
                           void* v_pool, int pool_dtype, int64_t pool_stride_block,
                           int64_t pool_stride_slot, int64_t pool_stride_head, int block_size,
                           int64_t num_slots, int num_heads, int head_dim, mf_stream_t stream) {
    mf::CopyArgs a{(const char*)k_src, (const char*)v_src, src_stride_t, src_stride_h,
                   (char*)k_pool, (char*)v_pool, pool_stride_block, pool_stride_slot,
                   pool_stride_head, slot_mapping, num_tokens, num_slots, block_size, num_heads,
                   head_dim};
    if (!mf::copy_args_ok(a, src_dtype, pool_dtype)) return MF_ERR_ARG;
    if (num_tokens == 0) return MF_OK;
    return mf::dispatch_copy<false>(src_dtype, pool_dtype, a, (hipStream_t)stream);
}

extern "C" int mf_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype,
                            int64_t pool_stride_block, int64_t pool_stride_slot,
                            int64_t pool_stride_head, int block_size, int64_t num_slots,
                            const int64_t* slot_mapping, int64_t num_tokens, void* k_dst,
                            void* v_dst, int dst_dtype, int64_t dst_stride_t,
                            int64_t dst_stride_h, int num_heads, int head_dim,
                            mf_stream_t stream) {
    mf::CopyArgs a{(const char*)k_dst, (const char*)v_dst, dst_stride_t, dst_stride_h,
                   (char*)k_pool, (char*)v_pool, pool_stride_block, pool_stride_slot,
                   pool_stride_head, slot_mapping, num_tokens, num_slots, block_size, num_heads,
                   head_dim};
    if (!mf::copy_args_ok(a, dst_dtype, pool_dtype)) return MF_ERR_ARG;
    if (num_tokens == 0) return MF_OK;
    return mf::dispatch_copy<true>(dst_dtype, pool_dtype, a, (hipStream_t)stream);
}

// ------------------------------------------------------------- block copy
//
// Copy-on-write data move: block `src` -> block `dst` in every layer of the K
// and V pools (memforge_ml/runtime/prefix_sharing.py:27-42). One block of one
// layer is `block_elems` contiguous elements, so the copy is a flat byte move
// in 16-byte vectors (4-byte words when the block is not 16-byte aligned).
// The pairs travel in the kernel arguments, so a call allocates nothing and
// issues no host-to-device copy.
namespace mf {
namespace {

constexpr int kCopyPairs = 32;

struct BlockCopyArgs {
    char* k;
    char* v;
    int64_t layer_bytes;  // stride between layers
    int64_t block_bytes;  // stride between blocks
    int64_t units;        // vector units per (block, layer)
    int num_layers;
    int64_t src[kCopyPairs];
    int64_t dst[kCopyPairs];
};

template <typename U>
__global__ __launch_bounds__(256) void block_copy_kernel(BlockCopyArgs a) {
    const int pair = blockIdx.z;
    const int layer = blockIdx.y >> 1;
    char* base = (blockIdx.y & 1) ? a.v : a.k;
    base += (int64_t)layer * a.layer_bytes;
    const U* s = (const U*)(base + a.src[pair] * a.block_bytes);
    U* d = (U*)(base + a.dst[pair] * a.block_bytes);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.units;
         i += (int64_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}

}  // namespace
}  // namespace mf

extern "C" int mf_kv_copy_blocks(void* k_pool, void* v_pool, int pool_dtype, int num_layers,
                                 int64_t pool_stride_layer, int64_t pool_stride_block,
                                 int64_t block_elems, int64_t num_blocks, const int64_t* pairs,
                                 int num_pairs, mf_stream_t stream) {
    if (!mf::dtype_ok(pool_dtype) || num_layers <= 0 || num_layers > 32767 || num_blocks <= 0 ||
        block_elems <= 0 || num_pairs < 0 || pool_stride_block < block_elems)
        return MF_ERR_ARG;
    if (num_layers > 1 && pool_stride_layer < num_blocks * pool_stride_block) return MF_ERR_ARG;
    if (num_pairs == 0) return MF_OK;
    if (!k_pool || !v_pool || !pairs) return MF_ERR_ARG;
    // Every index in range; no block written twice; no block both read and
    // written (the result would depend on the order of the copies).
    for (int i = 0; i < num_pairs; ++i) {
        const int64_t s = pairs[2 * i], d = pairs[2 * i + 1];
        if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return MF_ERR_ARG;
        if (s == d) continue;
        for (int j = 0; j < num_pairs; ++j) {
            if (pairs[2 * j] == pairs[2 * j + 1]) continue;
            if (j != i && pairs[2 * j + 1] == d) return MF_ERR_ARG;
            if (pairs[2 * j] == d) return MF_ERR_ARG;
        }
    }
    const int64_t es = pool_dtype == MF_F32 ? 4 : 2;
    mf::BlockCopyArgs a{};
    a.k = (char*)k_pool;
    a.v = (char*)v_pool;
    a.layer_bytes = pool_stride_layer * es;
    a.block_bytes = pool_stride_block * es;
    a.num_layers = num_layers;
    const int64_t bytes = block_elems * es;
    const bool vec16 = bytes % 16 == 0 && a.block_bytes % 16 == 0 && a.layer_bytes % 16 == 0 &&
                       (uintptr_t)k_pool % 16 == 0 && (uintptr_t)v_pool % 16 == 0;
    a.units = vec16 ? bytes / 16 : bytes / 4;
    if (!vec16 && (bytes % 4 || a.block_bytes % 4 || a.layer_bytes % 4 ||
                   (uintptr_t)k_pool % 4 || (uintptr_t)v_pool % 4))
        return MF_ERR_ARG;
    int64_t gx = (a.units + 255) / 256;
    if (gx > 1024) gx = 1024;
    for (int first = 0; first < num_pairs;) {
        int n = 0;
        for (; first < num_pairs && n < mf::kCopyPairs; ++first) {
            if (pairs[2 * first] == pairs[2 * first + 1]) continue;
            a.src[n] = pairs[2 * first];
            a.dst[n] = pairs[2 * first + 1];
            ++n;
        }
        if (n == 0) break;
        const dim3 grid((unsigned)gx, (unsigned)(2 * num_layers), (unsigned)n);
        if (vec16)
            hipLaunchKernelGGL(mf::block_copy_kernel<uint4>, grid, dim3(256), 0,
                               (hipStream_t)stream, a);
        else
            hipLaunchKernelGGL(mf::block_copy_kernel<uint32_t>, grid, dim3(256), 0,
                               (hipStream_t)stream, a);
        const int st = mf::check_launch();
        if (st != MF_OK) return st;
    }
    return MF_OK;
}
