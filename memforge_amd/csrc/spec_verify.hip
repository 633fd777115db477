// Speculative rejection sampling with caller-supplied randomness.
//
// Launch 1 (skipped when the target rows already are probabilities): softmax
// statistics of logits[b][i][:V] / T. Each row is split into 8192-element
// chunks, one 256-thread workgroup per (row, chunk), every element loaded once
// into registers with 16-byte vector loads; the workgroup writes its chunk's
// max, sum of exp(x - max) and first argmax of the raw logits.
// Launch 2 (one workgroup per (row, 2048-element chunk)): combines the chunk
// statistics of the row's K+1 target positions, runs the sequential accept
// loop over the K candidates in one lane, in double precision, exactly the
// reference's arithmetic, and takes one pass over its chunk of the stopping
// position for the final draw. The reference draws with
// torch.multinomial(w, 1), which for one sample is argmax(w / E) with Exp(1)
// draws E, where w is the residual max(p - q, 0) normalised twice (by its sum,
// then again in sample_from_probs) when the round rejected and the residual
// has mass, else the target row p normalised, or uniform when p has no mass.
// In exact arithmetic each normalisation divides every candidate by the same
// positive number and leaves the argmax where it is, so the pass keeps the
// three first-index argmaxes -- of max(p - q, 0) / E, of max(p, 0) / E and of
// 1 / E -- and whether any residual or target value is positive. In fp32 the
// reference's keys fl(fl(fl(d / S1) / S2) / E) carry two more roundings than
// fl(d / E) (and S1, S2 come from torch's own reduction order), so two
// candidates within about an ulp of each other can be ordered differently:
// the draw equals the reference's up to such near-ties (none in 1.28M seeded
// CPU draws at vocabularies 256 to 49,152). Launch 3 picks the family
// the reference's branches would take and combines the chunk winners.
// At this size the three launches are bound by dependent memory round trips,
// not bytes: the accept walk takes two (tokens with statistics, then the
// candidates' probabilities) and the draw one more. Fetching every
// position's chunk during the walk instead was measured slower on MI355X
// (C3: draw 13.9 us against 10.4 us; the extra rows cost more than the round
// trip they save).
// (memforge_ml/speculative/rejection_sampler.py:12-83,
//  memforge_ml/runtime/batched_speculative.py:112-124, 731-777)
#include <cfloat>
#include <climits>
#include <type_traits>

#include "mf_common.h"

namespace mf {
namespace {

constexpr int kStatThreads = 256;
constexpr int kStatVec = 8;                             // float4 groups per thread per chunk
constexpr int kChunk = kStatThreads * 4 * kStatVec;    // elements per statistics workgroup
constexpr int kPassThreads = 256;
constexpr int kPassVec = 2;                             // float4 groups per thread per pass chunk
constexpr int kPassChunk = kPassThreads * 4 * kPassVec;  // elements per draw-pass workgroup
constexpr int kMaxPositions = 64;                       // K + 1 target positions per row
constexpr int kStatBatch = 8;                           // chunk statistics loaded per round trip

struct VerifyArgs {
    int B, K, V;
    const int32_t* draft_tokens;
    const float* draft_probs;
    int64_t dp_sr, dp_sp;
    const char* logits;
    int ldt;
    int64_t tl_sr, tl_sp;
    float temperature;
    int target_is_probs;  // target rows are probabilities, not logits
    const float* u_accept;
    const float* noise;
    int64_t noise_sr;
    int32_t* out_tokens;
    uint8_t* out_is_draft;
    int32_t* out_count;
    int32_t* out_num_accepted;
    int nchunk;           // statistics chunks per row
    float* st_max;        // [rows][nchunk]
    float* st_sum;
    int32_t* st_arg;
    int32_t* row_stop;    // [B] stop position and whether it rejected
    int32_t* row_reject;
    int npass;            // draw-pass chunks per row
    float* part_best;     // [3][B][npass]: residual, target, uniform candidates
    int32_t* part_best_i;
    int32_t* part_any;    // [B][npass]: bit 0 some residual > 0, bit 1 some target p > 0
    int vec_logits, vec_q, vec_e;  // rows are aligned for vector loads
};

__device__ __forceinline__ const char* logit_row(const VerifyArgs& a, int b, int i) {
    const int es = a.ldt == MF_F32 ? 4 : 2;
    return a.logits + ((int64_t)b * a.tl_sr + (int64_t)i * a.tl_sp) * es;
}

__device__ __forceinline__ float logit_at(const VerifyArgs& a, const char* row, int v) {
    if (a.ldt == MF_F32) return ((const float*)row)[v];
    const uint32_t bits = ((const uint16_t*)row)[v];
    return a.ldt == MF_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

template <int DT>
__device__ __forceinline__ float logit_at_t(const VerifyArgs& a, int b, int i, int v) {
    constexpr int ES = DT == MF_F32 ? 4 : 2;
    const char* row = a.logits + ((int64_t)b * a.tl_sr + (int64_t)i * a.tl_sp) * ES;
    if constexpr (DT == MF_F32) return ((const float*)row)[v];
    else return bits_to_f32<DT>(((const uint16_t*)row)[v]);
}

// Four consecutive logits starting at e (e % 4 == 0); elements >= V read as 0
// and must be masked by the caller.
__device__ __forceinline__ void logits4(const VerifyArgs& a, const char* row, int e, float (&x)[4]) {
    if (a.vec_logits && e + 3 < a.V) {
        if (a.ldt == MF_F32) {
            const float4 f = *(const float4*)((const float*)row + e);
            x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
        } else {
            const uint2 u = *(const uint2*)((const uint16_t*)row + e);
            const uint32_t w[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                x[k] = a.ldt == MF_BF16 ? bf16_bits_to_f32(w[k]) : f16_bits_to_f32(w[k]);
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = e + k < a.V ? logit_at(a, row, e + k) : 0.f;
}

__device__ __forceinline__ void floats4(const float* row, int e, int V, int vec, float (&x)[4]) {
    if (vec && e + 3 < V) {
        const float4 f = *(const float4*)(row + e);
        x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = e + k < V ? row[e + k] : 0.f;
}

// N groups of 4 consecutive values at e0 + u * stride, all in bounds and
// aligned: unconditional vector loads, all issued before any is used.
template <int DT, int N>
__device__ __forceinline__ void vload_logits(const char* row, int e0, int stride, float (&x)[N][4]) {
    if constexpr (DT == MF_F32) {
        float4 f[N];
#pragma unroll
        for (int u = 0; u < N; ++u) f[u] = *(const float4*)((const float*)row + e0 + u * stride);
#pragma unroll
        for (int u = 0; u < N; ++u) { x[u][0] = f[u].x; x[u][1] = f[u].y; x[u][2] = f[u].z; x[u][3] = f[u].w; }
    } else {
        uint2 w[N];
#pragma unroll
        for (int u = 0; u < N; ++u) w[u] = *(const uint2*)((const uint16_t*)row + e0 + u * stride);
#pragma unroll
        for (int u = 0; u < N; ++u) {
            x[u][0] = bits_to_f32<DT>(w[u].x & 0xffffu);
            x[u][1] = bits_to_f32<DT>(w[u].x >> 16);
            x[u][2] = bits_to_f32<DT>(w[u].y & 0xffffu);
            x[u][3] = bits_to_f32<DT>(w[u].y >> 16);
        }
    }
}

template <int N>
__device__ __forceinline__ void vload_floats(const float* row, int e0, int stride, float (&x)[N][4]) {
    float4 f[N];
#pragma unroll
    for (int u = 0; u < N; ++u) f[u] = *(const float4*)(row + e0 + u * stride);
#pragma unroll
    for (int u = 0; u < N; ++u) { x[u][0] = f[u].x; x[u][1] = f[u].y; x[u][2] = f[u].z; x[u][3] = f[u].w; }
}

// Max with the first index among equal maxima; NaN never wins.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    const bool take = ov > v || (ov == v && oi < i);  // selects, not a branch
    v = take ? ov : v;
    i = take ? oi : i;
}

template <int NW>
__device__ float block_sum(float v, float* sh) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < NW; ++k) t += sh[k];
    return t;
}

template <int NW>
__device__ void block_argmax(float& v, int& i, float* shv, int* shi) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        argmax_merge(v, i, ov, oi);
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { shv[w] = v; shi[w] = i; }
    __syncthreads();
    v = shv[0]; i = shi[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) argmax_merge(v, i, shv[k], shi[k]);
}

template <int DT>
__global__ __launch_bounds__(kStatThreads) void row_stats_kernel(VerifyArgs a) {
    __shared__ float shv[4], shs[4];
    __shared__ int shi[4];
    const int c = blockIdx.x;    // chunk of the row
    const int row = blockIdx.y;  // b * (K + 1) + i
    const int b = row / (a.K + 1), i = row - b * (a.K + 1);
    const char* lrow = logit_row(a, b, i);
    const float T = a.temperature;
    const float kNegInf = -__builtin_huge_valf();
    const int base = c * kChunk + threadIdx.x * 4;

    float raw[kStatVec][4];
    if (a.vec_logits && (c + 1) * kChunk <= a.V) {
        vload_logits<DT, kStatVec>(lrow, base, kStatThreads * 4, raw);
    } else {
#pragma unroll
        for (int u = 0; u < kStatVec; ++u) logits4(a, lrow, base + u * kStatThreads * 4, raw[u]);
    }

    // argmax and max of the raw logits; x = raw / T is monotone in raw for
    // T > 0, so max(raw / T) is max(raw) / T exactly and is divided once.
    float am = kNegInf;
    int ai = INT_MAX;
#pragma unroll
    for (int u = 0; u < kStatVec; ++u) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = base + u * kStatThreads * 4 + k;
            if (e < a.V) argmax_merge(am, ai, raw[u][k], e);
        }
    }
    const float raw_max = am;  // this lane's max (NaN never wins)
    block_argmax<4>(am, ai, shv, shi);
    if (T > 0.f) {
        const bool unit = T == 1.f;
        const float m = raw_max == kNegInf ? kNegInf : (unit ? raw_max : raw_max / T);
        float s = 0.f;
        if (m != kNegInf) {
#pragma unroll
            for (int u = 0; u < kStatVec; ++u) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int e = base + u * kStatThreads * 4 + k;
                    if (e < a.V) s += expf((unit ? raw[u][k] : raw[u][k] / T) - m);
                }
            }
        }
        // the chunk's max of x / T is its max raw logit (the argmax above,
        // every thread holding it) divided once: division by T > 0 is
        // monotone, so no second max reduction is needed
        const float gm = am == kNegInf ? kNegInf : (unit ? am : am / T);
        const float scaled = (m == kNegInf) ? 0.f : s * expf(m - gm);
        const float tot = block_sum<4>(scaled, shs);
        if (threadIdx.x == 0) {
            a.st_max[(int64_t)row * a.nchunk + c] = gm;
            a.st_sum[(int64_t)row * a.nchunk + c] = tot;
        }
    } else if (threadIdx.x == 0) {
        // greedy: the chunk's largest raw logit, so the row's argmax combines
        // from the statistics alone
        a.st_max[(int64_t)row * a.nchunk + c] = am;
    }
    if (threadIdx.x == 0) a.st_arg[(int64_t)row * a.nchunk + c] = ai;
}

// Combined softmax statistics of the row's K+1 target positions (lane i
// combines position i's chunks), then the sequential accept loop (lane 0,
// double precision). Every workgroup of the row runs this -- it reads
// (K+1) x chunks statistics and K probabilities -- and the chunk-0 workgroup
// publishes the accepted tokens and the stopping position.
//
// Two round trips: the candidate tokens, uniforms and the first kStatBatch
// chunk statistics go out together; the candidates' draft and target
// probabilities follow once the tokens are in. Every lane issues the loads,
// at clamped positions (a lane past the last candidate or position repeats
// the last one; with no draft the candidate loads read stand-in buffers and
// are ignored), so none sits behind a branch: the compiler's wait counts are
// only exact for loads on every path.
template <int DT>
__device__ __forceinline__ void accept_row(const VerifyArgs& a, int b, float* s_max, float* s_sum, int* s_arg,
                                           int* s_stop, int* s_reject, bool publish) {
    const int K = a.K;
    const float T = a.temperature;
    const float kNegInf = -__builtin_huge_valf();
    const int lane = threadIdx.x;
    const bool cand = lane < K;
    const bool stat = !a.target_is_probs && lane < K + 1;
    const int lk = min(lane, max(K - 1, 0));
    const int tok = a.draft_tokens[(int64_t)b * K + lk];
    const float u = a.u_accept[(int64_t)b * K + lk];
    const int64_t o = (int64_t)(b * (K + 1) + min(lane, K)) * a.nchunk;
    float cm[kStatBatch], cs[kStatBatch];
    int ca[kStatBatch];
#pragma unroll
    for (int k = 0; k < kStatBatch; ++k) {
        const int c = min(k, a.nchunk - 1);  // clamped duplicates are masked below
        cm[k] = a.st_max[o + c];
        cs[k] = a.st_sum[o + c];
        ca[k] = a.st_arg[o + c];
    }
    // the address only: a token outside the vocabulary reads an entry in it
    const int tk = min(max(tok, 0), a.V - 1);
    const float q = a.draft_probs[(int64_t)b * a.dp_sr + (int64_t)lk * a.dp_sp + tk];
    const float raw = logit_at_t<DT>(a, b, lk, tk);
    // position `lane`'s row: max and sum of exp(x / T - max) (T > 0), or the
    // first argmax of the raw logits (T <= 0)
    float gm = kNegInf, tot = 0.f, v = kNegInf;
    int arg = INT_MAX;
    // Both readings of the statistics are combined, without branches (the
    // caller keeps the one its temperature needs): running max and sum of
    // the scaled rows, and the first argmax of the raw rows. The clamped
    // duplicate chunks change neither max nor argmax; only the sum masks them.
    auto combine = [&](int n) {
        float bm = gm;
#pragma unroll
        for (int k = 0; k < kStatBatch; ++k) bm = fmaxf(bm, cm[k]);
        float t = gm == kNegInf ? 0.f : tot * expf(gm - bm);
#pragma unroll
        for (int k = 0; k < kStatBatch; ++k) {
            const float e = expf(cm[k] - bm);
            t += (k < n && cm[k] != kNegInf) ? cs[k] * e : 0.f;
        }
        gm = bm;
        tot = t;
#pragma unroll
        for (int k = 0; k < kStatBatch; ++k) argmax_merge(v, arg, cm[k], ca[k]);
    };
    // Every lane combines (its clamped position's) statistics, and only the
    // statistics lanes keep the result: behind a lane condition the compiler
    // would sink the loads into the condition, after the candidate loads.
    combine(min(kStatBatch, a.nchunk));
    for (int c0 = kStatBatch; c0 < a.nchunk; c0 += kStatBatch) {
#pragma unroll
        for (int k = 0; k < kStatBatch; ++k) {
            const int c = min(c0 + k, a.nchunk - 1);
            cm[k] = a.st_max[o + c];
            cs[k] = a.st_sum[o + c];
            ca[k] = a.st_arg[o + c];
        }
        combine(min(kStatBatch, a.nchunk - c0));
    }
    if (stat) {
        s_max[lane] = gm;
        s_sum[lane] = tot;
        s_arg[lane] = arg;
    }
    __shared__ int s_tok[kMaxPositions];
    __shared__ float s_q[kMaxPositions], s_p[kMaxPositions], s_u[kMaxPositions];
    if (cand) {
        float pf;
        if (a.target_is_probs) pf = raw;
        else if (T <= 0.f) pf = tok == arg ? 1.f : 0.f;
        else pf = expf((T == 1.f ? raw : raw / T) - gm) / tot;
        s_tok[lane] = tok;
        s_q[lane] = q;
        s_p[lane] = pf;
        s_u[lane] = u;
    }
    __syncthreads();
    if (lane == 0) {
        int stop = K, reject = 0;
        for (int i = 0; i < K; ++i) {
            const int tk = s_tok[i];
            const double qd = (double)s_q[i];
            const double p = (double)s_p[i];
            const double ratio = p / (qd + 1e-9);
            const double acc = ratio < 1.0 ? ratio : 1.0;
            const double r = (double)s_u[i];
            if (publish) {
                a.out_tokens[(int64_t)b * (K + 1) + i] = tk;
                a.out_is_draft[(int64_t)b * (K + 1) + i] = 1;
            }
            if (!(r <= acc)) { stop = i; reject = 1; break; }
        }
        *s_stop = stop;
        *s_reject = reject;
        if (publish) {
            a.row_stop[b] = stop;
            a.row_reject[b] = reject;
        }
    }
    __syncthreads();
}

// The draw's pass over one (chunk, row): first-index argmaxes of the three
// candidate families at the stopping position (residual only when the round
// rejected), and the chunk's "has mass" bits.
template <int DT>
__global__ __launch_bounds__(kPassThreads) void draw_kernel(VerifyArgs a) {
    __shared__ float s_max[kMaxPositions], s_sum[kMaxPositions];
    __shared__ int s_arg[kMaxPositions];
    __shared__ int s_stop, s_reject;
    const int c = blockIdx.x, b = blockIdx.y;
    accept_row<DT>(a, b, s_max, s_sum, s_arg, &s_stop, &s_reject, c == 0);
    const int i = __builtin_amdgcn_readfirstlane(s_stop);
    const bool reject = __builtin_amdgcn_readfirstlane(s_reject) != 0;
    // the stopping position's softmax statistics, as accept_row combined them
    // (the draw's candidates only need their order, so the softmax divides
    // by its sum through one reciprocal; the accept test above used the
    // reference's exact division)
    const float inv_sum = 1.f / s_sum[i];
    auto tprob = [&](float raw, int v) -> float {
        if (a.target_is_probs) return raw;
        if (a.temperature <= 0.f) return v == s_arg[i] ? 1.f : 0.f;
        const float x = a.temperature == 1.f ? raw : raw / a.temperature;
        return expf(x - s_max[i]) * inv_sum;
    };
    const char* lrow = logit_row(a, b, i);
    const float* q = a.draft_probs + (int64_t)b * a.dp_sr + (int64_t)i * a.dp_sp;
    const float* Erow = a.noise + (int64_t)b * a.noise_sr;
    const int base = c * kPassChunk + threadIdx.x * 4;
    float x[kPassVec][4], qq[kPassVec][4], en[kPassVec][4];
    if ((c + 1) * kPassChunk <= a.V && a.vec_logits && (a.vec_q || !reject) && a.vec_e) {
        vload_logits<DT, kPassVec>(lrow, base, kPassThreads * 4, x);
        if (reject) vload_floats<kPassVec>(q, base, kPassThreads * 4, qq);
        vload_floats<kPassVec>(Erow, base, kPassThreads * 4, en);
    } else {
#pragma unroll
        for (int u = 0; u < kPassVec; ++u) {
            const int e = base + u * kPassThreads * 4;
            logits4(a, lrow, e, x[u]);
            if (reject) floats4(q, e, a.V, a.vec_q, qq[u]);
            floats4(Erow, e, a.V, a.vec_e, en[u]);
        }
    }
    const float kNegInf = -__builtin_huge_valf();
    float best[3] = {kNegInf, kNegInf, kNegInf};
    int best_i[3] = {INT_MAX, INT_MAX, INT_MAX};
    int any = 0;
#pragma unroll
    for (int u = 0; u < kPassVec; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = base + u * kPassThreads * 4 + k;
            if (e >= a.V) continue;
            // keys are correctly rounded quotients w / E, as torch.multinomial's
            // exponential race forms them (one rounding, not a reciprocal
            // and a product)
            const float p = tprob(x[u][k], e);
            if (reject) {
                const float d = fmaxf(p - qq[u][k], 0.f);
                any |= d > 0.f ? 1 : 0;
                argmax_merge(best[0], best_i[0], d / en[u][k], e);
            }
            const float w = fmaxf(p, 0.f);
            any |= w > 0.f ? 2 : 0;
            argmax_merge(best[1], best_i[1], w / en[u][k], e);
            argmax_merge(best[2], best_i[2], 1.f / en[u][k], e);
        }
    const int64_t po = (int64_t)b * a.npass + c;
    const int64_t fam = (int64_t)a.B * a.npass;
    // the three families' winners and the mass bits: each wave's by
    // shuffles, then the waves' through LDS in one round (the first-index
    // argmax order is total, so any combining order gives the same winner)
    constexpr int NW = kPassThreads / 64;
    __shared__ float s_best[3][NW];
    __shared__ int s_best_i[3][NW], s_any[NW];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        any |= __shfl_xor(any, off, 64);
#pragma unroll
        for (int f = 0; f < 3; ++f) {
            const float ov = __shfl_xor(best[f], off, 64);
            const int oi = __shfl_xor(best_i[f], off, 64);
            argmax_merge(best[f], best_i[f], ov, oi);
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int f = 0; f < 3; ++f) {
            s_best[f][w] = best[f];
            s_best_i[f][w] = best_i[f];
        }
        s_any[w] = any;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            t |= s_any[k];
            if (k > 0) {
#pragma unroll
                for (int f = 0; f < 3; ++f) argmax_merge(best[f], best_i[f], s_best[f][k], s_best_i[f][k]);
            }
        }
#pragma unroll
        for (int f = 0; f < 3; ++f) {
            a.part_best[f * fam + po] = best[f];
            a.part_best_i[f * fam + po] = best_i[f];
        }
        a.part_any[po] = t;
    }
}

// Combine each row's chunk winners (a kernel boundary, not a per-workgroup
// release fence: on this multi-XCD part a device-scope fence writes back L2).
// One wave per row: lane k takes chunks k, k + 64, ..., with every load of a
// chunk issued together, and the wave reduces by shuffles (the first-index
// argmax order is total, so any combining order gives the same winner).
// The family is the reference's branch: the residual when the round rejected
// and the residual has mass, else the target row, else uniform.
__global__ __launch_bounds__(64) void finish_kernel(VerifyArgs a) {
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    const int K = a.K;
    const int i = a.row_stop[b];
    const int rejected = a.row_reject[b];
    const int64_t po = (int64_t)b * a.npass;
    const int64_t fam = (int64_t)a.B * a.npass;
    int any = 0;
    float best[3] = {-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf()};
    int best_i[3] = {INT_MAX, INT_MAX, INT_MAX};
    for (int k = lane; k < a.npass; k += 64) {
        any |= a.part_any[po + k];
#pragma unroll
        for (int f = 0; f < 3; ++f) argmax_merge(best[f], best_i[f], a.part_best[f * fam + po + k],
                                                 a.part_best_i[f * fam + po + k]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        any |= __shfl_xor(any, off, 64);
#pragma unroll
        for (int f = 0; f < 3; ++f) {
            const float ov = __shfl_xor(best[f], off, 64);
            const int oi = __shfl_xor(best_i[f], off, 64);
            argmax_merge(best[f], best_i[f], ov, oi);
        }
    }
    if (lane != 0) return;
    const int f = (rejected && (any & 1)) ? 0 : ((any & 2) ? 1 : 2);
    const int tok = f == 0 ? best_i[0] : (f == 1 ? best_i[1] : best_i[2]);
    a.out_tokens[(int64_t)b * (K + 1) + i] = tok;
    a.out_is_draft[(int64_t)b * (K + 1) + i] = 0;
    a.out_count[b] = i + 1;
    a.out_num_accepted[b] = i;
}

inline int chunks_for(int vocab) { return (vocab + kChunk - 1) / kChunk; }
inline int pass_chunks_for(int vocab) { return (vocab + kPassChunk - 1) / kPassChunk; }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace mf

namespace {
struct Layout {
    int64_t st, rows, pass;  // float/int slots of each section
    int64_t total_bytes;
};
inline Layout layout_for(int64_t num_rows, int num_draft) {
    // sized for a vocabulary of up to 2^20 entries
    const int64_t rows = num_rows * (num_draft + 1);
    Layout l;
    l.st = rows * mf::chunks_for(1 << 20);
    l.rows = num_rows;
    l.pass = num_rows * mf::pass_chunks_for(1 << 20);
    l.total_bytes = (3 * l.st + 2 * l.rows + 7 * l.pass) * 4 + 256;
    return l;
}
}  // namespace

extern "C" int64_t mf_spec_verify_workspace_size(int num_rows, int num_draft) {
    if (num_rows < 0 || num_draft < 0) return 0;
    return layout_for(num_rows, num_draft).total_bytes;
}

extern "C" int mf_spec_verify(int num_rows, int num_draft, int vocab, const int32_t* draft_tokens,
                              const float* draft_probs, int64_t dp_stride_row, int64_t dp_stride_pos,
                              const void* target_logits, int target_dtype, int64_t tl_stride_row,
                              int64_t tl_stride_pos, float temperature, int target_is_probs,
                              const float* u_accept,
                              const float* exp_noise, int64_t noise_stride_row, int32_t* out_tokens,
                              uint8_t* out_is_draft, int32_t* out_count, int32_t* out_num_accepted,
                              void* workspace, int64_t workspace_bytes, mf_stream_t stream) {
    using namespace mf;
    if (num_rows < 0 || num_draft < 0 || vocab <= 0 || vocab > (1 << 20) || !dtype_ok(target_dtype))
        return MF_ERR_ARG;
    if (num_draft + 1 > kMaxPositions) return MF_ERR_UNSUPPORTED;
    if (num_rows == 0) return MF_OK;
    if (!target_logits || !exp_noise || !out_tokens || !out_is_draft || !out_count || !out_num_accepted)
        return MF_ERR_ARG;
    if (num_draft > 0 && (!draft_tokens || !draft_probs || !u_accept)) return MF_ERR_ARG;
    if (!workspace || workspace_bytes < mf_spec_verify_workspace_size(num_rows, num_draft))
        return MF_ERR_WORKSPACE;
    const int64_t nrow = (int64_t)num_rows * (num_draft + 1);
    const int nchunk = chunks_for(vocab);
    // a vector load covers 4 elements: 16 bytes of fp32, 8 bytes of bf16/f16
    const int es = target_dtype == MF_F32 ? 4 : 2;
    const bool vec_logits = ((uintptr_t)target_logits % (4 * es)) == 0 && (tl_stride_row % 4) == 0 &&
                            (tl_stride_pos % 4) == 0;
    const bool vec_q = num_draft == 0 ||
                       (aligned16(draft_probs) && (dp_stride_row % 4) == 0 && (dp_stride_pos % 4) == 0);
    const bool vec_e = aligned16(exp_noise) && (noise_stride_row % 4) == 0;
    const Layout l = layout_for(num_rows, num_draft);
    const int npass = pass_chunks_for(vocab);
    float* ws = (float*)workspace;
    float* p = ws;
    auto take = [&](int64_t n) { float* r = p; p += n; return r; };
    float* st_max = take(l.st);
    float* st_sum = take(l.st);
    int32_t* st_arg = (int32_t*)take(l.st);
    int32_t* row_stop = (int32_t*)take(l.rows);
    int32_t* row_reject = (int32_t*)take(l.rows);
    float* part_best = take(3 * l.pass);
    int32_t* part_best_i = (int32_t*)take(3 * l.pass);
    int32_t* part_any = (int32_t*)take(l.pass);
    if (num_draft == 0) {
        // every lane of the accept walk loads a candidate unconditionally;
        // with no draft those loads read these in-bounds stand-ins (a token
        // from the workspace, then an entry of noise row 0, which holds at
        // least `vocab` values) and are ignored
        draft_tokens = row_stop;
        u_accept = st_max;
        draft_probs = exp_noise;
        dp_stride_row = dp_stride_pos = 0;
    }
    VerifyArgs a{num_rows, num_draft, vocab, draft_tokens, draft_probs, dp_stride_row, dp_stride_pos,
                 (const char*)target_logits, target_dtype, tl_stride_row, tl_stride_pos, temperature,
                 target_is_probs, u_accept, exp_noise, noise_stride_row, out_tokens, out_is_draft, out_count,
                 out_num_accepted, nchunk, st_max, st_sum, st_arg, row_stop,
                 row_reject, npass, part_best, part_best_i, part_any,
                 vec_logits ? 1 : 0, vec_q ? 1 : 0, vec_e ? 1 : 0};
    hipStream_t st = (hipStream_t)stream;
    auto run = [&](auto dt_tag) -> int {
        constexpr int DT = decltype(dt_tag)::value;
        if (!target_is_probs) {
            hipLaunchKernelGGL(row_stats_kernel<DT>, dim3((unsigned)nchunk, (unsigned)nrow), dim3(kStatThreads), 0,
                               st, a);
            if (int e = check_launch()) return e;
        }
        const dim3 grid((unsigned)npass, (unsigned)num_rows);
        hipLaunchKernelGGL((draw_kernel<DT>), grid, dim3(kPassThreads), 0, st, a);
        if (int e = check_launch()) return e;
        hipLaunchKernelGGL(finish_kernel, dim3((unsigned)num_rows), dim3(64), 0, st, a);
        return check_launch();
    };
    if (target_dtype == MF_F32) return run(std::integral_constant<int, MF_F32>{});
    if (target_dtype == MF_BF16) return run(std::integral_constant<int, MF_BF16>{});
    return run(std::integral_constant<int, MF_F16>{});
}
