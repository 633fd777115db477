// Speculative rejection sampling with caller-supplied randomness.
//
// Launch 1 (one workgroup per target row (b, i), i <= K): softmax statistics
// of logits[b][i][:V] / T -- running max and sum of exp in a single pass --
// plus the first index of the maximum logit (the greedy distribution).
// Launch 2 (one workgroup per draft row b): the sequential accept loop over
// the K candidates (one lane, double precision, exactly the reference's
// arithmetic), then the resample over the vocabulary: the residual
// max(p - q, 0), its normalisation, the second normalisation the reference's
// sample_from_probs applies, and argmax(w / E) with first-index ties, which is
// torch.multinomial(w, 1) given the same Exp(1) draws E.
// (memforge_ml/speculative/rejection_sampler.py:12-83,
//  memforge_ml/runtime/batched_speculative.py:112-124, 731-777)
#include <cfloat>
#include <climits>

#include "mf_common.h"

namespace mf {
namespace {

constexpr int kThreads = 256;

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
    float* row_max;
    float* row_sum;
    int32_t* row_argmax;
};

__device__ __forceinline__ float load_logit(const VerifyArgs& a, int b, int i, int v) {
    const int64_t off = (int64_t)b * a.tl_sr + (int64_t)i * a.tl_sp + v;
    if (a.ldt == MF_F32) return ((const float*)a.logits)[off];
    const uint32_t bits = ((const uint16_t*)a.logits)[off];
    return a.ldt == MF_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

// Block reductions (256 threads = 4 waves).
__device__ float block_sum(float v, float* sh) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// Max with the first index among equal maxima; NaN never wins.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
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
    for (int k = 1; k < 4; ++k) argmax_merge(v, i, shv[k], shi[k]);
}

__global__ __launch_bounds__(kThreads) void row_stats_kernel(VerifyArgs a) {
    __shared__ float shv[4], shs[4];
    __shared__ int shi[4];
    const int row = blockIdx.x;  // b * (K + 1) + i
    const int b = row / (a.K + 1), i = row - b * (a.K + 1);
    const float T = a.temperature;
    const float kNegInf = -__builtin_huge_valf();
    float m = kNegInf, s = 0.f;
    float am = kNegInf;
    int ai = INT_MAX;
    for (int v = threadIdx.x; v < a.V; v += kThreads) {
        const float raw = load_logit(a, b, i, v);
        argmax_merge(am, ai, raw, v);
        if (T > 0.f) {
            const float x = raw / T;
            if (x > m) { s = s * expf(m - x) + 1.f; m = x; }
            else s += expf(x - m);
        }
    }
    block_argmax(am, ai, shv, shi);
    if (T > 0.f) {
        // merge (m, s) across the block
        float gm = m;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off, 64));
        const int w = threadIdx.x >> 6;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) shv[w] = gm;
        __syncthreads();
        gm = fmaxf(fmaxf(shv[0], shv[1]), fmaxf(shv[2], shv[3]));
        const float scaled = (m == kNegInf) ? 0.f : s * expf(m - gm);
        const float tot = block_sum(scaled, shs);
        if (threadIdx.x == 0) { a.row_max[row] = gm; a.row_sum[row] = tot; }
    }
    if (threadIdx.x == 0) a.row_argmax[row] = ai;
}

// Target probability of token v at position i of row b.
__device__ __forceinline__ float target_prob(const VerifyArgs& a, int b, int i, int v) {
    if (a.target_is_probs) return load_logit(a, b, i, v);
    const int row = b * (a.K + 1) + i;
    if (a.temperature <= 0.f) return v == a.row_argmax[row] ? 1.f : 0.f;
    const float x = load_logit(a, b, i, v) / a.temperature;
    return expf(x - a.row_max[row]) / a.row_sum[row];
}

__global__ __launch_bounds__(kThreads) void decide_kernel(VerifyArgs a) {
    __shared__ float shs[4];
    __shared__ float shv[4];
    __shared__ int shi[4];
    __shared__ int s_stop, s_reject;
    const int b = blockIdx.x;
    const int K = a.K;
    if (threadIdx.x == 0) {
        int stop = K, reject = 0;
        for (int i = 0; i < K; ++i) {
            const int tok = a.draft_tokens[(int64_t)b * K + i];
            const double q = (double)a.draft_probs[(int64_t)b * a.dp_sr + (int64_t)i * a.dp_sp + tok];
            const double p = (double)target_prob(a, b, i, tok);
            const double ratio = p / (q + 1e-9);
            const double acc = ratio < 1.0 ? ratio : 1.0;
            const double r = (double)a.u_accept[(int64_t)b * K + i];
            const bool ok = r <= acc;
            a.out_tokens[(int64_t)b * (K + 1) + i] = tok;
            a.out_is_draft[(int64_t)b * (K + 1) + i] = 1;
            if (!ok) { stop = i; reject = 1; break; }
        }
        s_stop = stop;
        s_reject = reject;
    }
    __syncthreads();
    const int i = s_stop;
    const bool reject = s_reject != 0;
    const float* q = a.draft_probs + (int64_t)b * a.dp_sr + (int64_t)i * a.dp_sp;
    const float* E = a.noise + (int64_t)b * a.noise_sr;

    // w_v before sample_from_probs' own normalisation:
    //   reject with positive residual: diff_v / diff_sum
    //   otherwise: target p_v (the reject-without-residual case and the bonus)
    float diff_sum = 0.f;
    bool use_diff = false;
    if (reject) {
        float part = 0.f;
        for (int v = threadIdx.x; v < a.V; v += kThreads)
            part += fmaxf(target_prob(a, b, i, v) - q[v], 0.f);
        diff_sum = block_sum(part, shs);
        use_diff = diff_sum > 0.f;
    }
    auto weight = [&](int v) -> float {
        if (use_diff) return fmaxf(target_prob(a, b, i, v) - q[v], 0.f) / diff_sum;
        return fmaxf(target_prob(a, b, i, v), 0.f);
    };
    float part = 0.f;
    for (int v = threadIdx.x; v < a.V; v += kThreads) part += weight(v);
    const float wsum = block_sum(part, shs);
    const float uniform = 1.f / (float)a.V;
    float best = -__builtin_huge_valf();
    int best_i = INT_MAX;
    for (int v = threadIdx.x; v < a.V; v += kThreads) {
        const float pv = wsum == 0.f ? uniform : weight(v) / wsum;
        argmax_merge(best, best_i, pv / E[v], v);
    }
    block_argmax(best, best_i, shv, shi);
    if (threadIdx.x == 0) {
        a.out_tokens[(int64_t)b * (K + 1) + i] = best_i;
        a.out_is_draft[(int64_t)b * (K + 1) + i] = 0;
        a.out_count[b] = i + 1;
        a.out_num_accepted[b] = i;
    }
}

}  // namespace
}  // namespace mf

extern "C" int64_t mf_spec_verify_workspace_size(int num_rows, int num_draft) {
    if (num_rows < 0 || num_draft < 0) return 0;
    return (int64_t)num_rows * (num_draft + 1) * 3 * 4 + 256;
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
    if (num_rows < 0 || num_draft < 0 || vocab <= 0 || !dtype_ok(target_dtype)) return MF_ERR_ARG;
    if (num_rows == 0) return MF_OK;
    if (!target_logits || !exp_noise || !out_tokens || !out_is_draft || !out_count || !out_num_accepted)
        return MF_ERR_ARG;
    if (num_draft > 0 && (!draft_tokens || !draft_probs || !u_accept)) return MF_ERR_ARG;
    if (!workspace || workspace_bytes < mf_spec_verify_workspace_size(num_rows, num_draft))
        return MF_ERR_WORKSPACE;
    const int64_t nrow = (int64_t)num_rows * (num_draft + 1);
    // The residual needs draft probabilities at the stop position; with no
    // candidates the bonus row is the only draw and q is never read.
    VerifyArgs a{num_rows, num_draft, vocab, draft_tokens, draft_probs, dp_stride_row, dp_stride_pos,
                 (const char*)target_logits, target_dtype, tl_stride_row, tl_stride_pos, temperature,
                 target_is_probs, u_accept, exp_noise, noise_stride_row, out_tokens, out_is_draft, out_count,
                 out_num_accepted, (float*)workspace, (float*)workspace + nrow,
                 (int32_t*)((float*)workspace + 2 * nrow)};
    hipStream_t st = (hipStream_t)stream;
    if (!target_is_probs) {
        hipLaunchKernelGGL(row_stats_kernel, dim3((unsigned)nrow), dim3(kThreads), 0, st, a);
        if (int e = check_launch()) return e;
    }
    hipLaunchKernelGGL(decide_kernel, dim3((unsigned)num_rows), dim3(kThreads), 0, st, a);
    return check_launch();
}
