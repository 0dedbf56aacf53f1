// K4: variable-length multi-head self-attention on MFMA (head_dim 32).
//
// Restates the attention core of selfAttention (arctic.zig:660-713): per
// head, S = Q_h K_h^T, S *= 1/sqrt(head_dim), row softmax (max, exp(x-max),
// sum, divide), O_h = P V_h.  Sequences are packed back to back
// (cu_seqlens), each attends only to its own keys, so the result equals the
// reference's per-sequence unpadded forward.
//
// Design (gfx950): one workgroup per (sequence, head); its K and V^T
// (L <= 512 keys) are staged in LDS once and every wave walks 16-query
// tiles over them.  S^T = K Q^T and O^T = V^T P^T use
// v_mfma_f32_16x16x32_f16 so that each lane owns one query.  The loop is
// VALU-bound (one exp per score against 128 MFMA flops), so per score it
// spends one FMA (scale and running max folded into the exp2 argument), one
// exp2, half a max3 and half a packed convert: the row max crosses the four
// lane rows with permlane swaps, keys past the end are masked only in the
// last 64-key block, and the row sum is a third MFMA against a ones operand
// (it sums the same f16 probabilities the P V product uses).  Softmax is the
// online (running max / rescale) form; the division by the row sum happens
// once at the end.
#include "common.h"

#include <vector>

namespace {

constexpr int kHeadDim = 32;
constexpr int kMaxKeys = 512;
constexpr int K_LD = kHeadDim + 8;     // halves per K row in LDS (80 B: conflict-free 16-byte reads)
constexpr int V_LD = kMaxKeys + 8;     // halves per V^T row in LDS (1040 B: likewise)

// Where key j sits in a V^T row.  Within each 32-key group, the keys the
// PV operand of lane row g takes ({4g..4g+3} and {16+4g..16+4g+3}, the
// order the S^T accumulators hold them in) are stored at 8g..8g+7, so one
// 16-byte read fetches them.
__device__ __forceinline__ int vt_pos(int key) {
    const int j = key & 31;
    return (key & ~31) + 8 * ((j & 15) >> 2) + 4 * (j >> 4) + (j & 3);
}

__global__ void __launch_bounds__(256) attn_varlen_kernel(const _Float16 *__restrict__ qkv, int ld,
                                                          _Float16 *__restrict__ out, int ld_out,
                                                          const int *__restrict__ cu_seqlens,
                                                          const int *__restrict__ order, int n_heads,
                                                          int hidden, float scale_log2) {
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kMaxKeys * K_LD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[kHeadDim * V_LD];

    const int item = blockIdx.x / n_heads;
    const int h = blockIdx.x % n_heads;
    const int b = order ? order[item] : item;
    const int start = cu_seqlens[b];
    // the host validates lengths; the clamp keeps every LDS index in bounds regardless
    const int L = min(max(cu_seqlens[b + 1] - start, 0), kMaxKeys);
    const int Lp = (L + 63) & ~63;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    const _Float16 *qbase = qkv + (size_t)start * ld + h * kHeadDim;
    const _Float16 *kbase = qbase + hidden;
    const _Float16 *vbase = qbase + 2 * hidden;

    // keys L..Lp-1 are zero-filled: their probabilities are 0 and 0 * V must stay 0
    for (int idx = tid; idx < Lp * 4; idx += 256) {
        const int key = idx >> 2, c = (idx & 3) * 8;
        half8_t kv = {}, vv = {};
        if (key < L) {
            kv = *(const half8_t *)(kbase + (size_t)key * ld + c);
            vv = *(const half8_t *)(vbase + (size_t)key * ld + c);
        }
        *(half8_t *)(Ks + key * K_LD + c) = kv;
        const int p = vt_pos(key);
#pragma unroll
        for (int i = 0; i < 8; i++) Vt[(c + i) * V_LD + p] = vv[i];
    }
    __syncthreads();

    const int g = lane >> 4;   // lane row: k-slots 8g..8g+7, C rows 4g..4g+3
    const int ql = lane & 15;  // query (C column) owned by this lane
    const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    for (int q0 = w * 16; q0 < L; q0 += 64) {
        const int qrow = q0 + ql;
        half8_t qf = {};
        if (qrow < L) qf = *(const half8_t *)(qbase + (size_t)qrow * ld + g * 8);
        float m = -INFINITY;  // running max of the raw scores
        f32x4_t o0 = {0, 0, 0, 0}, o1 = {0, 0, 0, 0}, lsum = {0, 0, 0, 0};
        for (int kb0 = 0; kb0 < Lp; kb0 += 64) {
            f32x4_t s[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const half8_t kf = *(const half8_t *)(Ks + (kb0 + 16 * t + ql) * K_LD + g * 8);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf, f32x4_t{0, 0, 0, 0}, 0, 0, 0);
            }
            if (kb0 + 64 > L) {  // the block holding the sequence end (wave-uniform)
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (kb0 + 16 * t + 4 * g + i >= L) s[t][i] = -INFINITY;
            }
            float mx = s[0][0];
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[t][i]);
            // finite: every 64-key block below Lp holds a key < L
            const float m_new = fmaxf(m, max_over_rows(mx));
            const float mc = m_new * scale_log2;
            const float alpha = __builtin_amdgcn_exp2f((m - m_new) * scale_log2);  // 0 on the first block
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) s[t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][i], scale_log2, -mc));
            o0 *= alpha;
            o1 *= alpha;
            lsum *= alpha;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                half8_t pf;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    pf[i] = (_Float16)s[2 * st][i];
                    pf[4 + i] = (_Float16)s[2 * st + 1][i];
                }
                const int kv = kb0 + 32 * st + 8 * g;
                const half8_t va = *(const half8_t *)(Vt + ql * V_LD + kv);
                const half8_t vb = *(const half8_t *)(Vt + (16 + ql) * V_LD + kv);
                o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf, o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, pf, o1, 0, 0, 0);
                lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf, lsum, 0, 0, 0);
            }
            m = m_new;
        }
        if (qrow < L) {
            const float inv = 1.0f / lsum[0];  // every row of the ones product holds the row sum
            _Float16 *dst = out + (size_t)(start + qrow) * ld_out + h * kHeadDim + 4 * g;
            half4_t r0, r1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                r0[i] = (_Float16)(o0[i] * inv);
                r1[i] = (_Float16)(o1[i] * inv);
            }
            *(half4_t *)dst = r0;
            *(half4_t *)(dst + 16) = r1;
        }
    }
}

}  // namespace

// qkv: f16 [T, 3*hidden] (Q | K | V per token), out: f16 [T, hidden].
// order: sequence ids (longest first) so the long blocks start early.
int tzh_attention_launch(hipStream_t st, const _Float16 *qkv, _Float16 *out, const int *cu_seqlens,
                         const int *order, int batch, int n_heads, int hidden) {
    if (hidden != n_heads * kHeadDim)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "attention kernel needs head_dim 32 (hidden %d, heads %d)", hidden,
                        n_heads);
    if (batch <= 0) return TZH_OK;
    const float scale = 1.0f / sqrtf((float)kHeadDim);  // arctic.zig:649
    const float scale_log2 = scale * 1.4426950408889634f;
    hipLaunchKernelGGL(attn_varlen_kernel, dim3(batch * n_heads), dim3(256), 0, st, qkv, 3 * hidden, out, hidden,
                       cu_seqlens, order, n_heads, hidden, scale_log2);
    TZH_LAUNCHED("attn_varlen_kernel");
    return TZH_OK;
}

extern "C" int tzh_attention_varlen(tzh_ctx *ctx, const uint16_t *qkv, uint16_t *out, const int32_t *cu_seqlens,
                                    int32_t batch, int32_t n_heads, int32_t hidden) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (batch < 0 || n_heads <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad batch/heads");
    if (batch > 0 && (!qkv || !out || !cu_seqlens)) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    if (batch == 0) return TZH_OK;
    std::vector<int32_t> cu((size_t)batch + 1);
    TZH_HIP(hipMemcpyAsync(cu.data(), cu_seqlens, cu.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    if (cu[0] < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "cu_seqlens[0] is negative");
    for (int32_t b = 0; b < batch; b++) {
        const int32_t L = cu[(size_t)b + 1] - cu[(size_t)b];
        if (L < 1 || L > kMaxKeys)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "sequence %d has length %d (must be 1..%d)", b, L, kMaxKeys);
    }
    return tzh_attention_launch(ctx->stream, (const _Float16 *)qkv, (_Float16 *)out, cu_seqlens, nullptr, batch,
                                n_heads, hidden);
}
