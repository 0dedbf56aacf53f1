// K3: int8-weight GEMM on MFMA with fused epilogues.
//
//   C[i,j] = epi( (sum_k A[i,k] * f32(Wq[j,k])) * f32(scale[j]) + bias[j] )
//
// restating matmulTransposeB_f32_i8_rowScale_bias (matmul_w8a32.zig:14-57)
// and the epilogues Arctic applies after it: GELU (arctic.zig:771-776) and
// residual + LayerNorm (arctic.zig:716-746, 779-809; layernorm.zig:26-117).
//
// Design (gfx950):
//   - v_mfma_f32_32x32x16_f16 with f32 accumulation.  A is rounded to f16 on
//     its way into LDS; the int8 weights stay int8 in HBM and are dequantised
//     to f16 in registers between the global load and the LDS store (exact:
//     |q| <= 127), once per element per block, so the MFMA loop reads both
//     operands as 16-byte LDS fragments.
//   - Block tile BM x BN, BK = 64 per stage, LDS double buffer, one barrier
//     per stage; global loads for stage k+1 are in flight while stage k runs.
//   - Block index -> tile mapping is XCD-aware: each of the 8 XCDs walks a
//     contiguous range of tiles (N fastest), so the A row-panel a tile needs
//     is fetched into that XCD's L2 once and reused across the N tiles.
//   - Epilogues stage the finished tile through the (then idle) LDS so that
//     every global store is a full 16-byte vector; the LayerNorm variant owns
//     whole 384-wide rows (BN = N) and normalises one 64-row half at a time
//     from LDS with the reference's two-pass mean / biased variance.
#include "common.h"

namespace {

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // halves per LDS operand row (16-byte pad: conflict-free b128 reads)

// 16 signed bytes -> 16 f16, exact.  Each byte b becomes the f16 with bit
// pattern 0x64xx where xx = b ^ 0x80, i.e. 1024 + (b + 128); subtracting
// 1152 leaves b.
__device__ __forceinline__ void i8x16_to_f16(uint4 q, half8_t &lo, half8_t &hi) {
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    half2_t h[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t a = (w[i] & 0xffu) | ((w[i] & 0xff00u) << 8) | 0x64006400u;
        const uint32_t b = ((w[i] >> 16) & 0xffu) | ((w[i] >> 8) & 0xff0000u) | 0x64006400u;
        h[2 * i] = __builtin_bit_cast(half2_t, a) - bias;
        h[2 * i + 1] = __builtin_bit_cast(half2_t, b) - bias;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        lo[2 * i] = h[i][0];
        lo[2 * i + 1] = h[i][1];
        hi[2 * i] = h[4 + i][0];
        hi[2 * i + 1] = h[4 + i][1];
    }
}

// bijective block -> tile remap so that XCD x (block ids x, x+8, ...) owns the
// contiguous tile range [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    const int per = total / 8, rem = total % 8;
    const int x = bid % 8, local = bid / 8;
    return x < rem ? x * (per + 1) + local : rem * (per + 1) + (x - rem) * per + local;
}

template <typename TA>
struct ALoad;

// f16 activations: 16-byte chunks of 8 halves.
template <>
struct ALoad<_Float16> {
    uint4 v;
    __device__ __forceinline__ void load(const _Float16 *p, bool ok) {
        v = ok ? *(const uint4 *)p : make_uint4(0, 0, 0, 0);
    }
    __device__ __forceinline__ void store(_Float16 *lds) const { *(uint4 *)lds = v; }
};

// f32 activations: 8 floats per chunk, rounded to f16 on the way to LDS.
template <>
struct ALoad<float> {
    f32x4_t a, b;
    __device__ __forceinline__ void load(const float *p, bool ok) {
        if (ok) {
            a = *(const f32x4_t *)p;
            b = *(const f32x4_t *)(p + 4);
        } else {
            a = f32x4_t{0, 0, 0, 0};
            b = a;
        }
    }
    __device__ __forceinline__ void store(_Float16 *lds) const {
        half8_t h;
        h[0] = (_Float16)a[0]; h[1] = (_Float16)a[1]; h[2] = (_Float16)a[2]; h[3] = (_Float16)a[3];
        h[4] = (_Float16)b[0]; h[5] = (_Float16)b[1]; h[6] = (_Float16)b[2]; h[7] = (_Float16)b[3];
        *(half8_t *)lds = h;
    }
};

template <typename T>
__device__ __forceinline__ float load_f32(const T *p);
template <>
__device__ __forceinline__ float load_f32<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<_Float16>(const _Float16 *p) { return (float)*p; }

// tanh-form GELU of arctic.zig:750-756 with tanh(u) = 1 - 2 / (exp(2u) + 1)
// on the hardware exp2 (a few ulp; saturates correctly to +-1).
__device__ __forceinline__ float gelu_fast(float x) {
    const float sqrt_2_over_pi = 0.7978845608f;
    const float coeff = 0.044715f;
    const float inner = sqrt_2_over_pi * (x + coeff * x * x * x);
    const float e = __builtin_amdgcn_exp2f(inner * 2.8853900817779268f);  // exp(2u) = 2^(2u*log2 e)
    const float t = 1.0f - 2.0f / (e + 1.0f);
    return 0.5f * x * (1.0f + t);
}

template <int BM, int BN, int WM, int WN>
struct Cfg {
    static constexpr int THREADS = WM * WN * 64;
    static constexpr int TM = BM / WM / 32;  // 32-row MFMA blocks per wave
    static constexpr int TN = BN / WN / 32;  // 32-col MFMA blocks per wave
    static constexpr int A_STAGE = BM * LDK * 2;  // bytes
    static constexpr int B_STAGE = BN * LDK * 2;  // bytes (f16 after dequant)
    static constexpr int OPERAND_BYTES = 2 * (A_STAGE + B_STAGE);
    static constexpr int A_CHUNKS = BM * BK / 8 / THREADS;   // 8-element chunks of A per thread
    static constexpr int B_CHUNKS = BN * BK / 16 / THREADS;  // 16-byte int8 chunks of B per thread
    static_assert(BM * BK / 8 % THREADS == 0, "A chunks must divide evenly");
    static_assert(BN * BK / 16 % THREADS == 0, "B chunks must divide evenly");
    static_assert(TM >= 1 && TN >= 1, "wave tile too small");
};

// Main loop shared by both epilogue families.  On return acc holds the f32
// sums for the wave's TM x TN blocks of 32x32; lane l holds, for block
// (tm, tn) element j, row (j/4)*8 + (l/32)*4 + j%4 and column l%32.  The
// loop ends with a barrier, so the caller may reuse all of `smem`.
template <typename TA, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void gemm_mainloop(const TA *__restrict__ A, const int8_t *__restrict__ W, int M,
                                              int K, int m0, int n0, char *smem,
                                              f32x16_t (&acc)[Cfg<BM, BN, WM, WN>::TM][Cfg<BM, BN, WM, WN>::TN]) {
    using C = Cfg<BM, BN, WM, WN>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int wm = w / WN, wn = w % WN;

    _Float16 *As[2] = {(_Float16 *)smem, (_Float16 *)(smem + C::A_STAGE)};
    _Float16 *Bs[2] = {(_Float16 *)(smem + 2 * C::A_STAGE), (_Float16 *)(smem + 2 * C::A_STAGE + C::B_STAGE)};

#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) acc[i][j] = f32x16_t{};

    ALoad<TA> ar[C::A_CHUNKS];
    uint4 br[C::B_CHUNKS];

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int c = tid + i * C::THREADS;
            const int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
            const int gr = m0 + r;
            ar[i].load(A + (size_t)(gr < M ? gr : 0) * K + k0 + kc, gr < M);
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; i++) {
            const int c = tid + i * C::THREADS;
            const int r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            br[i] = *(const uint4 *)(W + (size_t)(n0 + r) * K + k0 + kc);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int c = tid + i * C::THREADS;
            const int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
            ar[i].store(As[buf] + r * LDK + kc);
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; i++) {
            const int c = tid + i * C::THREADS;
            const int r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            half8_t lo, hi;
            i8x16_to_f16(br[i], lo, hi);
            *(half8_t *)(Bs[buf] + r * LDK + kc) = lo;
            *(half8_t *)(Bs[buf] + r * LDK + kc + 8) = hi;
        }
    };

    const int KT = K / BK;
    gload(0);
    sstore(0);
    __syncthreads();

    const int frow = lane & 31;
    const int kgrp = (lane >> 5) * 8;
    for (int kt = 0; kt < KT; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        const _Float16 *a_s = As[cur] + (wm * C::TM * 32 + frow) * LDK + kgrp;
        const _Float16 *b_s = Bs[cur] + (wn * C::TN * 32 + frow) * LDK + kgrp;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            half8_t af[C::TM], bf[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++) af[i] = *(const half8_t *)(a_s + i * 32 * LDK + ks * 16);
#pragma unroll
            for (int j = 0; j < C::TN; j++) bf[j] = *(const half8_t *)(b_s + j * 32 * LDK + ks * 16);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }
}

// Bias (+ optional GELU) epilogue; BN | N.  The finished tile is staged in
// LDS as TC and written back with 16-byte row-contiguous stores.
template <typename TA, typename TC, bool GELU, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM *WN * 64) gemm_w8_bias_kernel(const TA *__restrict__ A,
                                                                  const int8_t *__restrict__ W,
                                                                  const uint16_t *__restrict__ scale,
                                                                  const float *__restrict__ bias,
                                                                  TC *__restrict__ Cout, int M, int K, int N) {
    using C = Cfg<BM, BN, WM, WN>;
    constexpr int O_LD = BN + 16 / (int)sizeof(TC);  // staged row pitch (elements), 16-byte pad
    static_assert(BM * O_LD * (int)sizeof(TC) <= C::OPERAND_BYTES, "output tile must fit the operand LDS");
    __shared__ __attribute__((aligned(16))) char smem[C::OPERAND_BYTES];
    const int nbn = N / BN;
    const int nbm = (M + BM - 1) / BM;
    const int t = xcd_tile(blockIdx.x, nbm * nbn);
    const int m0 = (t / nbn) * BM, n0 = (t % nbn) * BN;

    f32x16_t acc[C::TM][C::TN];
    gemm_mainloop<TA, BM, BN, WM, WN>(A, W, M, K, m0, n0, smem, acc);

    TC *O = (TC *)smem;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wm = w / WN, wn = w % WN;
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const int cl = wn * C::TN * 32 + j * 32 + (lane & 31);
        const float s = f16_bits_to_f32(scale[n0 + cl]);
        const float b = bias ? bias[n0 + cl] : 0.0f;
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int rbase = wm * C::TM * 32 + i * 32 + (lane >> 5) * 4;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                float v = acc[i][j][e] * s + b;  // sum * s + bias (matmul_w8a32.zig:55)
                if (GELU) v = gelu_fast(v);
                O[(rbase + (e >> 2) * 8 + (e & 3)) * O_LD + cl] = (TC)v;
            }
        }
    }
    __syncthreads();
    constexpr int VEC = 16 / sizeof(TC);
    constexpr int PER_ROW = BN / VEC;
    for (int idx = threadIdx.x; idx < BM * PER_ROW; idx += C::THREADS) {
        const int r = idx / PER_ROW, c = (idx % PER_ROW) * VEC;
        if (m0 + r < M) *(uint4 *)(Cout + (size_t)(m0 + r) * N + n0 + c) = *(const uint4 *)(O + r * O_LD + c);
    }
}

// Bias + residual + LayerNorm epilogue over full rows (BN == N).  The block
// is WM x WN waves; each WM slab of BM/WM rows is staged to LDS as f32 in
// turn and normalised by all waves together.
template <typename TA, typename TC, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM *WN * 64) gemm_w8_ln_kernel(
    const TA *__restrict__ A, const int8_t *__restrict__ W, const uint16_t *__restrict__ scale,
    const float *__restrict__ bias, TC *__restrict__ Cout, int M, int K, const TC *__restrict__ R,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps) {
    using C = Cfg<BM, BN, WM, WN>;
    constexpr int SLAB = BM / WM;    // rows staged at a time
    constexpr int E_LD = BN + 4;     // floats per staged row
    static_assert(SLAB * E_LD * 4 <= C::OPERAND_BYTES, "LN slab must fit the operand LDS");
    __shared__ __attribute__((aligned(16))) char smem[C::OPERAND_BYTES];
    const int nbm = (M + BM - 1) / BM;
    const int t = xcd_tile(blockIdx.x, nbm);
    const int m0 = t * BM;

    f32x16_t acc[C::TM][C::TN];
    gemm_mainloop<TA, BM, BN, WM, WN>(A, W, M, K, m0, 0, smem, acc);

    float *E = (float *)smem;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wm = w / WN, wn = w % WN;
    constexpr int NW = WM * WN;
    constexpr int PER = BN / 64;
    float g[PER], bt[PER];
#pragma unroll
    for (int q = 0; q < PER; q++) {
        g[q] = gamma[lane + 64 * q];
        bt[q] = beta[lane + 64 * q];
    }
    for (int slab = 0; slab < WM; slab++) {
        if (wm == slab) {
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int col = wn * C::TN * 32 + j * 32 + (lane & 31);
                const float s = f16_bits_to_f32(scale[col]);
                const float b = bias ? bias[col] : 0.0f;
#pragma unroll
                for (int i = 0; i < C::TM; i++) {
                    const int rbase = i * 32 + (lane >> 5) * 4;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int rl = rbase + (e >> 2) * 8 + (e & 3);
                        const int row = m0 + slab * SLAB + rl;
                        const float res = row < M ? load_f32<TC>(R + (size_t)row * BN + col) : 0.0f;
                        E[rl * E_LD + col] = res + (acc[i][j][e] * s + b);  // input + tmp (arctic.zig:720)
                    }
                }
            }
        }
        __syncthreads();
        for (int rl = w; rl < SLAB; rl += NW) {
            const int row = m0 + slab * SLAB + rl;
            if (row >= M) break;
            float x[PER];
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < PER; q++) {
                x[q] = E[rl * E_LD + lane + 64 * q];
                sum += x[q];
            }
            const float mean = wave_sum(sum) / (float)BN;
            float vs = 0.0f;
#pragma unroll
            for (int q = 0; q < PER; q++) {
                const float d = x[q] - mean;
                vs += d * d;
            }
            const float var = wave_sum(vs) / (float)BN;
            const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
            for (int q = 0; q < PER; q++)
                Cout[(size_t)row * BN + lane + 64 * q] = (TC)(((x[q] - mean) * inv_std) * g[q] + bt[q]);
        }
        __syncthreads();
    }
}

using Plain = Cfg<128, 128, 2, 2>;
using LnCfg = Cfg<128, 384, 2, 4>;

template <typename TA, typename TC>
int launch_bias(hipStream_t st, const void *a, const int8_t *wq, const uint16_t *scale, const float *bias, void *c,
                int M, int K, int N, bool gelu) {
    const int blocks = ((M + 127) / 128) * (N / 128);
    if (gelu)
        hipLaunchKernelGGL((gemm_w8_bias_kernel<TA, TC, true, 128, 128, 2, 2>), dim3(blocks), dim3(Plain::THREADS), 0,
                           st, (const TA *)a, wq, scale, bias, (TC *)c, M, K, N);
    else
        hipLaunchKernelGGL((gemm_w8_bias_kernel<TA, TC, false, 128, 128, 2, 2>), dim3(blocks), dim3(Plain::THREADS), 0,
                           st, (const TA *)a, wq, scale, bias, (TC *)c, M, K, N);
    TZH_LAUNCHED("gemm_w8_bias_kernel");
    return TZH_OK;
}

template <typename TA, typename TC>
int launch_ln(hipStream_t st, const void *a, const int8_t *wq, const uint16_t *scale, const float *bias, void *c,
              int M, int K, const void *res, const float *gamma, const float *beta, float eps) {
    const int blocks = (M + 127) / 128;
    hipLaunchKernelGGL((gemm_w8_ln_kernel<TA, TC, 128, 384, 2, 4>), dim3(blocks), dim3(LnCfg::THREADS), 0, st,
                       (const TA *)a, wq, scale, bias, (TC *)c, M, K, (const TC *)res, gamma, beta, eps);
    TZH_LAUNCHED("gemm_w8_ln_kernel");
    return TZH_OK;
}

}  // namespace

// Internal entry used by the Arctic forward and the C-ABI.
int tzh_linear_w8_launch(hipStream_t st, const void *a, int32_t a_dtype, const int8_t *wq, const uint16_t *scale,
                         const float *bias, void *c, int32_t c_dtype, int64_t m, int64_t k, int64_t n,
                         int32_t epilogue, const void *residual, int32_t res_dtype, const float *gamma,
                         const float *beta, float eps) {
    if (m < 0 || k <= 0 || n <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad GEMM shape m=%lld k=%lld n=%lld",
                                                   (long long)m, (long long)k, (long long)n);
    if (m == 0) return TZH_OK;  // matmul_w8a32.zig:24
    if (m > (int64_t)1 << 30 || k > 65536 || n > 65536) return tzh_fail(TZH_ERR_TOO_LARGE, "GEMM shape too large");
    if (k % BK) return tzh_fail(TZH_ERR_INVALID_ARGS, "k=%lld must be a multiple of %d", (long long)k, BK);
    if ((a_dtype != TZH_F32 && a_dtype != TZH_F16) || (c_dtype != TZH_F32 && c_dtype != TZH_F16))
        return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "activations must be F32 or F16");
    if (!a || !wq || !scale || !c) return tzh_fail(TZH_ERR_INVALID_ARGS, "null operand");
    const int M = (int)m, K = (int)k, N = (int)n;
    const bool a32 = a_dtype == TZH_F32, c32 = c_dtype == TZH_F32;
    if (epilogue == TZH_EPI_BIAS || epilogue == TZH_EPI_BIAS_GELU) {
        if (N % 128) return tzh_fail(TZH_ERR_INVALID_ARGS, "n=%d must be a multiple of 128", N);
        const bool g = epilogue == TZH_EPI_BIAS_GELU;
        if (a32 && c32) return launch_bias<float, float>(st, a, wq, scale, bias, c, M, K, N, g);
        if (a32 && !c32) return launch_bias<float, _Float16>(st, a, wq, scale, bias, c, M, K, N, g);
        if (!a32 && c32) return launch_bias<_Float16, float>(st, a, wq, scale, bias, c, M, K, N, g);
        return launch_bias<_Float16, _Float16>(st, a, wq, scale, bias, c, M, K, N, g);
    }
    if (epilogue == TZH_EPI_BIAS_RES_LN) {
        if (N != 384) return tzh_fail(TZH_ERR_INVALID_ARGS, "LayerNorm epilogue needs n == 384 (got %d)", N);
        if (!residual || !gamma || !beta) return tzh_fail(TZH_ERR_INVALID_ARGS, "null residual/gamma/beta");
        if (res_dtype != c_dtype) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "residual dtype must equal output dtype");
        if (a32 && c32) return launch_ln<float, float>(st, a, wq, scale, bias, c, M, K, residual, gamma, beta, eps);
        if (a32 && !c32) return launch_ln<float, _Float16>(st, a, wq, scale, bias, c, M, K, residual, gamma, beta, eps);
        if (!a32 && c32) return launch_ln<_Float16, float>(st, a, wq, scale, bias, c, M, K, residual, gamma, beta, eps);
        return launch_ln<_Float16, _Float16>(st, a, wq, scale, bias, c, M, K, residual, gamma, beta, eps);
    }
    return tzh_fail(TZH_ERR_INVALID_ARGS, "unknown epilogue %d", epilogue);
}

int tzh_widen_codes_launch(hipStream_t st, const int8_t *q, _Float16 *out, int64_t n);
int tzh_tile_codes_w8_launch(hipStream_t st, const int8_t *q, uint8_t *out, int64_t n, int64_t k);
int tzh_linear_codes_launch(hipStream_t st, int num_cus, const _Float16 *x, const void *wc, int32_t w_format,
                            const uint16_t *scale, const float *bias, void *c, int32_t c_dtype, int64_t m, int64_t k,
                            int64_t n, int32_t epilogue, const void *res, const float *gamma, const float *beta,
                            float eps, float *ln_ws, int64_t ln_ws_rows);

extern "C" int tzh_linear_w8(tzh_ctx *ctx, const void *a, int32_t a_dtype, const int8_t *wq, const uint16_t *scale,
                             const float *bias, void *c, int32_t c_dtype, int64_t m, int64_t k, int64_t n,
                             int32_t epilogue, const void *residual, int32_t res_dtype, const float *gamma,
                             const float *beta, float eps) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    // f16 activations at the shapes the pipelined kernel covers: widen the
    // codes once into the context scratch and run the model's kernel
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool pipe_shape =
        k > 0 && k % 64 == 0 && k <= 65536 && m > 0 && m <= ((int64_t)1 << 30) &&
        (((epilogue == TZH_EPI_BIAS || epilogue == TZH_EPI_BIAS_GELU) && n > 0 && n % 128 == 0 && n <= 1536) ||
         (epilogue == TZH_EPI_BIAS_RES_LN && n == 384 && residual && gamma && beta && res_dtype == c_dtype));
    if (a_dtype == TZH_F16 && (c_dtype == TZH_F16 || c_dtype == TZH_F32) && pipe_shape && a && wq && scale && c &&
        al16(a) && al16(c) && (!residual || al16(residual))) {
        // scratch: the codes in the model's format (stage-tiled biased int8
        // when n is a multiple of 384 and the output f16, else widened to
        // f16), then (LayerNorm epilogue) the f32 rows of a split partial
        // round of tiles
        const bool w8t = n % 384 == 0 && c_dtype == TZH_F16;
        const size_t codes_bytes = ((size_t)(n * k * (w8t ? 1 : 2)) + 255) / 256 * 256;
        const int64_t ws_rows = epilogue == TZH_EPI_BIAS_RES_LN
                                    ? std::min<int64_t>((m + 127) / 128, ctx->num_cus / 3 + 1) * 128
                                    : 0;
        void *scratch = nullptr;
        TZH_TRY(tzh_ctx_scratch(ctx, codes_bytes + (size_t)ws_rows * 384 * 4, &scratch));
        if (w8t)
            TZH_TRY(tzh_tile_codes_w8_launch(ctx->stream, wq, (uint8_t *)scratch, n, k));
        else
            TZH_TRY(tzh_widen_codes_launch(ctx->stream, wq, (_Float16 *)scratch, n * k));
        return tzh_linear_codes_launch(ctx->stream, ctx->num_cus, (const _Float16 *)a, scratch,
                                       w8t ? TZH_WF_W8T : TZH_WF_F16, scale, bias, c, c_dtype, m, k, n, epilogue,
                                       residual, gamma, beta, eps,
                                       ws_rows ? (float *)((char *)scratch + codes_bytes) : nullptr, ws_rows);
    }
    return tzh_linear_w8_launch(ctx->stream, a, a_dtype, wq, scale, bias, c, c_dtype, m, k, n, epilogue, residual,
                                res_dtype, gamma, beta, eps);
}

extern "C" int tzh_matmul_w8a32(tzh_ctx *ctx, const float *a, const int8_t *wq, const uint16_t *scale,
                                const float *bias, float *c, int64_t m, int64_t k, int64_t n) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    return tzh_linear_w8_launch(ctx->stream, a, TZH_F32, wq, scale, bias, c, TZH_F32, m, k, n, TZH_EPI_BIAS, nullptr,
                                TZH_F32, nullptr, nullptr, 0.0f);
}
