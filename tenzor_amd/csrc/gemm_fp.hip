// K5: f32 / f64 GEMM on the matrix cores, for the general matmuls of the
// path: the `eval` matmul node (executor.zig:199-326, matmul.zig) with the
// fused bias + activation epilogue of FusedMatmulEpilogueKernel
// (fusion/codegen.zig:78-147), and the ONNX MatMul / Gemm operators
// (onnx/executor.zig:1489-1990, 4561-4634).
//
//   Y[b] = ops( alpha * opA(A[b]) opB(B[b]) ) + beta * C
//
// Products are exact and summed in the operand precision by
// v_mfma_f32_16x16x4_f32 / v_mfma_f64_16x16x4_f64 (157 / 79 TFLOP/s dense
// on MI355X), so the result is the reference's f32 (f64) matmul up to the
// order of the k sum.
//
// Design:
//   - 128 x 128 output tiles per 256-thread block, four waves of 64 x 64
//     (4 x 4 MFMA tiles of 16 x 16), k in stages of 16.  Operands are loaded
//     into registers with bounds checks (zero outside the matrix, 16-byte
//     vector loads where the rows allow), then written to a double-buffered
//     LDS tile as [row][k] (k contiguous): the stored A or B may be
//     k-contiguous (written as is) or row-contiguous (transposed on the way
//     in), so every transpose flag shares one MFMA loop.  The next stage's
//     loads are in flight while the current stage computes.
//   - A lane's MFMA operand for k step s of a stage is k = 4 (lane / 16) +
//     s, the same for both operands, so one 16-byte (f32) or 32-byte (f64)
//     LDS read gives a lane its four k steps.  Rows are padded to 20 f32 /
//     18 f64 elements: the sixteen rows a quarter-wave reads then start on
//     sixteen different bank groups.
//   - The MFMA takes B's columns as its A operand, so each lane holds four
//     output columns of one row (consecutive ones in f32: 16-byte stores of
//     Y rows).
#include "common.h"
#include "ew_program.h"  // unary_op<T>: the op semantics of the elementwise engine

#include <cstring>

namespace {

using tzh_ew::unary_op;

constexpr int kBM = 128, kBN = 128, kBK = 16, kThreads = 256;
constexpr int kMaxEpiOps = 4;

typedef double f64x4_t __attribute__((ext_vector_type(4)));

template <typename T>
struct Vec4 {
    using type = f32x4_t;
};
template <>
struct Vec4<double> {
    using type = f64x4_t;
};

// LDS row pitch in elements: 20 f32 (80 bytes) or 18 f64 (144 bytes), both
// 4 x an odd number of banks.
template <typename T>
constexpr int pitch() {
    return sizeof(T) == 4 ? 20 : 18;
}

template <typename T>
struct GemmArgs {
    int64_t m, n, k;
    int64_t lda, ldb, ldy;  // row pitches (elements) of the stored A, B and of Y
    int64_t tiles_m, tiles_n;
    int32_t nb;             // batch dimensions of the output
    int32_t vec_a, vec_b;   // 1: every 4-element run of a stored row starts 16-byte aligned
    int32_t vec_y;
    int64_t batch_shape[TZH_MAX_RANK];
    int64_t a_bstride[TZH_MAX_RANK], b_bstride[TZH_MAX_RANK];  // 0 where broadcast
    int64_t y_bstride;
    T alpha, beta;
    const T *c;             // beta * c[i * c_rs + j * c_cs], or null
    int64_t c_rs, c_cs;
    const T *bias;          // [n], added where ops[] holds TZH_OP_ADD
    int32_t n_ops;
    int32_t ops[kMaxEpiOps];
};

// Four consecutive elements of one stored row starting at p; element j is
// used only when j < valid (0..4).  `vec`: the run is 16-byte aligned.
template <typename T>
__device__ __forceinline__ void load4(const T *p, int valid, bool vec, T (&v)[4]) {
    if (vec && valid == 4) {
        if constexpr (sizeof(T) == 4) {
            const f32x4_t x = *(const f32x4_t *)p;
            v[0] = x[0], v[1] = x[1], v[2] = x[2], v[3] = x[3];
        } else {
            typedef double f64x2_t __attribute__((ext_vector_type(2)));
            const f64x2_t x = *(const f64x2_t *)p, y = *(const f64x2_t *)(p + 2);
            v[0] = x[0], v[1] = x[1], v[2] = y[0], v[3] = y[1];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = j < valid ? p[j] : (T)0;
    }
}

// One operand tile (128 rows of m or n, 16 k) per stage, two 4-element
// chunks per thread.  KC: the stored operand is k-contiguous (rows of k);
// else row-contiguous (rows of m or n, one per k).
template <typename T, bool KC>
struct TileLoader {
    T v[2][4];
    __device__ __forceinline__ void load(const T *X, int64_t ld, int64_t r0, int64_t R, int64_t k0, int64_t K,
                                         bool vec, int tid) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int q = tid + c * kThreads;
            if constexpr (KC) {
                const int64_t row = r0 + q / 4, kk = k0 + (q % 4) * 4;
                const int valid = row < R ? (int)(K - kk < 4 ? (K - kk > 0 ? K - kk : 0) : 4) : 0;
                load4<T>(X + (valid > 0 ? row * ld + kk : 0), valid, vec, v[c]);
            } else {
                const int64_t kk = k0 + q / 32, col = r0 + (q % 32) * 4;
                const int valid = kk < K ? (int)(R - col < 4 ? (R - col > 0 ? R - col : 0) : 4) : 0;
                load4<T>(X + (valid > 0 ? kk * ld + col : 0), valid, vec, v[c]);
            }
        }
    }
    __device__ __forceinline__ void store(T *tile, int tid) const {
        constexpr int P = pitch<T>();
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int q = tid + c * kThreads;
            if constexpr (KC) {
                T *d = tile + (q / 4) * P + (q % 4) * 4;
#pragma unroll
                for (int j = 0; j < 4; j++) d[j] = v[c][j];
            } else {
                const int kk = q / 32, col = (q % 32) * 4;
#pragma unroll
                for (int j = 0; j < 4; j++) tile[(col + j) * P + kk] = v[c][j];
            }
        }
    }
};

template <typename T>
__device__ __forceinline__ typename Vec4<T>::type mfma16(T a, T b, typename Vec4<T>::type c) {
    if constexpr (sizeof(T) == 4)
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// alpha * acc, plus beta * C when no ops come between them
template <typename T>
__device__ __forceinline__ T linear_value(const GemmArgs<T> &g, T acc, int64_t i, int64_t j) {
    T v = g.alpha * acc;
    if (g.c && g.n_ops == 0) v += g.beta * g.c[i * g.c_rs + j * g.c_cs];
    return v;
}

// TA: A is stored [k][m] (else [m][k]); TB: B is stored [n][k] (else [k][n]).
template <typename T, bool TA, bool TB>
__global__ void __launch_bounds__(kThreads) gemm_mfma_kernel(const T *__restrict__ A, const T *__restrict__ B,
                                                             T *__restrict__ Y, const GemmArgs<T> g) {
    constexpr int P = pitch<T>();
    using V4 = typename Vec4<T>::type;
    __shared__ __attribute__((aligned(16))) T as[2][kBM * P];
    __shared__ __attribute__((aligned(16))) T bs[2][kBN * P];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w & 1, wn = w >> 1;

    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t bi = (int64_t)blockIdx.x / tiles, t = (int64_t)blockIdx.x % tiles;
    const int64_t m0 = t / g.tiles_n * kBM, n0 = t % g.tiles_n * kBN;
    int64_t ao = 0, bo = 0, rem = bi;
    for (int d = g.nb - 1; d >= 0; d--) {
        const int64_t i = rem % g.batch_shape[d];
        rem /= g.batch_shape[d];
        ao += i * g.a_bstride[d];
        bo += i * g.b_bstride[d];
    }
    const T *Ab = A + ao, *Bb = B + bo;
    T *Yb = Y + bi * g.y_bstride;

    TileLoader<T, !TA> la;  // A rows are m
    TileLoader<T, TB> lb;   // B rows are n
    V4 acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = V4{};

    const int64_t S = (g.k + kBK - 1) / kBK;
    if (S > 0) {
        la.load(Ab, g.lda, m0, g.m, 0, g.k, g.vec_a, tid);
        lb.load(Bb, g.ldb, n0, g.n, 0, g.k, g.vec_b, tid);
        la.store(as[0], tid);
        lb.store(bs[0], tid);
    }
    __syncthreads();
    const int r16 = lane & 15, k4 = 4 * (lane >> 4);
    for (int64_t s = 0; s < S; s++) {
        const int buf = (int)(s & 1);
        if (s + 1 < S) {
            la.load(Ab, g.lda, m0, g.m, (s + 1) * kBK, g.k, g.vec_a, tid);
            lb.load(Bb, g.ldb, n0, g.n, (s + 1) * kBK, g.k, g.vec_b, tid);
        }
        V4 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const V4 *)&as[buf][(wm * 64 + i * 16 + r16) * P + k4];
#pragma unroll
        for (int j = 0; j < 4; j++) bf[j] = *(const V4 *)&bs[buf][(wn * 64 + j * 16 + r16) * P + k4];
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[j][i] = mfma16<T>(bf[j][q], af[i][q], acc[j][i]);
        if (s + 1 < S) {
            la.store(as[buf ^ 1], tid);
            lb.store(bs[buf ^ 1], tid);
        }
        __syncthreads();
    }

    // Lane l holds, for row m = m0 + wm*64 + 16 i + l%16, accumulator
    // element e of column n0 + wn*64 + 16 j + col(e): v_mfma_f32_16x16x4_f32
    // gives lane l rows 4 (l/16) + e of its D tile (four consecutive
    // columns here), v_mfma_f64_16x16x4_f64 rows l/16 + 4 e (measured on
    // MI355X).
    const int cq = lane >> 4;
    auto col = [&](int e) __attribute__((always_inline)) { return sizeof(T) == 4 ? 4 * cq + e : cq + 4 * e; };
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + wm * 64 + i * 16 + r16;
        if (m >= g.m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t nb = n0 + wn * 64 + j * 16;
            T *row = Yb + m * g.ldy + nb;
            if (sizeof(T) == 4 && g.vec_y && nb + col(3) < g.n) {
                *(f32x4_t *)(row + col(0)) = f32x4_t{(float)linear_value<T>(g, acc[j][i][0], m, nb + col(0)),
                                                     (float)linear_value<T>(g, acc[j][i][1], m, nb + col(1)),
                                                     (float)linear_value<T>(g, acc[j][i][2], m, nb + col(2)),
                                                     (float)linear_value<T>(g, acc[j][i][3], m, nb + col(3))};
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (nb + col(e) < g.n) row[col(e)] = linear_value<T>(g, acc[j][i][e], m, nb + col(e));
            }
        }
    }
    // The fused ops (bias adds and unary ops, in order) and then beta * C,
    // applied to the values this lane has just stored, read back from Y: in
    // a rolled loop the op code exists once, and the accumulators stay in
    // registers.
    if (g.n_ops == 0) return;
#pragma unroll 1
    for (int f = 0; f < 16; f++) {
        const int64_t m = m0 + wm * 64 + (f / 4) * 16 + r16, nb = n0 + wn * 64 + (f % 4) * 16;
        if (m >= g.m) continue;
#pragma unroll 1
        for (int e = 0; e < 4; e++) {
            const int64_t n = nb + col(e);
            if (n >= g.n) continue;
            T *p = Yb + m * g.ldy + n;
            T v = *p;
            for (int o = 0; o < g.n_ops; o++) v = g.ops[o] == TZH_OP_ADD ? v + g.bias[n] : unary_op<T>(g.ops[o], v);
            if (g.c) v += g.beta * g.c[m * g.c_rs + n * g.c_cs];
            *p = v;
        }
    }
}

// y[i] = a[i] * s (the scalar-operand MatMul of onnx/executor.zig:1545-1577);
// a == null: y[i] = 0 (the empty sums of k == 0)
template <typename T>
__global__ void scale_kernel(const T *__restrict__ a, T s, T *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a ? a[i] * s : (T)0;
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// The launch behind every entry point below and the eval planner's matmul
// node: a_trans / b_trans say how A and B are stored (see gemm_mfma_kernel).
// d describes the batch and the epilogue; pointers are device pointers.
int tzh_gemm_fp_launch(hipStream_t st, int32_t dtype, bool a_trans, bool b_trans, const void *a, const void *b,
                       void *y, const tzh_gemm_desc &d) {
    if (dtype != TZH_F32 && dtype != TZH_F64) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "GEMM dtype must be F32 or F64");
    if (d.m < 0 || d.n < 0 || d.k < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative GEMM dimension");
    if (d.nb < 0 || d.nb > TZH_MAX_RANK) return tzh_fail(TZH_ERR_INVALID_ARGS, "batch rank %d out of range", d.nb);
    if (d.n_ops < 0 || d.n_ops > kMaxEpiOps) return tzh_fail(TZH_ERR_INVALID_ARGS, "%d epilogue ops (at most %d)", d.n_ops, kMaxEpiOps);
    int64_t batches = 1;
    for (int i = 0; i < d.nb; i++) {
        if (d.batch_shape[i] < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative batch dimension");
        batches *= d.batch_shape[i];
    }
    if (d.m == 0 || d.n == 0 || batches == 0) return TZH_OK;
    for (int o = 0; o < d.n_ops; o++) {
        const int op = d.ops[o];
        if (op == TZH_OP_ADD && !d.bias) return tzh_fail(TZH_ERR_INVALID_ARGS, "bias add without a bias");
        if (op != TZH_OP_ADD && !tzh_ew::unary_ok(op))
            return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "epilogue op %d is not a unary op or a bias add", op);
    }
    const int64_t tm = (d.m + kBM - 1) / kBM, tn = (d.n + kBN - 1) / kBN;
    if (batches > ((int64_t)1 << 31) / (tm * tn)) return tzh_fail(TZH_ERR_TOO_LARGE, "GEMM grid too large");
    const int64_t vec_e = dtype == TZH_F32 ? 4 : 2;  // elements per 16 bytes
    auto vec_ok = [&](const void *p, int64_t ld, const int64_t *bstride) {
        if (!al16(p) || ld % vec_e) return 0;
        for (int i = 0; i < d.nb; i++)
            if (bstride[i] % vec_e) return 0;
        return 1;
    };
    if (!y || (d.k > 0 && (!a || !b))) return tzh_fail(TZH_ERR_INVALID_ARGS, "null GEMM operand");  // k == 0 reads neither
    auto fill = [&](auto tag) -> int {
        using T = decltype(tag);
        GemmArgs<T> g{};
        g.m = d.m, g.n = d.n, g.k = d.k, g.lda = d.lda, g.ldb = d.ldb, g.ldy = d.ldy;
        g.tiles_m = tm, g.tiles_n = tn, g.nb = d.nb;
        g.vec_a = vec_ok(a, d.lda, d.a_bstride);
        g.vec_b = vec_ok(b, d.ldb, d.b_bstride);
        g.vec_y = al16(y) && d.ldy % vec_e == 0 && (d.nb == 0 || d.y_bstride % vec_e == 0);
        for (int i = 0; i < d.nb; i++) {
            g.batch_shape[i] = d.batch_shape[i];
            g.a_bstride[i] = d.a_bstride[i];
            g.b_bstride[i] = d.b_bstride[i];
        }
        g.y_bstride = d.y_bstride;
        g.alpha = (T)d.alpha, g.beta = (T)d.beta;
        g.c = (const T *)d.c, g.c_rs = d.c_rs, g.c_cs = d.c_cs;
        g.bias = (const T *)d.bias;
        g.n_ops = d.n_ops;
        for (int o = 0; o < d.n_ops; o++) g.ops[o] = d.ops[o];
        const dim3 grid((unsigned)(batches * tm * tn));
        const T *A = (const T *)a, *B = (const T *)b;
        T *Y = (T *)y;
        if (a_trans && b_trans)
            hipLaunchKernelGGL((gemm_mfma_kernel<T, true, true>), grid, dim3(kThreads), 0, st, A, B, Y, g);
        else if (a_trans)
            hipLaunchKernelGGL((gemm_mfma_kernel<T, true, false>), grid, dim3(kThreads), 0, st, A, B, Y, g);
        else if (b_trans)
            hipLaunchKernelGGL((gemm_mfma_kernel<T, false, true>), grid, dim3(kThreads), 0, st, A, B, Y, g);
        else
            hipLaunchKernelGGL((gemm_mfma_kernel<T, false, false>), grid, dim3(kThreads), 0, st, A, B, Y, g);
        TZH_LAUNCHED("gemm_mfma_kernel");
        return TZH_OK;
    };
    return dtype == TZH_F32 ? fill(0.0f) : fill(0.0);
}

// ONNX Gemm (onnx/executor.zig:4561-4634): Y[m,n] = alpha * op(A) op(B) +
// beta * C, C broadcast from [c_rows, c_cols] (rows 1 or m, columns 1 or n;
// NULL: no C); lda / ldb are the stored row pitches (the reference's
// a.shape[1] / b.shape[1]); Y is contiguous [m, n].
extern "C" int tzh_gemm_f32(tzh_ctx *ctx, int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k,
                            float alpha, const float *a, int64_t lda, const float *b, int64_t ldb, float beta,
                            const float *c, int64_t c_rows, int64_t c_cols, float *y) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (m < 0 || n < 0 || k < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative Gemm dimension");
    if (m == 0 || n == 0) return TZH_OK;
    if (k > 0 && (lda < (trans_a ? m : k) || ldb < (trans_b ? k : n)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "row pitch smaller than the stored row");
    if (c && !((c_rows == 1 || c_rows == m) && (c_cols == 1 || c_cols == n)))
        return tzh_fail(TZH_ERR_SHAPE, "C of shape [%lld, %lld] does not broadcast to [%lld, %lld]",
                        (long long)c_rows, (long long)c_cols, (long long)m, (long long)n);
    tzh_gemm_desc d{};
    d.m = m, d.n = n, d.k = k, d.lda = lda, d.ldb = ldb, d.ldy = n;
    d.alpha = alpha, d.beta = beta;
    d.c = c, d.c_rs = c && c_rows > 1 ? c_cols : 0, d.c_cs = c && c_cols > 1 ? 1 : 0;
    return tzh_gemm_fp_launch(ctx->stream, TZH_F32, trans_a != 0, trans_b != 0, a, b, y, d);
}

// ONNX MatMul (onnx/executor.zig:1489-1990): NumPy matmul of A (a_ndim >= 1)
// and B, batch dimensions broadcast, a 1-D A a row and a 1-D B a column
// whose unit dimension the result drops; B of shape [] or [1] scales A
// elementwise (executor.zig:1545-1577); any zero dimension gives an empty
// (or, with k == 0, zero) result.  Writes the result shape to y_shape /
// *y_ndim (host, room for 8), and the result to y unless y is NULL.
extern "C" int tzh_matmul_nd(tzh_ctx *ctx, int32_t dtype, const void *a, const int64_t *a_shape, int32_t a_ndim,
                             const void *b, const int64_t *b_shape, int32_t b_ndim, void *y, int64_t *y_shape,
                             int32_t *y_ndim) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (dtype != TZH_F32 && dtype != TZH_F64) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "MatMul dtype must be F32 or F64");
    if (!y_shape || !y_ndim || a_ndim < 0 || b_ndim < 0 || a_ndim > TZH_MAX_RANK || b_ndim > TZH_MAX_RANK ||
        (a_ndim && !a_shape) || (b_ndim && !b_shape))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "bad MatMul shape arguments");
    int64_t an = 1;
    for (int i = 0; i < a_ndim; i++) {
        if (a_shape[i] < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative dimension");
        an *= a_shape[i];
    }
    for (int i = 0; i < b_ndim; i++)
        if (b_shape[i] < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative dimension");
    const size_t es = dtype == TZH_F32 ? 4 : 8;  // element bytes
    // scalar B: elementwise scale of A (its result keeps A's shape)
    if (b_ndim == 0 || (b_ndim == 1 && b_shape[0] == 1)) {
        *y_ndim = a_ndim;
        for (int i = 0; i < a_ndim; i++) y_shape[i] = a_shape[i];
        if (!y || an == 0) return TZH_OK;
        if (!a || !b) return tzh_fail(TZH_ERR_INVALID_ARGS, "null MatMul operand");
        double s = 0;
        TZH_HIP(hipMemcpyAsync(&s, b, es, hipMemcpyDeviceToHost, ctx->stream));
        TZH_HIP(hipStreamSynchronize(ctx->stream));
        const dim3 grid((unsigned)((an + 255) / 256));
        if (dtype == TZH_F32) {
            float sf;
            std::memcpy(&sf, &s, 4);
            hipLaunchKernelGGL(scale_kernel<float>, grid, dim3(256), 0, ctx->stream, (const float *)a, sf, (float *)y, an);
        } else {
            hipLaunchKernelGGL(scale_kernel<double>, grid, dim3(256), 0, ctx->stream, (const double *)a, s, (double *)y, an);
        }
        TZH_LAUNCHED("scale_kernel");
        return TZH_OK;
    }
    if (a_ndim < 1) return tzh_fail(TZH_ERR_SHAPE, "MatMul of a scalar A");
    const int64_t m = a_ndim == 1 ? 1 : a_shape[a_ndim - 2], k = a_shape[a_ndim - 1];
    const int64_t k2 = b_ndim == 1 ? b_shape[0] : b_shape[b_ndim - 2], nn = b_ndim == 1 ? 1 : b_shape[b_ndim - 1];
    if (k != k2) return tzh_fail(TZH_ERR_SHAPE, "MatMul inner dimensions differ (%lld vs %lld)", (long long)k, (long long)k2);
    tzh_gemm_desc d{};
    const int lb = a_ndim > 2 ? a_ndim - 2 : 0, rb = b_ndim > 2 ? b_ndim - 2 : 0;
    d.nb = lb > rb ? lb : rb;
    int64_t as = m * k, bs = k * nn;
    for (int i = d.nb - 1; i >= 0; i--) {
        const int li = i - (d.nb - lb), ri = i - (d.nb - rb);
        const int64_t ld = li >= 0 ? a_shape[li] : 1, rd = ri >= 0 ? b_shape[ri] : 1;
        if (ld != rd && ld != 1 && rd != 1) return tzh_fail(TZH_ERR_SHAPE, "MatMul batch dimensions do not broadcast");
        d.batch_shape[i] = ld > rd ? ld : rd;
        d.a_bstride[i] = ld == 1 ? 0 : as;
        d.b_bstride[i] = rd == 1 ? 0 : bs;
        if (li >= 0) as *= ld;
        if (ri >= 0) bs *= rd;
    }
    int w = 0;
    int64_t batches = 1;
    for (int i = 0; i < d.nb; i++) {
        y_shape[w++] = d.batch_shape[i];
        batches *= d.batch_shape[i];
    }
    if (a_ndim > 1) y_shape[w++] = m;
    if (b_ndim > 1) y_shape[w++] = nn;
    *y_ndim = w;
    if (!y) return TZH_OK;
    const int64_t yn = batches * m * nn;
    if (yn == 0) return TZH_OK;
    if (k == 0) {  // empty sums (A and B hold no elements)
        const dim3 grid((unsigned)((yn + 255) / 256));
        if (dtype == TZH_F32)
            hipLaunchKernelGGL(scale_kernel<float>, grid, dim3(256), 0, ctx->stream, (const float *)nullptr, 0.0f,
                               (float *)y, yn);
        else
            hipLaunchKernelGGL(scale_kernel<double>, grid, dim3(256), 0, ctx->stream, (const double *)nullptr, 0.0,
                               (double *)y, yn);
        TZH_LAUNCHED("scale_kernel");
        return TZH_OK;
    }
    if (!a || !b) return tzh_fail(TZH_ERR_INVALID_ARGS, "null MatMul operand");
    d.m = m, d.n = nn, d.k = k, d.lda = k, d.ldb = nn, d.ldy = nn, d.y_bstride = m * nn;
    d.alpha = 1.0, d.beta = 0.0;
    return tzh_gemm_fp_launch(ctx->stream, dtype, false, false, a, b, y, d);
}
