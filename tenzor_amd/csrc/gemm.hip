// K3 entry points for caller-owned int8 weights: matmulTransposeB_f32_i8_
// rowScale_bias (matmul_w8a32.zig:14-57) and the fused linear + epilogue
// calls Arctic makes after it (GELU, arctic.zig:771-776; residual +
// LayerNorm, arctic.zig:716-746, 779-809).
//
// Every shape runs on the pipelined MFMA kernel of gemm_pipe.hip.  Per call
// the int8 codes [n, k] are rewritten into its stage-tiled format, padded to
// n_pad (a multiple of 384) rows and k_pad (a multiple of 64) columns with
// code 0; when k is not a multiple of 64 the activation rows are copied with
// zero columns up to k_pad (the tail of matmul_w8a32.zig:50-52).  Padding
// adds only exact zeros to every sum, and padded output columns are never
// stored.  The rewritten codes (and the padded rows) live in the context
// scratch.
//
// f32 activations enter the MFMA as f16 halves hi + lo.  So that this is the
// reference's f32 arithmetic for rows of any scale (f16 alone spans 2^-24 ..
// 65504), the GEMM runs row-scaled: it splits X[t,:] * 2^e with e an exact
// power-of-two exponent per row that it chooses stage by stage from the
// row's largest magnitude (lowered, with the sums rescaled exactly, when a
// later stage holds larger values), and multiplies the sums by 2^-e before
// the scale and bias (linear_pipe_kernel in gemm_pipe.hip).  So the products
// carry the split's 2^-22 relative residual for every value within 2^17 of
// its row's largest.
#include "common.h"

#include <algorithm>
#include <mutex>

int tzh_tile_codes_w8_launch(hipStream_t st, const int8_t *q, uint8_t *out, int64_t n, int64_t k, int64_t n_pad,
                             int64_t k_pad);
int tzh_linear_codes_launch(hipStream_t st, int num_cus, const void *x, int32_t x_dtype, const void *wc,
                            int32_t w_format, const uint16_t *scale, const float *bias, void *c, int32_t c_dtype,
                            int64_t m, int64_t k, int64_t n, int64_t n_valid, int32_t epilogue, const void *res,
                            const float *gamma, const float *beta, float eps, float *ln_ws, int64_t ln_ws_rows,
                            bool row_scale);

namespace {

// c[i, j] = bias[j] (0 without a bias): the k == 0 product, an empty sum
// times the scale plus the bias (matmul_w8a32.zig:40-55)
__global__ void fill_bias_kernel(float *__restrict__ c, int64_t m, int64_t n, const float *__restrict__ bias) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * n) return;
    c[i] = bias ? bias[i % n] : 0.0f;
}

// rows [m, k] -> [m, k_pad] with zero columns k .. k_pad-1
template <typename T>
__global__ void pad_cols_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t m, int k, int k_pad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * k_pad) return;
    const int64_t r = i / k_pad;
    const int j = (int)(i % k_pad);
    y[i] = j < k ? x[r * k + j] : (T)0;
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }
size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Workspace of tzh_matmul_w8a32_noalloc: a file-scope device array, one per
// GPU, held until the process ends.  Host code never passes `scratch`
// itself (its host-side name is no device address): each device's address
// is looked up once with hipGetSymbolAddress and kept in scratch_ptr.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

int noalloc_scratch(tzh_ctx *ctx, void **out) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "device %d out of range", ctx->device);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[ctx->device]) {  // the device is current (tzh_ctx_enter)
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return tzh_fail(TZH_ERR_DEVICE, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        }
        g_scratch_ptr[ctx->device] = p;
    }
    *out = g_scratch_ptr[ctx->device];
    return TZH_OK;
}

// The workspace a linear needs: tiled codes, then (k % 64 != 0 or a
// misaligned a) the zero-padded activation rows, then (LayerNorm epilogue)
// the rows of a split partial round.
struct Workspace {
    size_t codes = 0, a = 0, ws = 0;
    int64_t ws_rows = 0;
    size_t total() const { return codes + a + ws; }
};

Workspace workspace_of(const tzh_ctx *ctx, const void *a, int32_t a_dtype, int64_t m, int64_t k, int64_t n, bool ln) {
    const int64_t n_pad = (n + 383) / 384 * 384, k_pad = (k + 63) / 64 * 64;
    Workspace w;
    w.codes = round256((size_t)n_pad * (size_t)k_pad);
    if (k != k_pad || !al16(a)) w.a = round256((size_t)m * (size_t)k_pad * (a_dtype == TZH_F32 ? 4 : 2));
    w.ws_rows = ln ? std::min<int64_t>((m + 127) / 128, ctx->num_cus / 3 + 1) * 128 : 0;
    w.ws = (size_t)w.ws_rows * 384 * 4;
    return w;
}

// `scratch_ptr` (device memory of at least workspace_of(...).total() bytes)
// or null: the context scratch, grown on demand.
int linear(tzh_ctx *ctx, const void *a, int32_t a_dtype, const int8_t *wq, const uint16_t *scale, const float *bias,
           void *c, int32_t c_dtype, int64_t m, int64_t k, int64_t n, int32_t epilogue, const void *residual,
           int32_t res_dtype, const float *gamma, const float *beta, float eps, void *scratch_ptr = nullptr) {
    if (m < 0 || k < 0 || n < 0)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "bad GEMM shape m=%lld k=%lld n=%lld", (long long)m, (long long)k,
                        (long long)n);
    if (m == 0 || n == 0) return TZH_OK;  // matmul_w8a32.zig:24
    if (m > (int64_t)1 << 30 || k > 65536 || n > 65536) return tzh_fail(TZH_ERR_TOO_LARGE, "GEMM shape too large");
    if ((a_dtype != TZH_F32 && a_dtype != TZH_F16) || (c_dtype != TZH_F32 && c_dtype != TZH_F16))
        return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "activations and output must be F32 or F16");
    if (!c || (k > 0 && (!a || !wq || !scale))) return tzh_fail(TZH_ERR_INVALID_ARGS, "null operand");
    const bool ln = epilogue == TZH_EPI_BIAS_RES_LN;
    if (epilogue != TZH_EPI_BIAS && epilogue != TZH_EPI_BIAS_GELU && !ln)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "unknown epilogue %d", epilogue);
    if (ln) {
        if (n != 384) return tzh_fail(TZH_ERR_INVALID_ARGS, "LayerNorm epilogue needs n == 384 (got %lld)", (long long)n);
        if (!residual || !gamma || !beta) return tzh_fail(TZH_ERR_INVALID_ARGS, "null residual/gamma/beta");
        if (res_dtype != c_dtype) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "residual dtype must equal output dtype");
        if (!al16(residual)) return tzh_fail(TZH_ERR_INVALID_ARGS, "residual must be 16-byte aligned");
    }
    if (k == 0) {
        // an empty sum: c = 0 * s + bias (matmul_w8a32.zig:40-55), the plain
        // bias epilogue of the reference's signature only
        if (epilogue != TZH_EPI_BIAS || c_dtype != TZH_F32)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "k == 0 is supported for the f32 bias epilogue only");
        if ((uintptr_t)c & 3) return tzh_fail(TZH_ERR_INVALID_ARGS, "c is not aligned to its element");
        const int64_t cnt = m * n;
        hipLaunchKernelGGL(fill_bias_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, ctx->stream,
                           (float *)c, m, n, bias);
        TZH_LAUNCHED("fill_bias_kernel");
        return TZH_OK;
    }
    const int64_t n_pad = (n + 383) / 384 * 384, k_pad = (k + 63) / 64 * 64;
    // f16 output is stored through whole-row tiles: every column must exist
    // and rows must keep 16-byte alignment
    if (c_dtype == TZH_F16 && (n != n_pad || !al16(c)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "f16 output needs n %% 384 == 0 and a 16-byte aligned c");
    if (((uintptr_t)c & 3) || (ln && !al16(c)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "c is not aligned to its element (16 bytes with the LayerNorm epilogue)");
    const Workspace wsz = workspace_of(ctx, a, a_dtype, m, k, n, ln);
    const bool pad_a = wsz.a > 0;
    const size_t codes_bytes = wsz.codes, a_bytes = wsz.a;
    const int64_t ws_rows = wsz.ws_rows;
    void *scratch = scratch_ptr;
    if (!scratch) TZH_TRY(tzh_ctx_scratch(ctx, wsz.total(), &scratch));
    uint8_t *codes = (uint8_t *)scratch;
    TZH_TRY(tzh_tile_codes_w8_launch(ctx->stream, wq, codes, n, k, n_pad, k_pad));
    const void *x = a;
    if (pad_a) {
        void *xp = (char *)scratch + codes_bytes;
        const int64_t cnt = m * k_pad;
        const dim3 grid((unsigned)((cnt + 255) / 256));
        if (a_dtype == TZH_F32)
            hipLaunchKernelGGL(pad_cols_kernel<float>, grid, dim3(256), 0, ctx->stream, (const float *)a, (float *)xp,
                               m, (int)k, (int)k_pad);
        else
            hipLaunchKernelGGL(pad_cols_kernel<_Float16>, grid, dim3(256), 0, ctx->stream, (const _Float16 *)a,
                               (_Float16 *)xp, m, (int)k, (int)k_pad);
        TZH_LAUNCHED("pad_cols_kernel");
        x = xp;
    }
    float *ws = ws_rows ? (float *)((char *)scratch + codes_bytes + a_bytes) : nullptr;
    return tzh_linear_codes_launch(ctx->stream, ctx->num_cus, x, a_dtype, codes, TZH_WF_W8T, scale, bias, c, c_dtype,
                                   m, k_pad, n_pad, n, epilogue, residual, gamma, beta, eps, ws, ws_rows,
                                   a_dtype == TZH_F32);
}

}  // namespace

extern "C" int tzh_linear_w8(tzh_ctx *ctx, const void *a, int32_t a_dtype, const int8_t *wq, const uint16_t *scale,
                             const float *bias, void *c, int32_t c_dtype, int64_t m, int64_t k, int64_t n,
                             int32_t epilogue, const void *residual, int32_t res_dtype, const float *gamma,
                             const float *beta, float eps) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    return linear(ctx, a, a_dtype, wq, scale, bias, c, c_dtype, m, k, n, epilogue, residual, res_dtype, gamma, beta,
                  eps);
}

extern "C" int tzh_matmul_w8a32(tzh_ctx *ctx, const float *a, const int8_t *wq, const uint16_t *scale,
                                const float *bias, float *c, int64_t m, int64_t k, int64_t n) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    return linear(ctx, a, TZH_F32, wq, scale, bias, c, TZH_F32, m, k, n, TZH_EPI_BIAS, nullptr, TZH_F32, nullptr,
                  nullptr, 0.0f);
}

extern "C" int tzh_matmul_w8a32_noalloc(tzh_ctx *ctx, const float *a, const int8_t *wq, const uint16_t *scale,
                                        const float *bias, float *c, int64_t m, int64_t k, int64_t n) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    // the shape errors, empty products and k == 0 of tzh_matmul_w8a32 (none
    // of which uses the workspace)
    if (m <= 0 || k <= 0 || n <= 0 || m > (int64_t)1 << 30 || k > 65536 || n > 65536)
        return linear(ctx, a, TZH_F32, wq, scale, bias, c, TZH_F32, m, k, n, TZH_EPI_BIAS, nullptr, TZH_F32, nullptr,
                      nullptr, 0.0f);
    const size_t need = workspace_of(ctx, a, TZH_F32, m, k, n, false).total();
    if (need > kNoAllocScratchBytes)
        return tzh_fail(TZH_ERR_TOO_LARGE,
                        "tzh_matmul_w8a32_noalloc needs %zu bytes of workspace for m=%lld k=%lld n=%lld; its static "
                        "workspace holds %zu (the tiled codes, n_pad * k_pad bytes, plus m * k_pad * 4 when k %% 64 "
                        "!= 0 or a is not 16-byte aligned)",
                        need, (long long)m, (long long)k, (long long)n, kNoAllocScratchBytes);
    void *ws = nullptr;
    TZH_TRY(noalloc_scratch(ctx, &ws));
    return linear(ctx, a, TZH_F32, wq, scale, bias, c, TZH_F32, m, k, n, TZH_EPI_BIAS, nullptr, TZH_F32, nullptr,
                  nullptr, 0.0f, ws);
}
