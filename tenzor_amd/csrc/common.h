// Shared host/device definitions for libtenzor_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/tenzor_hip.h"

// ---------------------------------------------------------------------------
// Error reporting: thread-local message, negative status codes.
// ---------------------------------------------------------------------------
int tzh_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void tzh_clear_error();

#define TZH_HIP(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return tzh_fail(TZH_ERR_DEVICE, "%s failed: %s (%s:%d)", #expr,              \
                            hipGetErrorString(e_), __FILE__, __LINE__);                  \
    } while (0)

#define TZH_TRY(expr)                                                                    \
    do {                                                                                 \
        int rc_ = (expr);                                                                \
        if (rc_ != TZH_OK) return rc_;                                                   \
    } while (0)

// After a kernel launch: report launch-configuration errors immediately.
#define TZH_LAUNCHED(name)                                                               \
    do {                                                                                 \
        hipError_t e_ = hipGetLastError();                                               \
        if (e_ != hipSuccess)                                                            \
            return tzh_fail(TZH_ERR_DEVICE, "launch of %s failed: %s", name,             \
                            hipGetErrorString(e_));                                      \
    } while (0)

// Device formats of a model's linear weights inside the library (not part of
// the C ABI): biased int8 codes stage-tiled in 384-row blocks (gemm_pipe.hip),
// or f32 weights [n, k] row-major (gemm_fp.hip).
enum { TZH_WF_W8T = 1, TZH_WF_F32 = 2 };

// ---------------------------------------------------------------------------
// Context: one device, one stream.
// ---------------------------------------------------------------------------
struct tzh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int num_cus = 256;
    // elementwise chains through the interpreter kernel instead of generated
    // kernels (environment TZH_EW_INTERPRETER=1 at tzh_init)
    bool ew_interpreter = false;
    // stream-ordered scratch used by eval for materialised reductions
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    int64_t scratch_allocs = 0;  // hipMalloc calls that (re)allocated the scratch
    // ring of kernel-program slots (device + pinned host staging)
    static constexpr int kProgSlots = 32;
    static constexpr size_t kProgSlotBytes = 4096;
    void *prog_dev = nullptr;
    void *prog_host = nullptr;
    hipEvent_t prog_ev[kProgSlots] = {};
    int prog_next = 0;
    // work-queue counters of persistent kernels (zero between launches)
    unsigned *work_queue = nullptr;
};

// Make ctx's device current for the calling thread.
int tzh_ctx_enter(tzh_ctx *ctx);
// Grow-only device scratch owned by the context (synchronises on growth).
int tzh_ctx_scratch(tzh_ctx *ctx, size_t bytes, void **out);
// The context's work-queue counters (allocated and zeroed on first use;
// the kernels that take items from them leave them at zero).
int tzh_ctx_work_queue(tzh_ctx *ctx, unsigned **out);
// Stream-ordered upload of a small kernel descriptor (<= kProgSlotBytes):
// copies `bytes` from src into the next device slot of the context's ring
// and returns its device address, valid for kernels enqueued next on the
// context's stream.
int tzh_ctx_upload_program(tzh_ctx *ctx, const void *src, size_t bytes, const void **dev_out);

// f32 / f64 GEMM on the matrix cores (gemm_fp.hip): Y[b] = ops(alpha *
// opA(A[b]) opB(B[b])) + beta * C, for b over the broadcast batch
// dimensions; A[b] = a + sum_d idx_d * a_bstride[d] (0 where broadcast),
// likewise B, and Y[b] = y + b * y_bstride.  lda / ldb / ldy are stored row
// pitches.  ops[] are applied in order: TZH_OP_ADD adds bias[col], any
// other code is that unary op (the elementwise engine's semantics).
struct tzh_gemm_desc {
    int64_t m = 0, n = 0, k = 0;
    int64_t lda = 0, ldb = 0, ldy = 0;
    int32_t nb = 0;
    int64_t batch_shape[TZH_MAX_RANK] = {};
    int64_t a_bstride[TZH_MAX_RANK] = {}, b_bstride[TZH_MAX_RANK] = {};
    int64_t y_bstride = 0;
    double alpha = 1.0, beta = 0.0;
    const void *c = nullptr;  // beta * c[i * c_rs + j * c_cs]
    int64_t c_rs = 0, c_cs = 0;
    const void *bias = nullptr;
    int32_t n_ops = 0;
    int32_t ops[4] = {};
};
// a_trans: A stored [k][m]; b_trans: B stored [n][k].
int tzh_gemm_fp_launch(hipStream_t st, int32_t dtype, bool a_trans, bool b_trans, const void *a, const void *b,
                       void *y, const tzh_gemm_desc &d);

// Host tokenizer (tokenizer.cpp) for the embedding entry points.
size_t tzh_tokenize(const tzh_tokenizer *tok, const uint8_t *text, size_t len, uint32_t *out, size_t cap);
void tzh_tokenize_raw(const tzh_tokenizer *tok, const uint8_t *text, size_t len, std::vector<uint32_t> &out);
uint32_t tzh_tokenizer_cls(const tzh_tokenizer *tok);
uint32_t tzh_tokenizer_sep(const tzh_tokenizer *tok);
// The context and hidden size a model was uploaded with (arctic.hip).
tzh_ctx *tzh_model_ctx(const tzh_model *m);
int tzh_model_hidden(const tzh_model *m);
// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

#define TZH_WAVE 64

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

#ifndef TZH_EMULATION
// v_permlane32_swap_b32: lanes 32..63 of `lo` trade values with lanes 0..31
// of `hi` (lanes 0..31 of `lo` and 32..63 of `hi` keep theirs).
__device__ __forceinline__ void lane_swap32(uint32_t &lo, uint32_t &hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
    lo = r[0];
    hi = r[1];
}

// True when `p` holds in any active lane of the wave.
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// v_permlane16_swap_b32: lanes 16..31 and 48..63 of `a` trade values with
// lanes 0..15 and 32..47 of `b` (lane i of one 16-lane row with lane i of
// the row below it).
__device__ __forceinline__ void lane_swap16(uint32_t &a, uint32_t &b) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
#endif

// The value of another lane of the wave by a DPP lane pattern (gfx9
// encodings): 0xB1 quad_perm [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1]
// (lane ^ 2), 0x141 row_half_mirror (lane 7 - i of each group of eight).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Maximum over the four lanes l % 16 + 16j (j = 0..3), left in all four:
// two row swaps instead of LDS-routed shuffles.
__device__ __forceinline__ float max_over_rows(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    lane_swap16(a, b);
    x = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = b = __builtin_bit_cast(uint32_t, x);
    lane_swap32(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// Sum over the four lanes l % 16 + 16j (j = 0..3), the same value left in
// all four: (x0 + x1) + (x2 + x3) up to the order of each addition's
// operands.
__device__ __forceinline__ float sum_over_rows(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    lane_swap16(a, b);
    x = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = b = __builtin_bit_cast(uint32_t, x);
    lane_swap32(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// f32 -> f16 pair x = hi + lo + r for 8 values: hi = f16(x), lo = f16(x - hi),
// both round-to-nearest-even (x - hi is exact in f32, so lo is x - hi
// rounded once).  |r| <= 2^-22 |x| for |x| >= 2^-3 (x - hi is then an f16
// normal) and <= 2^-25 below; valid for |x| < 65504.  On the GPU the low
// halves come from v_fma_mixlo/mixhi_f16 (fma(-hi, 1, x) formed exactly from
// the f16 hi and the f32 x, rounded once to f16), one instruction per value
// instead of a widen, a subtract and a narrow (the compiler's own selection
// takes 1.5 and, at the fused kernels' register counts, spills).  The
// compiler does not count inline asm as a VALU write, so it keeps no wait
// states between these writes and an MFMA reading the result, which the
// MFMA needs (two after a VALU write); each asm block therefore ends with
// "s_nop 1" (split_f32x8's also starts with one, below).
// tests/test_asm_hazards.py scans the generated code for both distances.
__device__ __forceinline__ uint32_t split_lo_pair(uint32_t hi2, float a, float b) {
#ifdef TZH_EMULATION
    const half2_t h = __builtin_bit_cast(half2_t, hi2);
    const half2_t l = {(_Float16)(a - (float)h[0]), (_Float16)(b - (float)h[1])};
    return __builtin_bit_cast(uint32_t, l);
#else
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, -%1, %4, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, -%1, %4, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "=&v"(d)
        : "v"(hi2), "v"(a), "v"(b), "v"(1.0f));
    return d;
#endif
}

__device__ __forceinline__ void split_f32x8(const f32x4_t &a, const f32x4_t &b, half8_t &hi, half8_t &lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        h[i] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)a[2 * i], (_Float16)a[2 * i + 1]});
        h[2 + i] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)b[2 * i], (_Float16)b[2 * i + 1]});
    }
#ifdef TZH_EMULATION
#pragma unroll
    for (int i = 0; i < 2; i++) {
        l[i] = split_lo_pair(h[i], a[2 * i], a[2 * i + 1]);
        l[2 + i] = split_lo_pair(h[2 + i], b[2 * i], b[2 * i + 1]);
    }
#else
    // the four pairs in one block, one trailing s_nop (see split_lo_pair).
    // The leading s_nop keeps the first write at least seven wait states
    // after an MFMA that read the output register as its accumulator input
    // (the register allocator reuses such a register for l[0] right away).
    asm("s_nop 2\n\t"
        "v_fma_mixlo_f16 %0, -%4, %16, %8 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, -%4, %16, %9 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %1, -%5, %16, %10 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %1, -%5, %16, %11 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %2, -%6, %16, %12 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %2, -%6, %16, %13 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %3, -%7, %16, %14 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %3, -%7, %16, %15 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "=&v"(l[0]), "=&v"(l[1]), "=&v"(l[2]), "=&v"(l[3])
        : "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(b[0]),
          "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(1.0f));
#endif
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    hi = __builtin_bit_cast(half8_t, u32x4v{h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(half8_t, u32x4v{l[0], l[1], l[2], l[3]});
}

// f32 -> f16 with round-to-nearest-even (v_cvt_f16_f32 honours the default RNE mode).
__device__ __forceinline__ _Float16 to_f16(float x) { return (_Float16)x; }

// f16 bits -> f32, exact.
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// Host-side f16 helpers (bit exact, RNE), used by the host quantizer and tests.
uint16_t tzh_host_f32_to_f16(float x);
float tzh_host_f16_to_f32(uint16_t h);

// tanh-form GELU of arctic.zig:750-756 with the device tanhf.
__device__ __forceinline__ float gelu_arctic(float x) {
    const float sqrt_2_over_pi = 0.7978845608f;
    const float coeff = 0.044715f;
    float inner = sqrt_2_over_pi * (x + coeff * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}
