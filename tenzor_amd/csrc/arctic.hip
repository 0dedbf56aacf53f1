// Arctic-embed-xs encoder forward on gfx950 (replaces arctic.zig:113-1013).
//
// Activations live in HBM as f32 between kernels, as in the reference
// (arctic.zig:599-635 keeps every activation f32); the GEMMs and attention
// form f32 products on the MFMA from exact f16 hi/lo splits, and every
// reduction, accumulation and normalisation is f32.  An opt-in f16
// activation mode (tzh_arctic_set_precision) halves the activation traffic
// at f16 rounding.  Sequences of a batch are packed
// back to back (cu_seqlens) so padded positions cost nothing and each
// sequence is forwarded at its true length, as the reference's per-sequence
// forward does (arctic.zig:874-898, 959-1013).
//
// Per layer (arctic.zig:814-826):
//   qkv  = h  @ Wqkv^T * s + b                    (one GEMM, N = 3*384)
//   ctx  = attention(qkv)                         (K4)
//   h1   = LN(h  + (ctx @ Wo^T * s + bo))          (GEMM + LN epilogue)
//   f    = gelu(h1 @ W1^T * s + b1)               (GEMM + GELU epilogue)
//   h    = LN(h1 + (f  @ W2^T * s + b2))           (GEMM + LN epilogue)
#include "common.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <numeric>
#include <string>
#include <vector>

#include "safetensors.h"
#include "tenzor_file.h"

int tzh_linear_codes_launch(hipStream_t st, int num_cus, const void *x, int32_t x_dtype, const void *wc,
                            int32_t w_format, const uint16_t *scale, const float *bias, void *c, int32_t c_dtype,
                            int64_t m, int64_t k, int64_t n, int64_t n_valid, int32_t epilogue, const void *res,
                            const float *gamma, const float *beta, float eps, float *ln_ws, int64_t ln_ws_rows,
                            bool row_scale);
int tzh_attention_launch(hipStream_t st, int num_cus, unsigned *queue, const void *qkv, void *out, int32_t dtype,
                         const int *cu_seqlens, const int *order, int batch, int n_heads, int hidden);
size_t tzh_mlp_pack_bytes();
int tzh_mlp_pack_launch(hipStream_t st, const void *w1, const void *w2, void *out);
int tzh_mlp_fused_launch(hipStream_t st, int num_cus, const float *x, const void *pack, const uint16_t *s1,
                         const float *b1, const uint16_t *s2, const float *b2, const float *gamma, const float *beta,
                         float eps, float *y, int64_t t, const float *ctx, const float *res, const void *opack,
                         const uint16_t *so, const float *bo, const float *gamma1, const float *beta1, void *scratch,
                         size_t scratch_bytes);
size_t tzh_mlp_tail_bytes(int num_cus);
size_t tzh_qkv_pack_bytes();
int tzh_qkv_pack_launch(hipStream_t st, const void *w, void *out);
int tzh_qkv_fused_launch(hipStream_t st, int num_cus, const float *x, const void *pack, const uint16_t *s,
                         const float *b, float *y, int64_t t);
size_t tzh_mlp_opack_bytes();
int tzh_mlp_opack_launch(hipStream_t st, const void *wo, void *out);

namespace {

constexpr int H = 384;  // hidden size the kernels are specialised for

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

// Pack ids of a (possibly padded) batch into [T] and record positions.
__global__ void pack_ids_kernel(const uint32_t *__restrict__ ids, int64_t stride, const int *__restrict__ cu,
                                uint32_t *__restrict__ tok_ids, int32_t *__restrict__ tok_pos, uint32_t vocab,
                                int *__restrict__ bad) {
    const int b = blockIdx.x;
    const int start = cu[b], L = cu[b + 1] - start;
    const uint32_t *src = stride ? ids + (int64_t)b * stride : ids + start;
    for (int j = threadIdx.x; j < L; j += blockDim.x) {
        uint32_t id = src[j];
        if (id >= vocab) {  // out-of-range id: counted, clamped to keep the gather in bounds
            atomicAdd(bad, 1);
            id = vocab - 1;
        }
        tok_ids[start + j] = id;
        tok_pos[start + j] = j;
    }
}

struct TableRef {
    const float *f32;
    const int8_t *q8;
    const uint16_t *scale;
    __device__ __forceinline__ float get(int64_t row, int col) const {
        if (f32) return f32[row * H + col];
        return (float)q8[row * H + col] * f16_bits_to_f32(scale[row]);  // arctic.zig:490-508
    }
};

// K2: x = (word[id] + pos[p]) + type[0], then LayerNorm (arctic.zig:543-585).
// One wave per token, six columns per lane.
template <typename TO>
__global__ void __launch_bounds__(256) embed_ln_kernel(const uint32_t *__restrict__ tok_ids,
                                                       const int32_t *__restrict__ tok_pos, int64_t T,
                                                       TableRef word, TableRef pos, TableRef type,
                                                       const float *__restrict__ gamma,
                                                       const float *__restrict__ beta, float eps,
                                                       TO *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const int64_t id = tok_ids[t];
    const int64_t p = tok_pos[t];
    float x[6];
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 6; q++) {
        const int c = lane + 64 * q;
        float v = word.get(id, c);
        v = v + pos.get(p, c);
        v = v + type.get(0, c);
        x[q] = v;
        sum += v;
    }
    const float mean = wave_sum(sum) / (float)H;
    float vs = 0.0f;
#pragma unroll
    for (int q = 0; q < 6; q++) {
        const float d = x[q] - mean;
        vs += d * d;
    }
    const float inv_std = 1.0f / sqrtf(wave_sum(vs) / (float)H + eps);
#pragma unroll
    for (int q = 0; q < 6; q++) {
        const int c = lane + 64 * q;
        out[t * H + c] = (TO)(((x[q] - mean) * inv_std) * gamma[c] + beta[c]);
    }
}

// K5: CLS row of every sequence, L2-normalised (arctic.zig:893-897, 851-863).
template <typename TI>
__global__ void __launch_bounds__(256) cls_l2_kernel(const TI *__restrict__ hidden, const int *__restrict__ cu,
                                                     int batch, float *__restrict__ out) {
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (b >= batch) return;
    const TI *row = hidden + (int64_t)cu[b] * H;
    float v[6], ss = 0.0f;
#pragma unroll
    for (int q = 0; q < 6; q++) {
        v[q] = (float)row[lane + 64 * q];
        ss += v[q] * v[q];
    }
    const float norm = sqrtf(wave_sum(ss));
#pragma unroll
    for (int q = 0; q < 6; q++) out[(int64_t)b * H + lane + 64 * q] = norm > 1e-12f ? v[q] / norm : v[q];
}

// Row-wise LayerNorm over the last dim, f32 in/out (layernorm.zig:26-117),
// one wave per row.
__global__ void __launch_bounds__(256) layernorm_rows_kernel(const float *x, const float *__restrict__ g,
                                                             const float *__restrict__ bta, float *y,
                                                             int64_t rows, int n, float eps) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + r * n;
    float s = 0.0f;
    for (int c = lane; c < n; c += 64) s += xr[c];
    const float mean = wave_sum(s) / (float)n;
    float vs = 0.0f;
    for (int c = lane; c < n; c += 64) {
        const float d = xr[c] - mean;
        vs += d * d;
    }
    const float inv_std = 1.0f / sqrtf(wave_sum(vs) / (float)n + eps);
    // all lanes have read their inputs before any write (wave_sum is a
    // wave-wide exchange), so x == y is safe
    for (int c = lane; c < n; c += 64) y[r * n + c] = ((xr[c] - mean) * inv_std) * g[c] + bta[c];
}

// GPU quantizer, bit-exact to quantize_arctic_xs.zig:94-115: one wave per
// row; the max is order-independent and each code depends on its element only.
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                                                            int8_t *__restrict__ q, uint16_t *__restrict__ scale) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *row = w + r * cols;
    float mx = 0.0f;
    for (int64_t c = lane; c < cols; c += 64) {
        const float a = fabsf(row[c]);
        mx = a > mx ? a : mx;
    }
    mx = wave_max(mx);
    const float s32 = mx == 0.0f ? 1.0f : mx / 127.0f;
    const _Float16 s16 = (_Float16)s32;  // v_cvt_f16_f32, round to nearest even
    if (lane == 0) scale[r] = __builtin_bit_cast(uint16_t, s16);
    const float inv = 1.0f / (float)s16;
    for (int64_t c = lane; c < cols; c += 64) {
        const float qf = roundf(row[c] * inv);
        // same saturation as the host quantizer for a zero f16 scale
        const int qi = isnan(qf) ? 0 : qf >= 127.0f ? 127 : qf <= -127.0f ? -127 : (int)qf;
        q[r * cols + c] = (int8_t)qi;
    }
}

// ---------------------------------------------------------------------------
// model state
// ---------------------------------------------------------------------------
struct DevTable {
    float *f32 = nullptr;
    int8_t *q8 = nullptr;
    uint16_t *scale = nullptr;
    TableRef ref() const { return TableRef{f32, q8, scale}; }
};

// One linear of a layer, in one of two device formats, chosen per linear
// as the reference's MatWeight is (arctic.zig:55-58):
//   TZH_WF_W8T: int8 codes with a per-row f16 scale, C = (X . q) * s + b;
//     the codes stay one byte each, biased and stage-tiled for the int8
//     GEMM (exact, |q| <= 127);
//   TZH_WF_F32: f32 weights [n, k] row-major for the f32 matrix-core GEMM
//     (gemm_fp.hip), C = X W^T + b.
struct DevLinear {
    void *w = nullptr;
    int32_t fmt = TZH_WF_F32;
    uint16_t *s = nullptr;
    float *b = nullptr;
    // per concatenated part (Q, K, V for the QKV linear): the largest
    // sum_k |W[j,k]| (int8: |q| * s) and the largest |bias[j]| over its rows,
    // so that |output| <= gain * max|input| + bmax
    float gain[3] = {}, bmax[3] = {};
};

struct DevLayer {
    DevLinear qkv, o, ffn1, ffn2;
    float *ln1_g = nullptr, *ln1_b = nullptr, *ln2_g = nullptr, *ln2_b = nullptr;
    // both feed-forward linears int8: their codes widened to f16 in the
    // fragment order of the fused feed-forward kernel (mlp.hip); mlp_o: the
    // O-projection's too, when it is int8 as well (the kernel then starts
    // from the attention context)
    void *mlp = nullptr, *mlp_o = nullptr;
    // qkvp: W_qkv in the fragment order of the same kernel's QKV mode
    void *qkvp = nullptr;
};

}  // namespace

struct tzh_model {
    tzh_ctx *ctx = nullptr;
    tzh_arctic_config cfg{};
    std::vector<void *> allocs;  // weight allocations
    DevTable word, pos, type;
    float *emb_g = nullptr, *emb_b = nullptr;
    std::vector<DevLayer> layers;
    // workspace, grown on demand
    int64_t cap_tokens = 0;
    int cap_batch = 0;
    // activation element type chosen by tzh_arctic_set_precision: TZH_F32
    // (the reference's) or TZH_F16 (opt-in, int8 models only)
    int32_t act = TZH_F32;
    size_t cap_es = 0;       // activation bytes per element the workspace was sized for
    void *h = nullptr, *h1 = nullptr, *qkv = nullptr, *attn = nullptr, *inter = nullptr;
    float *ln_ws = nullptr;  // f32 rows of a split LayerNorm GEMM round
    int64_t ln_ws_rows = 0;
    // Range of the f32 forward's f16 hi/lo splits (set at upload from the
    // weights): row_scaled when some int8 GEMM's input bound reaches 2^15
    // (the int8 GEMMs then run row-scaled); attn_bound, the bound of the
    // attention's split inputs (|q| log2(e)/sqrt(32), |k|, |v|) over the layers
    bool row_scaled = false;
    float attn_bound = 0.0f;
    // f32 forwards run the feed-forward block as one kernel (mlp.hip) where
    // the layer has its pack and no row scaling (tzh_arctic_set_ffn_fusion);
    // mlp_tail: that kernel's scratch for splitting its last round of panels
    bool fuse_ffn = true;
    void *mlp_tail = nullptr;
    size_t mlp_tail_bytes = 0;
    uint32_t *tok_ids = nullptr;
    int32_t *tok_pos = nullptr;
    int *meta = nullptr;  // device: cu[batch+1] | order[batch]
    int *bad_ids = nullptr;
    int *host_meta = nullptr;  // pinned staging
    hipEvent_t meta_done = nullptr;
    // host-slice entry points: pinned id staging, device ids and outputs
    uint32_t *host_ids = nullptr;
    int64_t host_ids_cap = 0;
    uint32_t *dev_ids = nullptr;
    int64_t dev_ids_cap = 0;
    float *dev_out = nullptr;
    int64_t dev_out_cap = 0;
    int last_launches = 0;
    // launch timing (tzh_arctic_set_timing): events[0] before the first
    // launch, events[i+1] after launch i, names[i] = its stage name; each
    // stage issued timing_reps times between its events
    bool timing = false;
    int timing_reps = 1;
    std::vector<hipEvent_t> events;
    std::vector<const char *> names;
    std::vector<int> name_reps;  // launches of each stage between its events
    int timed = 0;
};

namespace {

int dev_alloc(tzh_model *m, void **p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) {
        (void)hipGetLastError();
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "device allocation of %zu bytes failed", bytes);
    }
    m->allocs.push_back(*p);
    return TZH_OK;
}

template <typename T>
int upload(tzh_model *m, T **dst, const void *src, size_t count) {
    TZH_TRY(dev_alloc(m, (void **)dst, count * sizeof(T)));
    TZH_HIP(hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice));
    return TZH_OK;
}

int check_vec(const float *p, const char *what) {
    return p ? TZH_OK : tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s", what);
}

int upload_table(tzh_model *m, const tzh_mat_view &v, int64_t rows, DevTable &t, const char *what) {
    if (!v.data) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s", what);
    if (v.rows != rows || v.cols != H)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "%s has shape [%d,%d], expected [%lld,%d]", what, v.rows, v.cols,
                        (long long)rows, H);
    if (v.dtype == TZH_F32) return upload<float>(m, &t.f32, v.data, (size_t)rows * H);
    if (v.dtype == TZH_I8) {
        if (!v.scale) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s.scale", what);
        TZH_TRY(upload<int8_t>(m, &t.q8, v.data, (size_t)rows * H));
        return upload<uint16_t>(m, &t.scale, v.scale, (size_t)rows);
    }
    return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "Weight %s has unsupported dtype %d", what, v.dtype);
}

// Concatenate the row blocks of several [rows_i, cols] linears into one
// matrix (QKV fusion) with its biases.  Each block is int8 (I8 + F16 scale,
// the quantized model) or F32 (the f32 model).  Blocks that are all int8
// become tiled codes (TZH_WF_W8T); otherwise the linear is f32
// (TZH_WF_F32), its int8 blocks widened to f32(q) * f32(s), which is exact
// (an 8-bit code times an 11-bit scale fits the f32 significand).  Only a
// QKV whose three parts differ in dtype takes that widening; the product
// (x . (q s)) then differs from the reference's (x . q) * s by the rounding
// of f32 sums only.
int upload_linear(tzh_model *m, std::initializer_list<std::pair<const tzh_mat_view *, const float *>> parts,
                  int cols, DevLinear &out, const char *what) {
    int64_t rows = 0;
    for (auto &pb : parts) {
        const tzh_mat_view *v = pb.first;
        if (!v->data) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s", what);
        if (!pb.second) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s bias", what);
        if (v->dtype != TZH_I8 && v->dtype != TZH_F32)
            return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "Weight %s has unsupported dtype %d", what, v->dtype);
        if (v->dtype == TZH_I8 && !v->scale) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s.scale", what);
        if (v->cols != cols) return tzh_fail(TZH_ERR_INVALID_ARGS, "%s has %d columns, expected %d", what, v->cols, cols);
        rows += v->rows;
    }
    if (parts.size() > 3) return tzh_fail(TZH_ERR_INVALID_ARGS, "%s: too many parts", what);
    int pi = 0;
    for (auto &pb : parts) {
        const tzh_mat_view *v = pb.first;
        float g = 0.0f, bm = 0.0f;
        for (int r = 0; r < v->rows; r++) {
            double l1 = 0.0;
            if (v->dtype == TZH_F32) {
                const float *w = (const float *)v->data + (size_t)r * cols;
                for (int c = 0; c < cols; c++) l1 += std::fabs((double)w[c]);
            } else {
                const int8_t *q = (const int8_t *)v->data + (size_t)r * cols;
                for (int c = 0; c < cols; c++) l1 += std::abs((int)q[c]);
                l1 *= (double)tzh_host_f16_to_f32(((const uint16_t *)v->scale)[r]);
            }
            g = std::max(g, (float)l1);
            bm = std::max(bm, std::fabs(pb.second[r]));
        }
        out.gain[pi] = g;
        out.bmax[pi] = bm;
        pi++;
    }
    bool all_i8 = true;
    for (auto &pb : parts) all_i8 = all_i8 && pb.first->dtype == TZH_I8;
    if (!all_i8 || rows % 384 != 0 || cols % 64 != 0) {
        // MatWeight.f32 (arctic.zig:55-58): the rows as they are, [n, k]
        // row-major, for the f32 GEMM on the matrix cores (gemm_fp.hip)
        std::vector<float> w((size_t)(rows * cols)), b((size_t)rows);
        int64_t r0 = 0;
        for (auto &pb : parts) {
            const tzh_mat_view *v = pb.first;
            float *dst = w.data() + (size_t)r0 * cols;
            if (v->dtype == TZH_F32) {
                std::memcpy(dst, v->data, (size_t)v->rows * cols * 4);
            } else {
                const int8_t *q = (const int8_t *)v->data;
                const uint16_t *sc = (const uint16_t *)v->scale;
                for (int r = 0; r < v->rows; r++) {
                    const float s = tzh_host_f16_to_f32(sc[r]);
                    for (int c = 0; c < cols; c++) dst[(size_t)r * cols + c] = (float)q[(size_t)r * cols + c] * s;
                }
            }
            std::memcpy(b.data() + r0, pb.second, (size_t)v->rows * 4);
            r0 += v->rows;
        }
        out.fmt = TZH_WF_F32;
        out.s = nullptr;
        TZH_TRY(upload<float>(m, (float **)&out.w, w.data(), w.size()));
        return upload<float>(m, &out.b, b.data(), b.size());
    }
    // biased codes u = q + 128, stage-tiled: block of 384 rows, k stage of
    // 64 codes, row (the layout tile_codes_w8_kernel writes)
    const int kts = cols / 64;
    std::vector<uint8_t> t((size_t)(rows * cols));
    std::vector<uint16_t> s;
    std::vector<float> b;
    int64_t r0 = 0;
    for (auto &pb : parts) {
        const tzh_mat_view *v = pb.first;
        const int8_t *q = (const int8_t *)v->data;
        for (int r = 0; r < v->rows; r++) {
            const int64_t n = r0 + r;
            for (int kt = 0; kt < kts; kt++) {
                uint8_t *dst = &t[(size_t)((((n / 384) * kts + kt) * 384 + n % 384) * 64)];
                const int8_t *src = q + (size_t)r * cols + (size_t)kt * 64;
                for (int c = 0; c < 64; c++) dst[c] = (uint8_t)src[c] ^ 0x80u;
            }
        }
        s.insert(s.end(), (const uint16_t *)v->scale, (const uint16_t *)v->scale + v->rows);
        b.insert(b.end(), pb.second, pb.second + v->rows);
        r0 += v->rows;
    }
    out.fmt = TZH_WF_W8T;
    TZH_TRY(upload<uint8_t>(m, (uint8_t **)&out.w, t.data(), t.size()));
    TZH_TRY(upload<uint16_t>(m, &out.s, s.data(), s.size()));
    return upload<float>(m, &out.b, b.data(), b.size());
}

int check_config(const tzh_arctic_config &c) {
    if (c.hidden_size != H || c.num_attention_heads != 12 || c.intermediate_size != 1536)
        return tzh_fail(TZH_ERR_INVALID_ARGS,
                        "kernels are specialised for hidden 384, 12 heads, intermediate 1536 (got %d, %d, %d)",
                        c.hidden_size, c.num_attention_heads, c.intermediate_size);
    if (c.num_hidden_layers < 1 || c.num_hidden_layers > 64) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad layer count");
    if (c.max_position_embeddings < 1 || c.max_position_embeddings > 512)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "max_position_embeddings must be in [1, 512]");
    if (c.vocab_size < 1 || c.type_vocab_size < 1) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad vocab sizes");
    return TZH_OK;
}

void free_workspace(tzh_model *m) {
    void *bufs[] = {m->h, m->h1, m->qkv, m->attn, m->inter, m->ln_ws, m->tok_ids, m->tok_pos, m->meta};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    m->h = m->h1 = m->qkv = m->attn = m->inter = nullptr;
    m->ln_ws = nullptr;
    m->ln_ws_rows = 0;
    m->tok_ids = nullptr;
    m->tok_pos = nullptr;
    m->meta = nullptr;
    if (m->host_meta) (void)hipHostFree(m->host_meta);
    m->host_meta = nullptr;
    m->cap_tokens = 0;
    m->cap_batch = 0;
    m->cap_es = 0;
}

// The activation type a forward runs with: a model whose linears are all
// int8 (TZH_WF_W8T) runs in the chosen precision; any model with an f32
// linear runs in f32, each linear on its own format's GEMM (the f32 GEMM
// takes f32 activations only).
int32_t model_act(const tzh_model *m) {
    bool all_w8t = true;
    for (const DevLayer &d : m->layers)
        for (const DevLinear *l : {&d.qkv, &d.o, &d.ffn1, &d.ffn2}) all_w8t = all_w8t && l->fmt == TZH_WF_W8T;
    return all_w8t ? m->act : TZH_F32;
}

// y[T, n] = ops(x[T, k] W^T) + C for an f32-weight linear (W [n, k]), ops =
// bias add then `act_op` (or the bias add alone when act_op < 0).
int linear_f32w(hipStream_t st, const float *x, const DevLinear &l, float *y, int64_t T, int64_t k, int64_t n,
                int act_op, const float *residual) {
    tzh_gemm_desc d;
    d.m = T, d.n = n, d.k = k, d.lda = k, d.ldb = k, d.ldy = n;
    d.bias = l.b;
    d.ops[0] = TZH_OP_ADD;
    d.n_ops = 1;
    if (act_op >= 0) d.ops[d.n_ops++] = act_op;
    if (residual) d.c = residual, d.beta = 1.0, d.c_rs = n, d.c_cs = 1;
    return tzh_gemm_fp_launch(st, TZH_F32, false, true, x, l.w, y, d);
}

int layernorm_rows(hipStream_t st, const float *x, const float *g, const float *b, float *y, int64_t rows, int n,
                   float eps) {
    if (rows == 0) return TZH_OK;
    hipLaunchKernelGGL(layernorm_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, g, b, y, rows,
                       n, eps);
    TZH_LAUNCHED("layernorm_rows_kernel");
    return TZH_OK;
}

// The feed-forward block of layer d (feedForward, arctic.zig:760-811), y =
// LayerNorm(x + GELU(x W1^T + b1) W2^T + b2) for x, y [T, 384] in the
// activation type act: one kernel (mlp.hip) in f32 when both linears are
// int8 and their inputs need no row scaling, else the GEMM pair through the
// workspace's intermediate (`part` 1: the GELU GEMM, 2: the LayerNorm GEMM;
// an f32 second linear writes its pre-norm rows to the workspace's attn).
bool ffn_fused(const tzh_model *m, const DevLayer &d, int32_t act, bool rs) {
    return m->fuse_ffn && d.mlp && act == TZH_F32 && !rs;
}

int ffn_part(tzh_model *m, const DevLayer &d, hipStream_t st, int32_t act, bool rs, const void *x, void *y, int64_t T,
             int part) {
    const int cus = m->ctx->num_cus;
    const float eps = m->cfg.layer_norm_eps;
    if (part == 0)
        return tzh_mlp_fused_launch(st, cus, (const float *)x, d.mlp, d.ffn1.s, d.ffn1.b, d.ffn2.s, d.ffn2.b, d.ln2_g,
                                    d.ln2_b, eps, (float *)y, T, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                    nullptr, m->mlp_tail, m->mlp_tail_bytes);
    if (part == 1) {
        if (d.ffn1.fmt == TZH_WF_F32)
            return linear_f32w(st, (const float *)x, d.ffn1, (float *)m->inter, T, H, 1536, TZH_OP_GELU, nullptr);
        return tzh_linear_codes_launch(st, cus, x, act, d.ffn1.w, d.ffn1.fmt, d.ffn1.s, d.ffn1.b, m->inter, act, T, H,
                                       1536, 1536, TZH_EPI_BIAS_GELU, nullptr, nullptr, nullptr, 0.0f, nullptr, 0, rs);
    }
    if (d.ffn2.fmt == TZH_WF_F32) {
        TZH_TRY(linear_f32w(st, (const float *)m->inter, d.ffn2, (float *)m->attn, T, 1536, H, -1, (const float *)x));
        return layernorm_rows(st, (const float *)m->attn, d.ln2_g, d.ln2_b, (float *)y, T, H, eps);
    }
    return tzh_linear_codes_launch(st, cus, m->inter, act, d.ffn2.w, d.ffn2.fmt, d.ffn2.s, d.ffn2.b, y, act, T, 1536, H,
                                   H, TZH_EPI_BIAS_RES_LN, x, d.ln2_g, d.ln2_b, eps, m->ln_ws, m->ln_ws_rows, rs);
}

int ensure_workspace(tzh_model *m, int64_t tokens, int batch, size_t es) {
    if (tokens <= m->cap_tokens && batch <= m->cap_batch && es <= m->cap_es) return TZH_OK;
    TZH_HIP(hipStreamSynchronize(m->ctx->stream));
    const int64_t T = std::max<int64_t>(tokens, m->cap_tokens);
    const int B = std::max(batch, m->cap_batch);
    free_workspace(m);
    auto get = [&](void **p, size_t bytes) -> int {
        if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) {
            (void)hipGetLastError();
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "workspace allocation of %zu bytes failed", bytes);
        }
        return TZH_OK;
    };
    const size_t E = std::max(es, m->cap_es);
    TZH_TRY(get((void **)&m->h, (size_t)T * H * E));
    TZH_TRY(get((void **)&m->h1, (size_t)T * H * E));
    TZH_TRY(get((void **)&m->qkv, (size_t)T * 3 * H * E));
    TZH_TRY(get((void **)&m->attn, (size_t)T * H * E));
    TZH_TRY(get((void **)&m->inter, (size_t)T * 1536 * E));
    // a split partial round is at most a third of the CUs' 128-row tiles
    m->ln_ws_rows = std::min<int64_t>((T + 127) / 128, m->ctx->num_cus / 3 + 1) * 128;
    TZH_TRY(get((void **)&m->ln_ws, (size_t)m->ln_ws_rows * H * 4));
    TZH_TRY(get((void **)&m->tok_ids, (size_t)T * 4));
    TZH_TRY(get((void **)&m->tok_pos, (size_t)T * 4));
    TZH_TRY(get((void **)&m->meta, (size_t)(2 * B + 1) * 4));
    if (hipHostMalloc((void **)&m->host_meta, (size_t)(2 * B + 1) * 4, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        m->host_meta = nullptr;
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "pinned staging allocation failed");
    }
    m->cap_tokens = T;
    m->cap_batch = B;
    m->cap_es = E;
    return TZH_OK;
}

int model_new(tzh_ctx *ctx, const tzh_arctic_config &cfg, tzh_model **out) {
    TZH_TRY(check_config(cfg));
    unsigned *queue = nullptr;  // the attention's work queue, allocated now so that forwards never allocate it
    TZH_TRY(tzh_ctx_work_queue(ctx, &queue));
    tzh_model *m = new (std::nothrow) tzh_model();
    if (!m) return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "model allocation failed");
    m->ctx = ctx;
    m->cfg = cfg;
    m->layers.resize((size_t)cfg.num_hidden_layers);
    if (hipEventCreateWithFlags(&m->meta_done, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        delete m;
        return tzh_fail(TZH_ERR_DEVICE, "event creation failed");
    }
    void *bad = nullptr;
    if (dev_alloc(m, &bad, 16) != TZH_OK || hipMemset(bad, 0, 16) != hipSuccess) {
        (void)hipEventDestroy(m->meta_done);
        for (void *p : m->allocs) (void)hipFree(p);
        delete m;
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "allocation failed");
    }
    m->bad_ids = (int *)bad;
    *out = m;
    return TZH_OK;
}

void model_delete(tzh_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_workspace(m);
    if (m->host_ids) (void)hipHostFree(m->host_ids);
    if (m->dev_ids) (void)hipFree(m->dev_ids);
    if (m->dev_out) (void)hipFree(m->dev_out);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->meta_done) (void)hipEventDestroy(m->meta_done);
    for (hipEvent_t e : m->events) (void)hipEventDestroy(e);
    delete m;
}

// Bounds on the f32 forward's activations, from the weights alone: a
// LayerNorm output has |(x - mean) / std| <= sqrt(n - 1) (one element
// against n - 1 equal ones), so |y| <= sqrt(383) max|gamma| + max|beta|; a
// linear maps max|x| <= B to |y_j| <= B sum_k |W[j,k]| + |b_j|; attention
// outputs are convex combinations of V rows; |gelu(x)| <= max(|x|, 0.17).
// The f16 hi/lo split of an input is exact to 2^-22 for |x| < 65504; a
// margin of two covers the rounding of these sums.  A GEMM whose input bound
// reaches 2^15 makes the forward row-scale its int8 GEMMs (exact for any
// f32 input); the attention's bound is checked at each forward.
void set_range(tzh_model *m, const tzh_arctic_weights *w) {
    constexpr float kLimit = 32768.0f;
    auto ln_bound = [](const float *g, const float *b) {
        float mg = 0.0f, mb = 0.0f;
        for (int i = 0; i < H; i++) {
            mg = std::max(mg, std::fabs(g[i]));
            mb = std::max(mb, std::fabs(b[i]));
        }
        return std::sqrt((float)(H - 1)) * mg + mb;
    };
    auto out_bound = [](const DevLinear &l, int part, float in) { return in * l.gain[part] + l.bmax[part]; };
    bool rs = false;
    float attn = 0.0f;
    auto need = [&](const DevLinear &l, float in) {
        if (l.fmt == TZH_WF_W8T && !(in < kLimit)) rs = true;
    };
    float bh = ln_bound(w->layer_norm_gamma, w->layer_norm_beta);
    for (size_t li = 0; li < m->layers.size(); li++) {
        const DevLayer &d = m->layers[li];
        const tzh_layer_weights &lw = w->layers[li];
        need(d.qkv, bh);
        const float bq = out_bound(d.qkv, 0, bh), bk = out_bound(d.qkv, 1, bh), bv = out_bound(d.qkv, 2, bh);
        attn = std::max({attn, bq * 0.2551f, bk, bv});  // q is scaled by log2(e)/sqrt(32) before its split
        need(d.o, bv);
        const float bh1 = ln_bound(lw.attention.output_ln_gamma, lw.attention.output_ln_beta);
        need(d.ffn1, bh1);
        need(d.ffn2, std::max(out_bound(d.ffn1, 0, bh1), 0.17f));
        bh = ln_bound(lw.ffn.output_ln_gamma, lw.ffn.output_ln_beta);
    }
    m->row_scaled = rs;
    m->attn_bound = attn;
}

int upload_weights(tzh_model *m, const tzh_arctic_weights *w) {
    const tzh_arctic_config &c = m->cfg;
    TZH_TRY(upload_table(m, w->word_embeddings, c.vocab_size, m->word, "embeddings.word_embeddings.weight"));
    TZH_TRY(upload_table(m, w->position_embeddings, c.max_position_embeddings, m->pos,
                         "embeddings.position_embeddings.weight"));
    TZH_TRY(upload_table(m, w->token_type_embeddings, c.type_vocab_size, m->type,
                         "embeddings.token_type_embeddings.weight"));
    TZH_TRY(check_vec(w->layer_norm_gamma, "embeddings.LayerNorm.weight"));
    TZH_TRY(check_vec(w->layer_norm_beta, "embeddings.LayerNorm.bias"));
    TZH_TRY(upload<float>(m, &m->emb_g, w->layer_norm_gamma, H));
    TZH_TRY(upload<float>(m, &m->emb_b, w->layer_norm_beta, H));
    if (!w->layers) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: encoder layers");
    for (int l = 0; l < c.num_hidden_layers; l++) {
        const tzh_layer_weights &lw = w->layers[l];
        DevLayer &d = m->layers[(size_t)l];
        const tzh_attention_weights &a = lw.attention;
        const tzh_ffn_weights &f = lw.ffn;
        for (const tzh_mat_view *v : {&a.query_weight, &a.key_weight, &a.value_weight, &a.output_weight})
            if (v->data && (v->rows != H || v->cols != H))
                return tzh_fail(TZH_ERR_INVALID_ARGS, "layer %d attention weight shape [%d,%d]", l, v->rows, v->cols);
        if (f.intermediate_weight.data && (f.intermediate_weight.rows != 1536 || f.intermediate_weight.cols != H))
            return tzh_fail(TZH_ERR_INVALID_ARGS, "layer %d intermediate weight shape", l);
        if (f.output_weight.data && (f.output_weight.rows != H || f.output_weight.cols != 1536))
            return tzh_fail(TZH_ERR_INVALID_ARGS, "layer %d output weight shape", l);
        TZH_TRY(upload_linear(m, {{&a.query_weight, a.query_bias}, {&a.key_weight, a.key_bias},
                                  {&a.value_weight, a.value_bias}}, H, d.qkv, "attention.self.{query,key,value}.weight"));
        TZH_TRY(upload_linear(m, {{&a.output_weight, a.output_bias}}, H, d.o, "attention.output.dense.weight"));
        TZH_TRY(upload_linear(m, {{&f.intermediate_weight, f.intermediate_bias}}, H, d.ffn1, "intermediate.dense.weight"));
        TZH_TRY(upload_linear(m, {{&f.output_weight, f.output_bias}}, 1536, d.ffn2, "output.dense.weight"));
        TZH_TRY(check_vec(a.output_ln_gamma, "attention.output.LayerNorm.weight"));
        TZH_TRY(check_vec(a.output_ln_beta, "attention.output.LayerNorm.bias"));
        TZH_TRY(check_vec(f.output_ln_gamma, "output.LayerNorm.weight"));
        TZH_TRY(check_vec(f.output_ln_beta, "output.LayerNorm.bias"));
        TZH_TRY(upload<float>(m, &d.ln1_g, a.output_ln_gamma, H));
        TZH_TRY(upload<float>(m, &d.ln1_b, a.output_ln_beta, H));
        TZH_TRY(upload<float>(m, &d.ln2_g, f.output_ln_gamma, H));
        TZH_TRY(upload<float>(m, &d.ln2_b, f.output_ln_beta, H));
        if (d.ffn1.fmt == TZH_WF_W8T && d.ffn2.fmt == TZH_WF_W8T) {
            TZH_TRY(dev_alloc(m, &d.mlp, tzh_mlp_pack_bytes()));
            TZH_TRY(tzh_mlp_pack_launch(m->ctx->stream, d.ffn1.w, d.ffn2.w, d.mlp));
            if (!m->mlp_tail) {
                m->mlp_tail_bytes = tzh_mlp_tail_bytes(m->ctx->num_cus);
                TZH_TRY(dev_alloc(m, &m->mlp_tail, m->mlp_tail_bytes));
            }
            if (d.o.fmt == TZH_WF_W8T) {
                TZH_TRY(dev_alloc(m, &d.mlp_o, tzh_mlp_opack_bytes()));
                TZH_TRY(tzh_mlp_opack_launch(m->ctx->stream, d.o.w, d.mlp_o));
            }
        }
        if (d.qkv.fmt == TZH_WF_W8T) {
            TZH_TRY(dev_alloc(m, &d.qkvp, tzh_qkv_pack_bytes()));
            TZH_TRY(tzh_qkv_pack_launch(m->ctx->stream, d.qkv.w, d.qkvp));
        }
    }
    TZH_HIP(hipStreamSynchronize(m->ctx->stream));
    set_range(m, w);
    return TZH_OK;
}

// ---------------------------------------------------------------------------
// safetensors -> host views (arctic.zig:113-166, 258-287)
// ---------------------------------------------------------------------------
// Host tensors of a safetensors file (read into memory) or of a mapped
// .tenzor file, looked up by name.
struct HostStore {
    StFile st;
    TzFile tz;
    bool tenzor = false;
    std::vector<std::vector<uint8_t>> owned;  // aligned copies
};

struct HostTensor {
    int32_t dtype;  // TZH_*
    std::vector<int64_t> shape;
    const uint8_t *data;
    size_t bytes;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

bool find_tensor(const HostStore &hs, const std::string &name, HostTensor &out) {
    if (hs.tenzor) {
        const tzh_tenzor_entry *e = hs.tz.find(name);
        if (!e) return false;
        out.dtype = tenzor_dtype_to_tzh(e->dtype);
        out.shape.assign(e->shape, e->shape + (e->ndim < 5 ? e->ndim : 5));
        out.data = hs.tz.data + e->data_offset;
        out.bytes = (size_t)e->data_size;
        return true;
    }
    const StTensor *t = hs.st.get(name);
    if (!t) return false;
    out.dtype = t->dtype;
    out.shape = t->shape;
    out.data = hs.st.data(*t);
    out.bytes = (size_t)(t->end - t->start);
    return true;
}

const void *aligned_data(HostStore &hs, const HostTensor &t) {
    const int es = st_dtype_size(t.dtype);
    if (((uintptr_t)t.data % (uintptr_t)es) == 0) return t.data;  // safetensors.zig:147-161
    hs.owned.emplace_back(t.data, t.data + t.bytes);
    return hs.owned.back().data();
}

// The tensor's bytes must be its shape's worth (the formats do not check).
int find_checked(HostStore &hs, const std::string &name, HostTensor &t) {
    if (!find_tensor(hs, name, t)) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "Missing weight: %s", name.c_str());
    if (t.dtype < 0) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "Weight %s has an unknown dtype", name.c_str());
    if ((uint64_t)t.numel() * (uint64_t)st_dtype_size(t.dtype) != t.bytes)
        return tzh_fail(TZH_ERR_INVALID_FORMAT, "Weight %s: %zu bytes for its shape", name.c_str(), t.bytes);
    return TZH_OK;
}

int get_f32(HostStore &hs, const std::string &name, const float **out) {
    HostTensor t;
    TZH_TRY(find_checked(hs, name, t));
    if (t.dtype != TZH_F32) return tzh_fail(TZH_ERR_WRONG_DTYPE, "Weight %s has wrong dtype, expected F32", name.c_str());
    *out = (const float *)aligned_data(hs, t);
    return TZH_OK;
}

int get_f32_alt(HostStore &hs, const std::string &primary, const std::string &alt, const float **out) {
    HostTensor t;
    if (find_tensor(hs, primary, t)) return get_f32(hs, primary, out);  // arctic.zig:245-256
    return get_f32(hs, alt, out);
}

int get_mat(HostStore &hs, const std::string &name, tzh_mat_view &v) {
    HostTensor t;
    TZH_TRY(find_checked(hs, name, t));
    std::memset(&v, 0, sizeof v);
    if (t.shape.size() != 2)
        return tzh_fail(TZH_ERR_INVALID_FORMAT, "Weight %s must be 2-D", name.c_str());
    v.rows = (int32_t)t.shape[0];
    v.cols = (int32_t)t.shape[1];
    if (t.dtype == TZH_F32) {
        v.dtype = TZH_F32;
        v.data = aligned_data(hs, t);
        return TZH_OK;
    }
    if (t.dtype == TZH_I8) {  // arctic.zig:273-281
        v.dtype = TZH_I8;
        v.data = aligned_data(hs, t);
        const std::string sname = name + ".scale";
        HostTensor s;
        TZH_TRY(find_checked(hs, sname, s));
        if (s.dtype != TZH_F16) return tzh_fail(TZH_ERR_WRONG_DTYPE, "Weight %s has wrong dtype, expected F16", sname.c_str());
        if (s.numel() != v.rows) return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s has %lld entries, expected %d", sname.c_str(), (long long)s.numel(), v.rows);
        v.scale = (const uint16_t *)aligned_data(hs, s);
        return TZH_OK;
    }
    return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "Weight %s has unsupported dtype %s", name.c_str(), st_dtype_name(t.dtype));
}

}  // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
extern "C" int tzh_arctic_upload(tzh_ctx *ctx, const tzh_arctic_weights *weights, tzh_model **out) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!weights || !out) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *out = nullptr;
    tzh_model *m = nullptr;
    TZH_TRY(model_new(ctx, weights->config, &m));
    const int rc = upload_weights(m, weights);
    if (rc != TZH_OK) {
        const std::string msg = tzh_last_error();
        model_delete(m);
        return tzh_fail(rc, "%s", msg.c_str());
    }
    *out = m;
    return TZH_OK;
}

// ModelWeights.fromSafeTensors (arctic.zig:113-166) over either file format.
static int load_from_store(tzh_ctx *ctx, HostStore &hs, const tzh_arctic_config *config, tzh_model **out) {
    HostTensor probe;
    const bool bert = find_tensor(hs, "bert.embeddings.word_embeddings.weight", probe);  // arctic.zig:131
    const std::string pre = bert ? "bert." : "";
    tzh_arctic_weights w;
    std::memset(&w, 0, sizeof w);
    w.config = *config;
    TZH_TRY(check_config(*config));
    TZH_TRY(get_mat(hs, pre + "embeddings.word_embeddings.weight", w.word_embeddings));
    TZH_TRY(get_mat(hs, pre + "embeddings.position_embeddings.weight", w.position_embeddings));
    TZH_TRY(get_mat(hs, pre + "embeddings.token_type_embeddings.weight", w.token_type_embeddings));
    TZH_TRY(get_f32_alt(hs, pre + "embeddings.LayerNorm.weight", pre + "embeddings.LayerNorm.gamma", &w.layer_norm_gamma));
    TZH_TRY(get_f32_alt(hs, pre + "embeddings.LayerNorm.bias", pre + "embeddings.LayerNorm.beta", &w.layer_norm_beta));
    std::vector<tzh_layer_weights> layers((size_t)config->num_hidden_layers);
    for (int l = 0; l < config->num_hidden_layers; l++) {
        const std::string b = pre + "encoder.layer." + std::to_string(l) + ".";  // arctic.zig:302
        tzh_attention_weights &a = layers[(size_t)l].attention;
        tzh_ffn_weights &f = layers[(size_t)l].ffn;
        TZH_TRY(get_mat(hs, b + "attention.self.query.weight", a.query_weight));
        TZH_TRY(get_f32(hs, b + "attention.self.query.bias", &a.query_bias));
        TZH_TRY(get_mat(hs, b + "attention.self.key.weight", a.key_weight));
        TZH_TRY(get_f32(hs, b + "attention.self.key.bias", &a.key_bias));
        TZH_TRY(get_mat(hs, b + "attention.self.value.weight", a.value_weight));
        TZH_TRY(get_f32(hs, b + "attention.self.value.bias", &a.value_bias));
        TZH_TRY(get_mat(hs, b + "attention.output.dense.weight", a.output_weight));
        TZH_TRY(get_f32(hs, b + "attention.output.dense.bias", &a.output_bias));
        TZH_TRY(get_f32_alt(hs, b + "attention.output.LayerNorm.weight", b + "attention.output.LayerNorm.gamma", &a.output_ln_gamma));
        TZH_TRY(get_f32_alt(hs, b + "attention.output.LayerNorm.bias", b + "attention.output.LayerNorm.beta", &a.output_ln_beta));
        TZH_TRY(get_mat(hs, b + "intermediate.dense.weight", f.intermediate_weight));
        TZH_TRY(get_f32(hs, b + "intermediate.dense.bias", &f.intermediate_bias));
        TZH_TRY(get_mat(hs, b + "output.dense.weight", f.output_weight));
        TZH_TRY(get_f32(hs, b + "output.dense.bias", &f.output_bias));
        TZH_TRY(get_f32_alt(hs, b + "output.LayerNorm.weight", b + "output.LayerNorm.gamma", &f.output_ln_gamma));
        TZH_TRY(get_f32_alt(hs, b + "output.LayerNorm.bias", b + "output.LayerNorm.beta", &f.output_ln_beta));
    }
    w.layers = layers.data();
    return tzh_arctic_upload(ctx, &w, out);
}

extern "C" int tzh_arctic_load_safetensors(tzh_ctx *ctx, const char *path, const tzh_arctic_config *config,
                                           tzh_model **out) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!out || !config || !path) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *out = nullptr;
    HostStore hs;
    TZH_TRY(st_load(path, hs.st));
    return load_from_store(ctx, hs, config, out);
}

extern "C" int tzh_arctic_load_tenzor(tzh_ctx *ctx, const char *path, const tzh_arctic_config *config,
                                      tzh_model **out) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!out || !config || !path) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *out = nullptr;
    HostStore hs;
    hs.tenzor = true;
    TZH_TRY(hs.tz.open(path));
    return load_from_store(ctx, hs, config, out);
}

extern "C" int tzh_arctic_free(tzh_model *model) {
    model_delete(model);
    return TZH_OK;
}

namespace {

__global__ void f16_to_f32_kernel(const _Float16 *__restrict__ x, float *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (float)x[i];
}

// Shared body of the batch entry points: embeddings, the first n_layers
// encoder layers, then either CLS + L2 into `outputs` or the f32 hidden
// state into `hidden_out`.
int run_forward(tzh_model *m, float *outputs, float *hidden_out, const uint32_t *ids, const int32_t *lengths,
                int32_t batch, int64_t ids_stride, int32_t n_layers) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    TZH_TRY(tzh_ctx_enter(m->ctx));
    if (batch == 0) return TZH_OK;  // arctic.zig:967
    if (batch < 0 || !(outputs || hidden_out) || !ids || !lengths)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "bad batch arguments");
    if (n_layers < 0 || n_layers > m->cfg.num_hidden_layers)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "n_layers %d out of range", n_layers);
    if (ids_stride < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative ids_stride");
    int64_t T = 0;
    for (int b = 0; b < batch; b++) {
        if (lengths[b] < 1 || lengths[b] > m->cfg.max_position_embeddings)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "sequence %d has length %d (must be 1..%d)", b, lengths[b],
                            m->cfg.max_position_embeddings);
        if (ids_stride && lengths[b] > ids_stride)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "sequence %d length %d exceeds ids_stride %lld", b, lengths[b],
                            (long long)ids_stride);
        T += lengths[b];
    }
    if (T > ((int64_t)1 << 30)) return tzh_fail(TZH_ERR_TOO_LARGE, "batch of %lld tokens is too large", (long long)T);
    const int32_t act = model_act(m);
    const size_t es = act == TZH_F32 ? 4 : 2;
    if (act == TZH_F32 && !(m->attn_bound < 32768.0f))
        return tzh_fail(TZH_ERR_TOO_LARGE,
                        "the weights bound the attention's inputs (|q|/sqrt(32), |k|, |v|) only by %g; the f32 "
                        "attention splits them into f16 halves, which needs a bound below 32768",
                        (double)m->attn_bound);
    TZH_TRY(ensure_workspace(m, T, batch, es));
    hipStream_t st = m->ctx->stream;

    // metadata: cu_seqlens and a longest-first order for attention
    TZH_HIP(hipEventSynchronize(m->meta_done));  // previous copy out of the staging buffer finished
    int *cu = m->host_meta, *order = m->host_meta + batch + 1;
    cu[0] = 0;
    for (int b = 0; b < batch; b++) cu[b + 1] = cu[b] + lengths[b];
    std::iota(order, order + batch, 0);
    std::stable_sort(order, order + batch, [&](int x, int y) { return lengths[x] > lengths[y]; });
    TZH_HIP(hipMemcpyAsync(m->meta, m->host_meta, (size_t)(2 * batch + 1) * 4, hipMemcpyHostToDevice, st));
    TZH_HIP(hipEventRecord(m->meta_done, st));
    const int *d_cu = m->meta, *d_order = m->meta + batch + 1;

    int launches = 0;
    // With timing on, an event after every launch (and one before the
    // first).  The events skip the system-scope fence (a writeback and
    // invalidation of the caches at every event, which would lengthen and
    // slow each timed launch); tzh_arctic_launch_times synchronises the
    // stream before it reads them.
    auto mark = [&](const char *name, int issued = 1) -> int {
        if (m->timing) {
            if ((size_t)launches + 1 >= m->events.size()) {
                hipEvent_t e;
                TZH_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
                m->events.push_back(e);
            }
            m->names.resize((size_t)launches + 1);
            m->names[(size_t)launches] = name;
            m->name_reps.resize((size_t)launches + 1);
            m->name_reps[(size_t)launches] = issued;
            TZH_HIP(hipEventRecord(m->events[(size_t)launches + 1], st));
        }
        launches++;
        return TZH_OK;
    };
    if (m->timing) {
        if (m->events.empty()) {
            hipEvent_t e;
            TZH_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
            m->events.push_back(e);
        }
        TZH_HIP(hipEventRecord(m->events[0], st));
    }
    hipLaunchKernelGGL(pack_ids_kernel, dim3(batch), dim3(256), 0, st, ids, ids_stride, d_cu, m->tok_ids, m->tok_pos,
                       (uint32_t)m->cfg.vocab_size, m->bad_ids);
    TZH_LAUNCHED("pack_ids_kernel");
    TZH_TRY(mark("pack_ids"));
    // Every later stage reads buffers that it does not write, so issuing it
    // again gives the same result: with timing on, each is issued
    // timing_reps times between its events (pack_ids, which counts
    // clamped ids, once).
    const int reps = m->timing ? m->timing_reps : 1;
    auto stage = [&](const char *name, auto &&launch) -> int {
        for (int r = 0; r < reps; r++) TZH_TRY(launch());
        return mark(name, reps);
    };
    TZH_TRY(stage("embed_ln", [&]() -> int {
        if (act == TZH_F32)
            hipLaunchKernelGGL(embed_ln_kernel<float>, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, m->tok_ids,
                               m->tok_pos, T, m->word.ref(), m->pos.ref(), m->type.ref(), m->emb_g, m->emb_b,
                               m->cfg.layer_norm_eps, (float *)m->h);
        else
            hipLaunchKernelGGL(embed_ln_kernel<_Float16>, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st,
                               m->tok_ids, m->tok_pos, T, m->word.ref(), m->pos.ref(), m->type.ref(), m->emb_g,
                               m->emb_b, m->cfg.layer_norm_eps, (_Float16 *)m->h);
        TZH_LAUNCHED("embed_ln_kernel");
        return TZH_OK;
    }));
    const float eps = m->cfg.layer_norm_eps;
    for (int32_t li = 0; li < n_layers; li++) {
        const DevLayer &d = m->layers[(size_t)li];
        const int cus = m->ctx->num_cus;
        // Each linear runs on its own format's GEMM.  f32 weights: the f32
        // GEMM (f32 activations; model_act makes the forward f32 whenever a
        // linear is f32); a LayerNorm stage writes its pre-norm rows (x W^T +
        // b, then + residual) into a buffer the stage does not read (inter
        // for the O-projection, attn for FFN2) and normalises them.  int8
        // weights: the int8 GEMM in the forward's precision.
        for (const DevLinear *l : {&d.qkv, &d.o, &d.ffn1, &d.ffn2})
            if ((l->fmt != TZH_WF_F32 && l->fmt != TZH_WF_W8T) || (l->fmt == TZH_WF_F32 && act != TZH_F32))
                return tzh_fail(TZH_ERR_INVALID_ARGS, "layer %d: weight format %d cannot run with activation type %d", li,
                                l->fmt, act);
        float *const hf = (float *)m->h, *const h1f = (float *)m->h1;
        // row-scaled int8 GEMMs when the weights do not bound their inputs
        // inside the split's range (set_range)
        const bool rs = m->row_scaled && act == TZH_F32;
        TZH_TRY(stage("qkv", [&]() {
            if (d.qkv.fmt == TZH_WF_F32) return linear_f32w(st, hf, d.qkv, (float *)m->qkv, T, H, 3 * H, -1, nullptr);
            // int8 QKV of the f32 forward on the fused kernel's QKV mode
            // (X in registers, the weights streamed through LDS)
            if (m->fuse_ffn && d.qkvp && act == TZH_F32 && !rs)
                return tzh_qkv_fused_launch(st, cus, hf, d.qkvp, d.qkv.s, d.qkv.b, (float *)m->qkv, T);
            return tzh_linear_codes_launch(st, cus, m->h, act, d.qkv.w, d.qkv.fmt, d.qkv.s, d.qkv.b, m->qkv, act, T,
                                           H, 3 * H, 3 * H, TZH_EPI_BIAS, nullptr, nullptr, nullptr, 0.0f, nullptr, 0, rs);
        }));
        TZH_TRY(stage("attention", [&]() {
            return tzh_attention_launch(st, m->ctx->num_cus, m->ctx->work_queue, m->qkv, m->attn, act, d_cu, d_order,
                                        batch, 12, H);
        }));
        // the O-projection, its LayerNorm and the feed-forward block as one
        // kernel (mlp.hip) where the layer has both packs: (attn, h) -> h1,
        // then h and h1 trade places, so the next layer reads its input from
        // h (the stage writes no buffer it reads: timing repeats leave the
        // result unchanged)
        if (ffn_fused(m, d, act, rs) && d.mlp_o) {
            TZH_TRY(stage("attn_ffn", [&]() {
                return tzh_mlp_fused_launch(st, cus, nullptr, d.mlp, d.ffn1.s, d.ffn1.b, d.ffn2.s, d.ffn2.b, d.ln2_g,
                                            d.ln2_b, eps, h1f, T, (const float *)m->attn, hf, d.mlp_o, d.o.s, d.o.b,
                                            d.ln1_g, d.ln1_b, m->mlp_tail, m->mlp_tail_bytes);
            }));
            std::swap(m->h, m->h1);
            continue;
        }
        TZH_TRY(stage("attn_out_ln", [&]() {
            if (d.o.fmt == TZH_WF_F32) {
                TZH_TRY(linear_f32w(st, (const float *)m->attn, d.o, (float *)m->inter, T, H, H, -1, hf));
                return layernorm_rows(st, (const float *)m->inter, d.ln1_g, d.ln1_b, h1f, T, H, eps);
            }
            return tzh_linear_codes_launch(st, cus, m->attn, act, d.o.w, d.o.fmt, d.o.s, d.o.b, m->h1, act, T, H, H,
                                           H, TZH_EPI_BIAS_RES_LN, m->h, d.ln1_g, d.ln1_b, eps, m->ln_ws,
                                           m->ln_ws_rows, rs);
        }));
        if (ffn_fused(m, d, act, rs)) {
            TZH_TRY(stage("ffn", [&]() { return ffn_part(m, d, st, act, rs, m->h1, m->h, T, 0); }));
        } else {
            TZH_TRY(stage("ffn1_gelu", [&]() { return ffn_part(m, d, st, act, rs, m->h1, m->h, T, 1); }));
            TZH_TRY(stage("ffn2_ln", [&]() { return ffn_part(m, d, st, act, rs, m->h1, m->h, T, 2); }));
        }
    }
    if (outputs) {
        TZH_TRY(stage("cls_l2", [&]() -> int {
            if (act == TZH_F32)
                hipLaunchKernelGGL(cls_l2_kernel<float>, dim3((unsigned)((batch + 3) / 4)), dim3(256), 0, st,
                                   (const float *)m->h, d_cu, batch, outputs);
            else
                hipLaunchKernelGGL(cls_l2_kernel<_Float16>, dim3((unsigned)((batch + 3) / 4)), dim3(256), 0, st,
                                   (const _Float16 *)m->h, d_cu, batch, outputs);
            TZH_LAUNCHED("cls_l2_kernel");
            return TZH_OK;
        }));
    }
    if (hidden_out) {
        const int64_t n = T * H;
        if (act == TZH_F32) {
            TZH_HIP(hipMemcpyAsync(hidden_out, m->h, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
        } else {
            hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                               (const _Float16 *)m->h, hidden_out, n);
            TZH_LAUNCHED("f16_to_f32_kernel");
        }
        TZH_TRY(mark("hidden_f32"));
    }
    m->timed = m->timing ? launches : 0;
    m->last_launches = launches;
    return TZH_OK;
}

}  // namespace

tzh_ctx *tzh_model_ctx(const tzh_model *m) { return m->ctx; }
int tzh_model_hidden(const tzh_model *m) { return m->cfg.hidden_size; }

extern "C" int tzh_arctic_forward_batch(tzh_model *m, float *outputs, const uint32_t *ids, const int32_t *lengths,
                                        int32_t batch, int64_t ids_stride) {
    if (!outputs && batch > 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "null outputs");
    return run_forward(m, outputs, nullptr, ids, lengths, batch, ids_stride,
                       m ? m->cfg.num_hidden_layers : 0);
}

extern "C" int tzh_arctic_hidden(tzh_model *m, float *hidden, const uint32_t *ids, const int32_t *lengths,
                                 int32_t batch, int64_t ids_stride, int32_t n_layers) {
    if (!hidden && batch > 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "null hidden");
    return run_forward(m, nullptr, hidden, ids, lengths, batch, ids_stride, n_layers);
}

extern "C" int tzh_arctic_forward(tzh_model *m, float *output, const uint32_t *token_ids, int64_t seq_len) {
    if (seq_len <= 0 || seq_len > 512) return tzh_fail(TZH_ERR_INVALID_ARGS, "seq_len %lld out of range", (long long)seq_len);
    const int32_t len = (int32_t)seq_len;
    return tzh_arctic_forward_batch(m, output, token_ids, &len, 1, 0);
}

// Host-slice batch (arctic.forwardBatch / forwardBatchParallel argument
// shapes): the sequences are packed into pinned staging, uploaded with one
// copy, forwarded, and the embeddings copied back; returns when they are in
// `outputs` (host).
extern "C" int tzh_arctic_forward_batch_host(tzh_model *m, float *outputs, const tzh_ids_slice *batch,
                                             int32_t batch_n) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    TZH_TRY(tzh_ctx_enter(m->ctx));
    if (batch_n == 0) return TZH_OK;  // arctic.zig:967
    if (batch_n < 0 || !outputs || !batch) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad batch arguments");
    std::vector<int32_t> lengths((size_t)batch_n);
    int64_t T = 0;
    for (int32_t b = 0; b < batch_n; b++) {
        const uint64_t L = batch[b].len;
        if (L < 1 || L > (uint64_t)m->cfg.max_position_embeddings || !batch[b].ids)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "sequence %d has length %llu (must be 1..%d)", b,
                            (unsigned long long)L, m->cfg.max_position_embeddings);
        lengths[(size_t)b] = (int32_t)L;
        T += (int64_t)L;
    }
    hipStream_t st = m->ctx->stream;
    TZH_HIP(hipStreamSynchronize(st));  // the staging and device buffers are free again
    if (T > m->host_ids_cap) {
        if (m->host_ids) TZH_HIP(hipHostFree(m->host_ids));
        m->host_ids = nullptr;
        m->host_ids_cap = 0;
        if (hipHostMalloc((void **)&m->host_ids, (size_t)T * 4, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            m->host_ids = nullptr;
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "pinned id staging of %lld ids failed", (long long)T);
        }
        m->host_ids_cap = T;
    }
    auto grow = [](void **p, int64_t &cap, int64_t want, size_t es) -> int {
        if (want <= cap) return TZH_OK;
        if (*p) TZH_HIP(hipFree(*p));
        *p = nullptr;
        cap = 0;
        if (hipMalloc(p, (size_t)want * es) != hipSuccess) {
            (void)hipGetLastError();
            *p = nullptr;
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "device buffer of %lld elements failed", (long long)want);
        }
        cap = want;
        return TZH_OK;
    };
    TZH_TRY(grow((void **)&m->dev_ids, m->dev_ids_cap, T, 4));
    TZH_TRY(grow((void **)&m->dev_out, m->dev_out_cap, (int64_t)batch_n * H, 4));
    int64_t off = 0;
    for (int32_t b = 0; b < batch_n; b++) {
        std::memcpy(m->host_ids + off, batch[b].ids, (size_t)batch[b].len * 4);
        off += (int64_t)batch[b].len;
    }
    TZH_HIP(hipMemcpyAsync(m->dev_ids, m->host_ids, (size_t)T * 4, hipMemcpyHostToDevice, st));
    TZH_TRY(run_forward(m, m->dev_out, nullptr, m->dev_ids, lengths.data(), batch_n, 0, m->cfg.num_hidden_layers));
    TZH_HIP(hipMemcpyAsync(outputs, m->dev_out, (size_t)batch_n * H * 4, hipMemcpyDeviceToHost, st));
    TZH_HIP(hipStreamSynchronize(st));
    return TZH_OK;
}

// One host sequence (arctic.forward argument shapes).
extern "C" int tzh_arctic_forward_host(tzh_model *m, float *output, const uint32_t *token_ids, int64_t seq_len) {
    if (seq_len <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "seq_len %lld out of range", (long long)seq_len);
    const tzh_ids_slice one{token_ids, (uint64_t)seq_len};
    return tzh_arctic_forward_batch_host(m, output, &one, 1);
}

extern "C" int tzh_arctic_last_launch_count(tzh_model *m) { return m ? m->last_launches : 0; }

extern "C" int tzh_arctic_set_precision(tzh_model *m, int32_t dtype) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    if (dtype != TZH_F32 && dtype != TZH_F16)
        return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "activation precision must be F32 or F16 (got %d)", dtype);
    m->act = dtype;
    return TZH_OK;
}

extern "C" int tzh_arctic_set_ffn_fusion(tzh_model *m, int32_t enable) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    m->fuse_ffn = enable != 0;
    return TZH_OK;
}

extern "C" int tzh_arctic_feed_forward(tzh_model *m, int32_t layer, const float *input, float *output,
                                       int64_t seq_len) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    if (layer < 0 || layer >= (int32_t)m->layers.size())
        return tzh_fail(TZH_ERR_INVALID_ARGS, "layer %d out of range [0, %zu)", layer, m->layers.size());
    if (seq_len < 0 || seq_len > ((int64_t)1 << 30)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad token count");
    if (seq_len == 0) return TZH_OK;
    if (!input || !output) return tzh_fail(TZH_ERR_INVALID_ARGS, "null input or output");
    if ((((uintptr_t)input | (uintptr_t)output) & 15) != 0)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "input and output must be 16-byte aligned");
    const size_t bytes = (size_t)seq_len * H * 4;
    if ((const char *)input < (const char *)output + bytes && (const char *)output < (const char *)input + bytes)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "input and output overlap");
    TZH_TRY(tzh_ctx_enter(m->ctx));
    const DevLayer &d = m->layers[(size_t)layer];
    const bool rs = m->row_scaled;
    hipStream_t st = m->ctx->stream;
    if (ffn_fused(m, d, TZH_F32, rs)) return ffn_part(m, d, st, TZH_F32, rs, input, output, seq_len, 0);
    TZH_TRY(ensure_workspace(m, seq_len, 1, 4));
    TZH_TRY(ffn_part(m, d, st, TZH_F32, rs, input, output, seq_len, 1));
    return ffn_part(m, d, st, TZH_F32, rs, input, output, seq_len, 2);
}

extern "C" int tzh_arctic_precision(tzh_model *m, int32_t *dtype) {
    tzh_clear_error();
    if (!m || !dtype) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *dtype = model_act(m);
    return TZH_OK;
}

extern "C" int tzh_arctic_set_timing(tzh_model *m, int32_t enable) {
    tzh_clear_error();
    if (!m) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model");
    if (enable < 0 || enable > 1000) return tzh_fail(TZH_ERR_INVALID_ARGS, "timing repetitions %d out of 0..1000", enable);
    m->timing = enable != 0;
    m->timing_reps = enable > 0 ? enable : 1;
    m->timed = 0;
    return TZH_OK;
}

extern "C" int tzh_arctic_launch_times(tzh_model *m, float *us, const char **names, int32_t capacity,
                                       int32_t *count) {
    tzh_clear_error();
    if (!m || !count) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    TZH_TRY(tzh_ctx_enter(m->ctx));
    *count = m->timed;
    if (m->timed == 0) return TZH_OK;
    TZH_HIP(hipStreamSynchronize(m->ctx->stream));
    TZH_HIP(hipEventSynchronize(m->events[(size_t)m->timed]));
    for (int i = 0; i < m->timed && i < capacity; i++) {
        float ms = 0.0f;
        TZH_HIP(hipEventElapsedTime(&ms, m->events[(size_t)i], m->events[(size_t)i + 1]));
        if (us) us[i] = ms * 1000.0f / (float)m->name_reps[(size_t)i];
        if (names) names[i] = m->names[(size_t)i];
    }
    return TZH_OK;
}

// Number of out-of-range token ids seen (and clamped) since the model was
// created; synchronises the model's stream.
extern "C" int tzh_arctic_bad_id_count(tzh_model *m, int32_t *count) {
    tzh_clear_error();
    if (!m || !count) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    TZH_TRY(tzh_ctx_enter(m->ctx));
    TZH_HIP(hipMemcpyAsync(count, m->bad_ids, 4, hipMemcpyDeviceToHost, m->ctx->stream));
    TZH_HIP(hipStreamSynchronize(m->ctx->stream));
    return TZH_OK;
}

extern "C" int tzh_layernorm_last_dim(tzh_ctx *ctx, const float *x, const float *gamma, const float *beta, float *y,
                                      int64_t rows, int64_t n, float eps) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (rows < 0 || n <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad shape");
    if (rows == 0) return TZH_OK;
    if (!x || !gamma || !beta || !y) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    hipLaunchKernelGGL(layernorm_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, ctx->stream, x, gamma,
                       beta, y, rows, (int)n, eps);
    TZH_LAUNCHED("layernorm_rows_kernel");
    return TZH_OK;
}

extern "C" int tzh_quantize_rows(tzh_ctx *ctx, const float *w, int64_t rows, int64_t cols, int8_t *q,
                                 uint16_t *scale) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (rows < 0 || cols < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad shape");
    if (rows == 0) return TZH_OK;
    if (!w || !q || !scale) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, ctx->stream, w, rows,
                       cols, q, scale);
    TZH_LAUNCHED("quantize_rows_kernel");
    return TZH_OK;
}
