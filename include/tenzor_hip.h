/*
 * tenzor_hip.h — C-ABI of the MI355X (gfx950) backend for tenzor's
 * lazy elementwise/broadcast/reduce evaluation and the int8-weight
 * Arctic-embed-xs encoder forward.
 *
 * Conventions (mirroring the Zig surfaces this library replaces):
 *   - Every entry point returns 0 (TZH_OK) on success and a negative status
 *     on failure; tzh_last_error() returns a thread-local message for the
 *     last failure.  No C++ exception crosses this boundary.
 *   - The caller owns output buffers (tensor.zig:129-134 semantics).
 *   - "device pointer" arguments are HBM addresses (hipMalloc'd, by
 *     tzh_malloc or by any HIP allocator such as torch's caching allocator on
 *     the same device).  Host pointers are marked "host".
 *   - A tzh_ctx enqueues all work asynchronously on one HIP stream chosen
 *     at tzh_init (NULL = the default stream).  tzh_sync() waits for it.  A context is not
 *     thread-safe (one per thread), like arctic.InferenceContext
 *     (arctic.zig:407-482).
 */
#ifndef TENZOR_HIP_H
#define TENZOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TZH_ABI_VERSION 2
#define TZH_MAX_RANK 8 /* shape.zig:10 MAX_RANK */

/* ------------------------------------------------------------------ */
/* Status codes.  The Zig error names they stand for are cited.        */
/* ------------------------------------------------------------------ */
enum {
    TZH_OK = 0,
    TZH_ERR_INVALID_ARGS = -1,      /* std.debug.assert preconditions, e.g. matmul_w8a32.zig:24-29 */
    TZH_ERR_OUT_OF_MEMORY = -2,     /* error.OutOfMemory */
    TZH_ERR_DEVICE = -3,            /* HIP runtime failure */
    TZH_ERR_MISSING_WEIGHT = -4,    /* error.MissingWeight, arctic.zig:194-197 */
    TZH_ERR_WRONG_DTYPE = -5,       /* error.WrongDtype, arctic.zig:198-201 */
    TZH_ERR_UNSUPPORTED_DTYPE = -6, /* error.UnsupportedDtype, arctic.zig:282-285 */
    TZH_ERR_INVALID_FORMAT = -7,    /* error.InvalidFormat, safetensors.zig:173-180 */
    TZH_ERR_IO = -8,                /* file system errors */
    TZH_ERR_UNSUPPORTED_OP = -9,    /* @compileError("Unsupported ... operation"), elementwise.zig:143,191 */
    TZH_ERR_SHAPE = -10,            /* "Shapes not broadcast compatible", expr.zig:366-375 */
    TZH_ERR_TOO_LARGE = -11         /* input beyond a documented size limit */
};

/* Element types; numbering follows safetensors DType order (safetensors.zig:13-26). */
enum {
    TZH_F16 = 0, TZH_BF16 = 1, TZH_F32 = 2, TZH_F64 = 3,
    TZH_I8 = 4, TZH_I16 = 5, TZH_I32 = 6, TZH_I64 = 7,
    TZH_U8 = 8, TZH_U16 = 9, TZH_U32 = 10, TZH_U64 = 11, TZH_BOOL = 12
};

/* Operation tags; numbering is the ordinal of ops.OpTag (expr.zig:19-91),
 * so a Zig caller passes @intFromEnum(Expr.operation) unchanged. */
enum {
    TZH_OP_NEG = 0, TZH_OP_ABS = 1, TZH_OP_EXP = 2, TZH_OP_EXP2 = 3, TZH_OP_LOG = 4,
    TZH_OP_LOG2 = 5, TZH_OP_LOG10 = 6, TZH_OP_SQRT = 7, TZH_OP_RSQRT = 8, TZH_OP_SIN = 9,
    TZH_OP_COS = 10, TZH_OP_TAN = 11, TZH_OP_TANH = 12, TZH_OP_SINH = 13, TZH_OP_COSH = 14,
    TZH_OP_ASIN = 15, TZH_OP_ACOS = 16, TZH_OP_ATAN = 17, TZH_OP_SIGMOID = 18, TZH_OP_RELU = 19,
    TZH_OP_LEAKY_RELU = 20, TZH_OP_GELU = 21, TZH_OP_SILU = 22, TZH_OP_SOFTPLUS = 23,
    TZH_OP_CEIL = 24, TZH_OP_FLOOR = 25, TZH_OP_ROUND = 26, TZH_OP_SIGN = 27,
    TZH_OP_ADD = 28, TZH_OP_SUB = 29, TZH_OP_MUL = 30, TZH_OP_DIV = 31, TZH_OP_POW = 32,
    TZH_OP_MAX = 33, TZH_OP_MIN = 34, TZH_OP_MOD = 35, TZH_OP_ATAN2 = 36,
    TZH_OP_EQ = 37, TZH_OP_NE = 38, TZH_OP_LT = 39, TZH_OP_LE = 40, TZH_OP_GT = 41, TZH_OP_GE = 42,
    TZH_OP_MATMUL = 43, TZH_OP_TRANSPOSE = 44,
    TZH_OP_SUM = 45, TZH_OP_PROD = 46, TZH_OP_REDUCE_MAX = 47, TZH_OP_REDUCE_MIN = 48,
    TZH_OP_MEAN = 49, TZH_OP_VARIANCE = 50
};

/* Node kinds; numbering is the ordinal of ops.NodeKind (expr.zig:137-149). */
enum {
    TZH_NODE_TENSOR = 0, TZH_NODE_CONSTANT = 1, TZH_NODE_UNARY = 2, TZH_NODE_BINARY = 3,
    TZH_NODE_MATMUL = 4, TZH_NODE_REDUCE = 5, TZH_NODE_RESHAPE = 6, TZH_NODE_TRANSPOSE = 7,
    TZH_NODE_SOFTMAX = 8, TZH_NODE_LAYERNORM = 9, TZH_NODE_GATHER = 10
};

/* ------------------------------------------------------------------ */
/* Errors, version, context, memory                                    */
/* ------------------------------------------------------------------ */
const char *tzh_last_error(void);
int tzh_abi_version(void);

typedef struct tzh_ctx tzh_ctx;

/* Create a context on `device`.  `stream` is the hipStream_t to enqueue on;
 * NULL is the device's default stream (the caller keeps ownership).
 * Replaces InferenceContext.init/initWithPool (arctic.zig:436-465) and the
 * allocator argument of executor.eval/evalInto (executor.zig:29-54). */
int tzh_init(int device, void *stream, tzh_ctx **out);
int tzh_destroy(tzh_ctx *ctx);
int tzh_sync(tzh_ctx *ctx);
void *tzh_stream(tzh_ctx *ctx);

/* Diagnostic, no counterpart in the reference: the size of the context's
 * grow-only device scratch (which tzh_matmul_w8a32, tzh_linear_w8 and
 * tzh_eval_into use for their workspaces) and how many device allocations
 * have (re)sized it since tzh_init. */
int tzh_ctx_scratch_info(tzh_ctx *ctx, int64_t *bytes, int64_t *allocs);

int tzh_malloc(tzh_ctx *ctx, size_t bytes, void **dptr);
int tzh_free(tzh_ctx *ctx, void *dptr);
int tzh_memcpy_h2d(tzh_ctx *ctx, void *dst_device, const void *src_host, size_t bytes);
int tzh_memcpy_d2h(tzh_ctx *ctx, void *dst_host, const void *src_device, size_t bytes);

/* ------------------------------------------------------------------ */
/* Lazy expression evaluation (replaces executor.eval/evalInto,        */
/* executor.zig:29-93, for NodeKind tensor/constant/unary/binary/reduce)*/
/* ------------------------------------------------------------------ */

/* One node of an expression DAG in post-order (children before parents,
 * root last).  This is what a comptime walk over an Expr type emits. */
typedef struct {
    int32_t kind;     /* TZH_NODE_* */
    int32_t op;       /* TZH_OP_* for unary / binary / reduce */
    int32_t lhs;      /* index of the input (unary/reduce) or left operand node */
    int32_t rhs;      /* index of the right operand node (binary), else -1 */
    int32_t leaf;     /* TZH_NODE_TENSOR: index into the leaves array */
    int32_t axis;     /* TZH_NODE_REDUCE: reduced axis, or -1 for all axes (ReduceExpr .{}) */
    int32_t keepdims; /* TZH_NODE_REDUCE: keep_dims */
    int32_t ndim;     /* rank of this node's result */
    int64_t shape[TZH_MAX_RANK]; /* result shape (expr.zig ShapeOf) */
    double value;     /* TZH_NODE_CONSTANT: ScalarExpr.value (converted to dtype) */
    int32_t aux;      /* TZH_NODE_LAYERNORM: index of the beta node (gamma is rhs) */
    int32_t pad_;
    int32_t perm[TZH_MAX_RANK]; /* TZH_NODE_TRANSPOSE: output axis i is input axis perm[i] */
} tzh_node;
/* Node fields per kind beyond kind/op/lhs/rhs/shape:
 *   TZH_NODE_SOFTMAX    lhs = input, axis = softmax_axis (expr.zig:665-676)
 *   TZH_NODE_LAYERNORM  lhs = input, rhs = gamma, aux = beta, axis = norm_dims
 *                       (expr.zig:705-747); eps 1e-5 (layernorm.zig:15)
 *   TZH_NODE_TRANSPOSE  lhs = input, perm (expr.zig:925-972)
 *   TZH_NODE_RESHAPE    lhs = input (same element count, contiguous data)
 *   TZH_NODE_MATMUL     lhs, rhs (executor.zig:199-326)
 *   TZH_NODE_GATHER     lhs = table [vocab, embed], rhs = an integer index leaf;
 *                       result shape = indices shape ++ [embed] (expr.zig:775-830).
 *                       A row whose index is outside [0, vocab) is NaN (the
 *                       reference panics in safe builds, gather.zig:17-21). */

/* A leaf tensor: contiguous row-major device data (Tensor.data, tensor.zig:28-60). */
typedef struct {
    const void *data; /* device pointer */
    int32_t ndim;
    int32_t dtype;    /* 0 or the expression's element type (TZH_F32 / TZH_F64): a value tensor;
                         TZH_I32, TZH_U32, TZH_I64 or TZH_U64: the integer indices of a gather
                         node (Tensor(u32, ...), executor.zig:425-477); anything else is
                         TZH_ERR_WRONG_DTYPE */
    int64_t shape[TZH_MAX_RANK];
} tzh_leaf;

/* Evaluate the DAG rooted at tape[n_nodes-1] into `out` (device, numel of
 * the root shape elements of `dtype`).  dtype is TZH_F32 or TZH_F64 (the
 * element type shared by every node, expr.zig:358-364).  Elementwise chains
 * are evaluated in a single pass without temporaries; a reduce node fuses
 * the chain below it into its reduction.  Broadcasting follows NumPy rules
 * (shape.zig:168-204, strides.zig:92-121). */
/* Node kinds evaluated: tensor, constant, unary, binary, reduce, and
 * matmul, softmax, layernorm, transpose, reshape, gather
 * (executor.zig:199-535), which are computed into a temporary when another
 * node reads them.  Matmul follows numpy's rules: a 1-D lhs is a row and a
 * 1-D rhs a column whose unit dimension the result drops; batch dimensions
 * broadcast (at most 65 535 batches). */
int tzh_eval_into(tzh_ctx *ctx, const tzh_node *tape, int32_t n_nodes,
                  const tzh_leaf *leaves, int32_t n_leaves, int32_t dtype, void *out);

/* ------------------------------------------------------------------ */
/* Kernel-level entry points                                           */
/* ------------------------------------------------------------------ */

/* c[i,j] = (sum_k a[i,k]*f32(wq[j,k])) * f32(scale[j]) + bias[j]
 * Replaces matmulTransposeB_f32_i8_rowScale_bias (matmul_w8a32.zig:14-57).
 * a f32 [m,k], wq i8 [n,k] row-major, scale f16 bits [n], bias f32 [n] (may be
 * NULL = zeros), c f32 [m,n]; all device pointers; any m, k, n >= 0 (k and n
 * are padded with zero codes internally, as the tail loop of
 * matmul_w8a32.zig:50-52 adds the last k % 8 products).  As in the
 * reference, m == 0 or n == 0 does nothing (matmul_w8a32.zig:24) and k == 0
 * writes c[i,j] = bias[j] (0 without a bias).  f32 arithmetic over the
 * whole f32 range: each row of a is scaled by an exact power of two 2^e
 * that puts its largest magnitude in [2^14, 2^15), each product a*q is
 * formed on the MFMA from an exact f16 split of the scaled value (hi + lo,
 * to 2^-22 relative for every value within 2^17 of its row's largest), the
 * sums run in f32 and are multiplied by 2^-e (exact) before the scale and
 * bias.  Rows holding inf or NaN give NaN where the reference gives inf or
 * NaN.  The int8 codes are rewritten into the kernel's tiled format in the
 * context scratch on every call (with the row exponents, and a copy of a
 * with zero columns when k % 64 != 0). */
int tzh_matmul_w8a32(tzh_ctx *ctx, const float *a, const int8_t *wq, const uint16_t *scale,
                     const float *bias, float *c, int64_t m, int64_t k, int64_t n);

/* tzh_matmul_w8a32 without any device allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as tzh_matmul_w8a32, but the tiled codes,
 * the row exponents (and zero-padded rows of a when k % 64 != 0 or a is not
 * 16-byte aligned) go to a static 32 MiB device workspace, one per GPU, held
 * until the process ends: n_pad * k_pad + m * 4 (+ m * k_pad * 4) bytes,
 * each rounded up to 256, must fit (n_pad, k_pad: n and k rounded up to 384
 * and 64), else TZH_ERR_TOO_LARGE.  Calls that overlap on one GPU (other
 * streams or threads) share that workspace and race. */
int tzh_matmul_w8a32_noalloc(tzh_ctx *ctx, const float *a, const int8_t *wq, const uint16_t *scale,
                             const float *bias, float *c, int64_t m, int64_t k, int64_t n);

/* ONNX Gemm (onnx/executor.zig:4561-4634) on the matrix cores: y[m,n] =
 * alpha * op(A) op(B) + beta * C with op = transpose when trans_a / trans_b;
 * A is stored [m,k] (or [k,m] when trans_a) with row pitch lda, B [k,n] (or
 * [n,k]) with pitch ldb (the reference's a.shape[1] / b.shape[1]); C is NULL
 * or [c_rows, c_cols] with c_rows in {1, m} and c_cols in {1, n},
 * broadcast to [m,n]; y is contiguous [m,n].  Device pointers.  Products are
 * exact f32 (v_mfma_f32_16x16x4_f32), sums f32 in another order than the
 * reference's. */
int tzh_gemm_f32(tzh_ctx *ctx, int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k, float alpha,
                 const float *a, int64_t lda, const float *b, int64_t ldb, float beta, const float *c,
                 int64_t c_rows, int64_t c_cols, float *y);

/* ONNX MatMul (onnx/executor.zig:1489-1990), F32 or F64, on the matrix
 * cores: NumPy matmul of contiguous A [..., m, k] and B [..., k, n] with
 * broadcast batch dimensions; a 1-D A is a row and a 1-D B a column whose
 * unit dimension the result drops; B of shape [] or [1] scales A
 * elementwise (executor.zig:1545-1577); k == 0 gives zeros, any other zero
 * dimension an empty result.  Writes the result's shape to y_shape (host,
 * room for TZH_MAX_RANK) and *y_ndim, and the result to y (contiguous)
 * unless y is NULL (a shape query). */
int tzh_matmul_nd(tzh_ctx *ctx, int32_t dtype, const void *a, const int64_t *a_shape, int32_t a_ndim,
                  const void *b, const int64_t *b_shape, int32_t b_ndim, void *y, int64_t *y_shape,
                  int32_t *y_ndim);

/* Epilogues for tzh_linear_w8. */
enum {
    TZH_EPI_BIAS = 0,          /* y = acc*s + b                         (arctic.zig:622-633) */
    TZH_EPI_BIAS_GELU = 1,     /* y = gelu(acc*s + b)                   (arctic.zig:771-776) */
    TZH_EPI_BIAS_RES_LN = 2    /* y = LN(res + (acc*s + b)), N == 384   (arctic.zig:716-746, 779-809) */
};

/* General int8-weight linear with fused epilogue.  a_dtype and c_dtype are
 * TZH_F32 or TZH_F16; residual (EPI_BIAS_RES_LN only) has res_dtype ==
 * c_dtype and shape [m,n]; gamma/beta f32 [n].  f32 activations take the
 * row-scaled hi/lo split of tzh_matmul_w8a32 (f32 arithmetic over the whole
 * f32 range), f16 ones one MFMA; accumulation is f32.  Any k >= 1 (k == 0
 * only with the f32 bias epilogue, c = bias); m == 0 or n == 0 does
 * nothing; f16 output needs n % 384 == 0, the LayerNorm epilogue n == 384. */
int tzh_linear_w8(tzh_ctx *ctx, const void *a, int32_t a_dtype, const int8_t *wq,
                  const uint16_t *scale, const float *bias, void *c, int32_t c_dtype,
                  int64_t m, int64_t k, int64_t n, int32_t epilogue,
                  const void *residual, int32_t res_dtype, const float *gamma,
                  const float *beta, float eps);

/* y = ((x-mean)*inv_std)*gamma + beta over the last dim, two-pass mean /
 * biased variance, inv_std = 1/sqrt(var+eps).  Replaces layerNormLastDim
 * (layernorm.zig:26-117).  x, y f32 [rows, n] (may alias). */
int tzh_layernorm_last_dim(tzh_ctx *ctx, const float *x, const float *gamma, const float *beta,
                           float *y, int64_t rows, int64_t n, float eps);

/* Multi-head self-attention core of selfAttention (arctic.zig:660-713) over
 * packed variable-length sequences: for every sequence b (tokens
 * cu_seqlens[b] .. cu_seqlens[b+1]) and head h, softmax(Q_h K_h^T /
 * sqrt(32)) V_h.  qkv: device [T, 3*hidden] (Q | K | V columns), out: device
 * [T, hidden], both of element type dtype (TZH_F32: products of f32
 * operands formed from exact f16 hi/lo splits, f32 sums; TZH_F16: f16
 * operands), cu_seqlens: device int32 [batch+1].  head_dim must be 32 and
 * sequences at most 512 tokens.  The f32 kernel takes (sequence, head)
 * items from a work queue held by the context (two counters, allocated and
 * zeroed at the first call, back at zero after every launch); calls on one
 * context are ordered by its stream, so they never share it. */
int tzh_attention_varlen(tzh_ctx *ctx, const void *qkv, void *out, int32_t dtype, const int32_t *cu_seqlens,
                         int32_t batch, int32_t n_heads, int32_t hidden);

/* Per-row symmetric int8 quantization with f16 scale, bit-exact to
 * quantize_arctic_xs.zig:94-115.  Device pointers: w f32 [rows,cols],
 * q i8 [rows,cols], scale f16 bits [rows]. */
int tzh_quantize_rows(tzh_ctx *ctx, const float *w, int64_t rows, int64_t cols,
                      int8_t *q, uint16_t *scale);

/* Host-side version of the same quantizer (host pointers, no device work). */
int tzh_quantize_rows_host(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *scale);

/* The quantize_arctic_xs tool (quantize_arctic_xs.zig:42-145, written at 139): read a
 * safetensors file, quantize every tensor shouldQuantize() selects
 * (quantize_arctic_xs.zig:22-34), write I8 `<name>` + F16 `<name>.scale`,
 * copy the rest.  If n_quantized is not NULL it receives the count. */
int tzh_quantize_safetensors(const char *in_path, const char *out_path, int32_t *n_quantized);

/* ------------------------------------------------------------------ */
/* Arctic-embed-xs model (replaces arctic.zig ModelWeights / forward*) */
/* ------------------------------------------------------------------ */

/* arctic.Config (arctic.zig:29-42). */
typedef struct {
    int32_t hidden_size;             /* 384 */
    int32_t num_hidden_layers;       /* 6 */
    int32_t num_attention_heads;     /* 12 */
    int32_t intermediate_size;       /* 1536 */
    int32_t vocab_size;              /* 30522 */
    int32_t max_position_embeddings; /* 512 */
    int32_t type_vocab_size;         /* 2 */
    float layer_norm_eps;            /* 1e-12 */
} tzh_arctic_config;

/* One weight matrix, arctic.MatWeight (arctic.zig:47-58): either F32 data or
 * I8 data [rows, cols] row-major with F16 per-row scale. Host pointers. */
typedef struct {
    const void *data;
    const uint16_t *scale; /* F16 bits [rows] when dtype == TZH_I8, else NULL */
    int32_t dtype;         /* TZH_F32 or TZH_I8 */
    int32_t rows;
    int32_t cols;
    int32_t pad_;
} tzh_mat_view;

/* arctic.AttentionWeights (arctic.zig:70-81). Host pointers. */
typedef struct {
    tzh_mat_view query_weight;  const float *query_bias;
    tzh_mat_view key_weight;    const float *key_bias;
    tzh_mat_view value_weight;  const float *value_bias;
    tzh_mat_view output_weight; const float *output_bias;
    const float *output_ln_gamma;
    const float *output_ln_beta;
} tzh_attention_weights;

/* arctic.FeedForwardWeights (arctic.zig:84-91). Host pointers. */
typedef struct {
    tzh_mat_view intermediate_weight; const float *intermediate_bias;
    tzh_mat_view output_weight;       const float *output_bias;
    const float *output_ln_gamma;
    const float *output_ln_beta;
} tzh_ffn_weights;

typedef struct {
    tzh_attention_weights attention;
    tzh_ffn_weights ffn;
} tzh_layer_weights;

/* arctic.ModelWeights (arctic.zig:100-108) as host views. */
typedef struct {
    tzh_arctic_config config;
    tzh_mat_view word_embeddings;       /* [vocab, hidden] */
    tzh_mat_view position_embeddings;   /* [max_pos, hidden] */
    tzh_mat_view token_type_embeddings; /* [type_vocab, hidden] */
    const float *layer_norm_gamma;
    const float *layer_norm_beta;
    const tzh_layer_weights *layers;    /* [num_hidden_layers] */
} tzh_arctic_weights;

typedef struct tzh_model tzh_model;

/* Upload host weights to HBM (MatWeight, arctic.zig:55-58; ModelWeights,
 * arctic.zig:100).  Encoder linears are I8 + F16 scale (MatWeight.q8) or
 * F32 (MatWeight.f32); other
 * dtypes give TZH_ERR_UNSUPPORTED_DTYPE.  On the device int8 codes stay
 * one byte each (biased, u = q + 128, tiled in the GEMM's stage order) with
 * their f16 row scale; f32 linears stay f32 (computed exactly in f32 on the
 * matrix cores), each linear in its own format; a QKV whose three parts
 * differ in dtype is held as one f32 matrix (int8 parts widened exactly to
 * q * s).  Embedding tables may be F32 or I8.  The upload also bounds every
 * activation the f32 forward splits into f16 halves, from the weights alone
 * (LayerNorm outputs by sqrt(383) max|gamma| + max|beta|, each linear by
 * its rows' sum |W| and |bias|): int8 GEMMs whose input bound reaches 2^15
 * then run row-scaled (as tzh_matmul_w8a32), and a forward whose attention
 * inputs' bound reaches 2^15 returns TZH_ERR_TOO_LARGE instead of computing
 * NaN.  The model is bound to ctx's device and stream. */
int tzh_arctic_upload(tzh_ctx *ctx, const tzh_arctic_weights *weights, tzh_model **out);

/* ModelWeights.fromSafeTensors (arctic.zig:113-166): "bert." prefix
 * optional, LayerNorm weight|gamma and bias|beta, I8 weights need an F16
 * "<name>.scale".  Errors: TZH_ERR_MISSING_WEIGHT, TZH_ERR_WRONG_DTYPE,
 * TZH_ERR_UNSUPPORTED_DTYPE, TZH_ERR_INVALID_FORMAT, TZH_ERR_IO. */
int tzh_arctic_load_safetensors(tzh_ctx *ctx, const char *path, const tzh_arctic_config *config,
                                tzh_model **out);
int tzh_arctic_free(tzh_model *model);

/* Batched forward: arctic.forwardBatch / forwardBatchParallel
 * (arctic.zig:902-918, 959-1013).  Sequence b has lengths[b] tokens
 * (host int32 array, 1..max_position_embeddings) whose ids are at
 * ids + b*ids_stride (device u32; ids_stride == 0 means the sequences are
 * packed back to back).  Each sequence is forwarded at its own length, the
 * reference's semantics for a padded+masked batch.  outputs: device f32
 * [batch, hidden], each row the L2-normalised CLS embedding. */
int tzh_arctic_forward_batch(tzh_model *model, float *outputs, const uint32_t *ids,
                             const int32_t *lengths, int32_t batch, int64_t ids_stride);

/* Hidden state after the embeddings and the first n_layers encoder layers
 * (arctic.zig:830-848 stopped early; n_layers == 0 gives the embedding
 * LayerNorm output), for every token of the packed batch: hidden device f32
 * [sum(lengths), hidden_size].  Same batch arguments as
 * tzh_arctic_forward_batch. */
int tzh_arctic_hidden(tzh_model *model, float *hidden, const uint32_t *ids, const int32_t *lengths,
                      int32_t batch, int64_t ids_stride, int32_t n_layers);

/* Single sequence (arctic.forward, arctic.zig:874-898): ids device u32 [seq_len]. */
int tzh_arctic_forward(tzh_model *model, float *output, const uint32_t *token_ids, int64_t seq_len);

/* One sequence of a ragged host batch: a Zig `[]const u32` as an extern struct. */
typedef struct {
    const uint32_t *ids;
    uint64_t len;
} tzh_ids_slice;

/* The reference's host-memory entry points, same argument shapes:
 * arctic.forwardBatch / forwardBatchParallel (arctic.zig:902-918, 959-1013:
 * outputs []f32 [batch * hidden], token_ids_batch []const []const u32) and
 * arctic.forward (arctic.zig:874-898: output []f32 [hidden], token_ids
 * []const u32).  Host pointers: the ids are packed into pinned staging and
 * uploaded with one copy; the call returns when the embeddings are in
 * `outputs`.  The reference's InferenceContext / BatchContextPool / thread
 * pool arguments have no counterpart: the model's context and stream do
 * their work. */
int tzh_arctic_forward_batch_host(tzh_model *model, float *outputs, const tzh_ids_slice *batch, int32_t batch_n);
int tzh_arctic_forward_host(tzh_model *model, float *output, const uint32_t *token_ids, int64_t seq_len);

/* Number of out-of-range token ids (>= vocab_size) seen since the model was
 * created.  Such ids are clamped to vocab_size-1 so the gather stays in
 * bounds (the reference panics on the slice bounds check in safe builds).
 * Synchronises the model's stream. */
int tzh_arctic_bad_id_count(tzh_model *model, int32_t *count);

/* Last-batch timing hook: number of kernel launches the previous
 * tzh_arctic_forward_batch enqueued (for launch-overhead accounting). */
int tzh_arctic_last_launch_count(tzh_model *model);

/* Activation precision of the forward (no counterpart in the reference,
 * whose activations are always f32): TZH_F32 (the default: f32 activations
 * in HBM, products of f32 operands from exact f16 hi/lo splits, f32 sums, as
 * arctic.zig:599-635 computes) or TZH_F16 (opt-in: activations rounded to
 * f16 between kernels, half the activation traffic).  A model whose linears
 * hold f32 weights (MatWeight.f32), or mixes f32 and int8 linears, runs in
 * f32 whatever is set: each linear on its own format's GEMM (f32 weights on
 * the f32 GEMM of tzh_gemm_f32, int8 weights on the int8 GEMM), as the
 * reference loads each MatWeight independently (arctic.zig:55-58, 258-287).
 * tzh_arctic_precision reports the precision the next forward uses. */
int tzh_arctic_set_precision(tzh_model *model, int32_t dtype);
int tzh_arctic_precision(tzh_model *model, int32_t *dtype);

/* The feed-forward block of one encoder layer (replaces feedForward,
 * arctic.zig:760-811): output = LayerNorm(input + (GELU(input W1^T s1 + b1)
 * W2^T s2 + b2)) with the layer's intermediate and output linears and its
 * output LayerNorm, for device f32 input and output [seq_len, hidden]
 * (16-byte aligned, not overlapping; layer in [0, num_hidden_layers)),
 * in f32 whatever tzh_arctic_set_precision chose, enqueued on the model's
 * stream.  A layer whose two linears are int8 runs it as one kernel, the
 * 1536-wide intermediate kept on chip (its last, partial round of 64-token
 * panels split by chunks over the idle CUs and finished by a second, small
 * kernel), unless the model's weights call for row scaling; other layers
 * run the GEMM pair. */
int tzh_arctic_feed_forward(tzh_model *model, int32_t layer, const float *input, float *output, int64_t seq_len);

/* Fused feed-forward switch (no counterpart in the reference): enable = 0
 * makes the forward and tzh_arctic_feed_forward run every feed-forward block
 * as the GEMM pair (GELU epilogue, then residual + LayerNorm epilogue), and
 * the forward every O-projection and QKV projection on the int8 GEMM, even
 * where the fused kernel applies; nonzero (the default) restores them.  They agree to the f32
 * rounding of their different summation orders. */
int tzh_arctic_set_ffn_fusion(tzh_model *model, int32_t enable);

/* Launch tracing (no counterpart in the reference, whose CPU path has no
 * kernels to time): with timing enabled (enable = n >= 1), every later
 * forward records a HIP event on the model's stream before its first and
 * after each of its stages, and issues each stage after pack_ids n times
 * back to back between its events (every such stage reads only buffers it
 * does not write, so the result is unchanged), which spreads the cost of
 * an event over n launches.  enable = 0 turns it off; n <= 1000. */
int tzh_arctic_set_timing(tzh_model *model, int32_t enable);

/* Per-launch durations of the most recent timed forward, in launch order:
 * us[i] (microseconds between the events around stage i, divided by the
 * times it was issued) and names[i]
 * (static stage names: "pack_ids", "embed_ln", "qkv", "attention",
 * "attn_out_ln" and "ffn" (the fused feed-forward kernel), or "attn_ffn"
 * (the O-projection, its LayerNorm and the feed-forward block as one
 * kernel; both fused stages include the kernel that finishes the rows of a
 * split last round), or "attn_out_ln", "ffn1_gelu" and "ffn2_ln" (the GEMM pair),
 * "cls_l2", "hidden_f32"), at most
 * `capacity` entries; *count = number of launches (0 if the last forward was
 * not timed).  Waits for that forward to finish.  Either array may be NULL. */
int tzh_arctic_launch_times(tzh_model *model, float *us, const char **names, int32_t capacity, int32_t *count);

/* ------------------------------------------------------------------ */
/* The .tenzor file format (io/tenzor_format.zig)                      */
/* ------------------------------------------------------------------ */

/* tenzor_format.DType (tenzor_format.zig:25-37). */
enum {
    TZH_TZ_F32 = 0, TZH_TZ_F16 = 1, TZH_TZ_BF16 = 2, TZH_TZ_F64 = 3, TZH_TZ_I8 = 4, TZH_TZ_I16 = 5,
    TZH_TZ_I32 = 6, TZH_TZ_I64 = 7, TZH_TZ_U8 = 8, TZH_TZ_U16 = 9, TZH_TZ_U32 = 10, TZH_TZ_U64 = 11
};

/* tenzor_format.TensorEntry (tenzor_format.zig:83-104), the 48-byte index
 * entry exactly as stored in the file. */
typedef struct {
    uint64_t name_hash; /* FNV-1a of the tensor name */
    uint8_t dtype;      /* TZH_TZ_* */
    uint8_t ndim;
    uint8_t pad_[2];
    uint32_t shape[5];
    uint64_t data_offset; /* from the start of the data section */
    uint64_t data_size;   /* bytes */
} tzh_tenzor_entry;

typedef struct tzh_tenzor_file tzh_tenzor_file;

/* hashName (tenzor_format.zig:107-114): 64-bit FNV-1a. */
uint64_t tzh_tenzor_name_hash(const char *name, int64_t len);

/* TenzorFile.open / close (tenzor_format.zig:140-204): maps the file
 * read-only.  Bad magic, version or section bounds give
 * TZH_ERR_INVALID_FORMAT (the reference's InvalidMagic, UnsupportedVersion,
 * InvalidFormat); open or mmap failures TZH_ERR_IO.  Unlike the reference,
 * every section and tensor is checked to lie inside the file. */
int tzh_tenzor_open(const char *path, tzh_tenzor_file **out);
int tzh_tenzor_close(tzh_tenzor_file *file);

/* Header fields and the metadata JSON (a pointer into the mapping, not
 * NUL-terminated).  Any output may be NULL. */
int tzh_tenzor_info(const tzh_tenzor_file *file, uint32_t *tensor_count, const char **metadata_json,
                    int64_t *metadata_size);

/* TenzorFile.getTensor + getData (tenzor_format.zig:208-237): the first
 * entry whose hash is the name's, and a host pointer to its bytes inside
 * the mapping (valid until close).  TZH_ERR_MISSING_WEIGHT if absent. */
int tzh_tenzor_get(const tzh_tenzor_file *file, const char *name, tzh_tenzor_entry *entry, const void **data);

/* convertFromSafetensors (tenzor_format.zig:440-484, the `convert`
 * command of main.zig:1028-1045): every tensor in header order, BOOL
 * stored as u8, metadata "{}"; the file is byte-identical to the
 * reference writer's. */
int tzh_tenzor_convert_safetensors(const char *safetensors_path, const char *tenzor_path);

/* ModelWeights from a .tenzor file: the names, dtypes and errors of
 * tzh_arctic_load_safetensors (arctic.zig:113-166), with tensors read
 * straight from the mapping. */
int tzh_arctic_load_tenzor(tzh_ctx *ctx, const char *path, const tzh_arctic_config *config, tzh_model **out);

/* ------------------------------------------------------------------ */
/* WordPiece tokenizer and the embed command's text paths              */
/* ------------------------------------------------------------------ */

/* io/tokenizer.Tokenizer (tokenizer.zig:9-15): vocabulary map, [UNK] 100,
 * [CLS] 101, [SEP] 102, words over 200 bytes give [UNK].  Host object;
 * encoding is read-only, so one tokenizer may serve several threads. */
typedef struct tzh_tokenizer tzh_tokenizer;

/* Tokenizer.init / deinit (tokenizer.zig:17-31); the vocabulary starts empty. */
int tzh_tokenizer_create(tzh_tokenizer **out);
int tzh_tokenizer_free(tzh_tokenizer *tok);

/* Tokenizer.loadVocab / loadVocabFromBytes (tokenizer.zig:34-74): one token
 * per line, its id the line index (empty lines count, a trailing '\r' is
 * stripped, a repeated token takes the later index).  TZH_ERR_IO when the
 * file cannot be read. */
int tzh_tokenizer_load_vocab(tzh_tokenizer *tok, const char *path);
int tzh_tokenizer_load_vocab_bytes(tzh_tokenizer *tok, const char *data, int64_t len);

/* vocab.put(token, id), as the reference's tokenizer tests build their
 * vocabularies (tokenizer.zig:291-437). */
int tzh_tokenizer_put(tzh_tokenizer *tok, const char *token, int64_t len, uint32_t id);

/* Tokenizer.encode (tokenizer.zig:78-118): [CLS] pieces [SEP] into
 * out[0, capacity) (host), capacity >= 2 (else TZH_ERR_INVALID_ARGS, the
 * reference's assert); pieces stop at capacity - 1, inside a word too.
 * *n = number of ids written. */
int tzh_tokenizer_encode(const tzh_tokenizer *tok, const char *text, int64_t len, uint32_t *out,
                         int64_t capacity, int64_t *n);

/* Tokenizer.encodeRaw (tokenizer.zig:122-151): the pieces of the whole
 * text, no markers.  *n = number of pieces; TZH_ERR_TOO_LARGE (nothing
 * written) when that exceeds capacity, so out = NULL, capacity = 0 asks
 * for the size. */
int tzh_tokenizer_encode_raw(const tzh_tokenizer *tok, const char *text, int64_t len, uint32_t *out,
                             int64_t capacity, int64_t *n);

/* Number of chunks runEmbed cuts a document of total_tokens pieces into
 * (main.zig:803-806): 510-piece chunks every 460 pieces,
 * 1 + (total - 461) / 460 of them above 510 pieces.  A tail of up to 410
 * pieces past the last chunk is not embedded, as in the reference. */
int tzh_embed_chunk_count(int64_t total_tokens, int64_t *count);

/* runEmbed's document path (main.zig:786-933) for n_docs documents at
 * once: each text (host bytes texts[d], lens[d]) is encodeRaw'd, cut into
 * chunks [CLS] + pieces[460k, min(460k + 510, total)) + [SEP], and all
 * chunks of all documents go through one batched forward; each document's
 * chunk embeddings are then averaged (in chunk order, times 1/chunks) and
 * L2-normalised (sequential sum of squares, divided by the norm when it is
 * positive).  outputs: device f32 [n_docs, hidden].  chunk_counts (host,
 * may be NULL) receives each document's chunk count.  A document of
 * 511..920 pieces is TZH_ERR_TOO_LARGE: the reference copies such a
 * document into one 512-id chunk buffer (main.zig:903-906), past its end.
 * Returns once the ids are on the device; the forward and the pooling run
 * on the model's stream. */
int tzh_arctic_embed_documents(tzh_model *model, const tzh_tokenizer *tok, const char *const *texts,
                               const int64_t *lens, int32_t n_docs, float *outputs, int32_t *chunk_counts);

/* runEmbed's positional-text path (main.zig:935-1019): each text is
 * encode'd into 512 ids ([CLS] ... [SEP], cut at 511) and the texts go
 * through one batched forward.  outputs: device f32 [n_texts, hidden];
 * n_tokens (host, may be NULL) receives each text's id count. */
int tzh_arctic_embed_texts(tzh_model *model, const tzh_tokenizer *tok, const char *const *texts,
                           const int64_t *lens, int32_t n_texts, float *outputs, int32_t *n_tokens);

#ifdef __cplusplus
}
#endif

#endif /* TENZOR_HIP_H */
