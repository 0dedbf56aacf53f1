/*
 * oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of mattneel/tenzor's hot path (the int8-weight
 * Arctic-embed-xs forward and the lazy elementwise/reduce executor), used as
 * the parity checker for the HIP backend and as the CPU baseline ("port") in
 * bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Pinning of each
 * function (known answers, closed forms, independent libraries) lives in
 * tests/test_oracle_pins.py.
 */
#ifndef TZH_ORACLE_H
#define TZH_ORACLE_H

#include <stdint.h>
#include "../include/tenzor_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* f32 <-> f16 bit conversions (Zig @floatCast, round-to-nearest-even). */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);

/* quantize_arctic_xs.zig:94-115 */
void orc_quantize_rows(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *scale);

/* matmul_w8a32.zig:14-57 */
void orc_matmul_w8a32(const float *a, const int8_t *wq, const uint16_t *scale, const float *bias,
                      float *c, int64_t m, int64_t k, int64_t n);

/* arctic.zig:609-621 (f32 MatWeight: matmulTransposeB then += bias) */
void orc_linear_f32(const float *a, const float *w, const float *bias, float *c,
                    int64_t m, int64_t k, int64_t n);

/* layernorm.zig:26-117 */
void orc_layernorm(const float *x, const float *gamma, const float *beta, float *y,
                   int64_t rows, int64_t n, float eps);

/* arctic.zig:750-756 */
float orc_gelu(float x);

/* arctic.zig:851-863 */
void orc_l2_normalize(float *v, int64_t n);

/* arctic.zig:660-713, one head: q,k,v are [L, ld] with the head's 32 columns
 * starting at column 0 of each row; out likewise. scores: [L*L] scratch. */
void orc_attention_head(const float *q, const float *k, const float *v, float *out,
                        int64_t L, int64_t ld, int64_t head_dim, float *scores);

/* arctic.zig:543-585 */
void orc_embeddings(float *out, const uint32_t *ids, int64_t L, const tzh_arctic_weights *w);

/* arctic.zig:874-898.  Returns 0 or -1 (bad arguments). */
int orc_arctic_forward(const tzh_arctic_weights *w, const uint32_t *ids, int64_t L, float *out);

/* arctic.zig:874-898 but stops after `n_layers_run` encoder layers and
 * writes the full hidden state [L, hidden] (no CLS/L2) — layer-wise parity. */
int orc_arctic_hidden(const tzh_arctic_weights *w, const uint32_t *ids, int64_t L,
                      int32_t n_layers_run, float *hidden_out);

/* arctic.zig:959-1013: sequence b is ids[offsets[b] .. offsets[b]+lengths[b]);
 * threads split the batch into contiguous ranges (threading.zig:127-177). */
int orc_arctic_forward_batch(const tzh_arctic_weights *w, const uint32_t *ids,
                             const int64_t *offsets, const int32_t *lengths, int32_t batch,
                             float *out, int32_t nthreads);

/* executor.zig:29-196, 327-360 + elementwise.zig + simd.zig + reduce.zig:
 * evaluates the DAG with one materialised temporary per non-leaf node, as the
 * reference executor does.  Leaves hold HOST pointers here.  Returns 0 or a
 * TZH_ERR_* code. */
int orc_eval(const tzh_node *tape, int32_t n_nodes, const tzh_leaf *leaves, int32_t n_leaves,
             int32_t dtype, void *out);

/* Scalar op semantics (simd.zig:118-315), exposed for pin tests. */
float orc_unary_f32(int32_t op, float x);
float orc_binary_f32(int32_t op, float a, float b);
double orc_unary_f64(int32_t op, double x);
double orc_binary_f64(int32_t op, double a, double b);

/* Vectorised forms of the scalar semantics above (test helpers). */
void orc_unary_vec_f32(int32_t op, const float *x, float *y, int64_t n);
void orc_binary_vec_f32(int32_t op, const float *a, const float *b, float *y, int64_t n);
void orc_gelu_vec(const float *x, float *y, int64_t n);

/* config-2 chain exp((a + b[j]) * c) over rows x cols, the result of
 * executor.evalInto on BinaryExpr(.add,A,B).mul(c).exp(): three passes with
 * two temporaries (executor.zig:551-578).  tmp1/tmp2 are caller scratch of
 * rows*cols floats. */
void orc_chain_add_mul_exp(const float *a, const float *b_row, const float *c, float *out,
                           int64_t rows, int64_t cols, float *tmp1, float *tmp2);

#ifdef __cplusplus
}
#endif

#endif
