// K1: single-pass elementwise / broadcast / reduce chains for tzh_eval_into.
//
// Replaces executor.evalInto (executor.zig:49-196, 327-360), which
// materialises one temporary per non-leaf child (executor.zig:551-578).
// Here a post-order expression DAG becomes a small stack program that every
// thread runs over VEC contiguous output elements, reading each leaf once
// through its broadcast projection and writing the result once.  A reduce
// node evaluates the chain below it inside the reduction (no temporary);
// only a reduce that feeds further elementwise work is materialised.
//
// Op semantics follow simd.zig:107-315 (tanh = 2*sigmoid(2x)-1, gelu with
// that tanh, relu = @max(x,0), round half away from zero) and
// elementwise.zig:124-207 (supported op set).
#include "ew_program.h"

#include <cmath>
#include <cstring>
#include <type_traits>
#include <vector>

namespace tzh_ew {

FastDiv make_fastdiv(uint64_t d) {
    FastDiv f{};
    if (d == 0 || d > 0xffffffffull) return FastDiv{0, 0, 0, 0};  // unused: 64-bit path
    int l = 0;
    while ((1ull << l) < d) l++;
    f.d = (uint32_t)d;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    f.s1 = l > 0 ? 1 : 0;
    f.s2 = l > 0 ? (uint32_t)(l - 1) : 0;
    return f;
}

}  // namespace tzh_ew

namespace {

using namespace tzh_ew;

// Chains run as generated kernels (ew_jit.cpp) unless the context asks for
// the interpreter.
constexpr bool kHaveJit = true;

template <typename T, int V>
struct Vec {
    T v[V];
};

// scalar op semantics (simd.zig:107-315): ew_shared.inc
// ------------------------------------------------------------------------
// leaf loads
// ------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ int64_t leaf_offset(const EwLeaf &lf, const EwProgram &p, int64_t flat) {
    if (p.small) {
        const uint32_t f = (uint32_t)flat;
        if (!lf.general) {
            const uint32_t q = lf.div == 1 ? f : fast_div(lf.fdiv, f);
            return lf.mod > (int64_t)0xffffffff ? q : q - fast_div(lf.fmod, q) * lf.fmod.d;
        }
        uint32_t off = 0, rem = f;
        for (int d = p.ndim - 1; d >= 0; d--) {
            const uint32_t q = fast_div(p.fshape[d], rem);
            off += (rem - q * p.fshape[d].d) * (uint32_t)lf.strides[d];
            rem = q;
        }
        return off;
    }
    if (!lf.general) return (flat / lf.div) % lf.mod;
    int64_t off = 0, rem = flat;
    for (int d = p.ndim - 1; d >= 0; d--) {
        const int64_t ix = rem % p.shape[d];
        rem /= p.shape[d];
        off += ix * lf.strides[d];
    }
    return off;
}

template <typename T, int V>
__device__ __forceinline__ Vec<T, V> load_leaf(const EwLeaf &lf, const EwProgram &p, int64_t flat) {
    Vec<T, V> r;
    const T *base = (const T *)lf.ptr;
    if (lf.vec == VEC_CONTIG) {
        const int64_t off = leaf_offset<T>(lf, p, flat);
        if constexpr (V * sizeof(T) == 16) {
            const f32x4_t raw = *(const f32x4_t *)(base + off);
            __builtin_memcpy(&r, &raw, 16);
        } else {
#pragma unroll
            for (int e = 0; e < V; e++) r.v[e] = base[off + e];
        }
    } else if (lf.vec == VEC_SPLAT) {
        const T x = base[leaf_offset<T>(lf, p, flat)];
#pragma unroll
        for (int e = 0; e < V; e++) r.v[e] = x;
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) r.v[e] = base[leaf_offset<T>(lf, p, flat + e)];
    }
    return r;
}

// value stack with a uniform stack pointer: four named slots (not an array,
// which the compiler would index dynamically in scratch memory) selected by
// scalar branches on the wave-uniform slot number.
template <typename T, int V>
struct Stack {
    Vec<T, V> s0, s1, s2, s3;
    // element-wise value selects: no slot is ever addressed through a pointer
    __device__ __forceinline__ Vec<T, V> get(int i) const {
        Vec<T, V> r;
#pragma unroll
        for (int e = 0; e < V; e++)
            r.v[e] = i == 0 ? s0.v[e] : i == 1 ? s1.v[e] : i == 2 ? s2.v[e] : s3.v[e];
        return r;
    }
    __device__ __forceinline__ void set(int i, const Vec<T, V> &x) {
#pragma unroll
        for (int e = 0; e < V; e++) {
            s0.v[e] = i == 0 ? x.v[e] : s0.v[e];
            s1.v[e] = i == 1 ? x.v[e] : s1.v[e];
            s2.v[e] = i == 2 ? x.v[e] : s2.v[e];
            s3.v[e] = i == 3 ? x.v[e] : s3.v[e];
        }
    }
};

template <typename T, int V>
__device__ __forceinline__ Vec<T, V> run_program(const EwProgram &p, int64_t flat) {
    Stack<T, V> st;
    for (int i = 0; i < p.n_nodes; i++) {
        const EwNode &nd = p.nodes[i];
        if (nd.kind == EK_LEAF) {
            st.set(nd.slot, load_leaf<T, V>(p.leaves[nd.arg], p, flat));
        } else if (nd.kind == EK_CONST) {
            Vec<T, V> x;
#pragma unroll
            for (int e = 0; e < V; e++) x.v[e] = (T)nd.cval;
            st.set(nd.slot, x);
        } else if (nd.kind == EK_UNARY) {
            Vec<T, V> x = st.get(nd.slot);
#pragma unroll
            for (int e = 0; e < V; e++) x.v[e] = unary_op<T>(nd.op, x.v[e]);
            st.set(nd.slot, x);
        } else {
            Vec<T, V> a = st.get(nd.slot);
            const Vec<T, V> b = st.get(nd.slot + 1);
#pragma unroll
            for (int e = 0; e < V; e++) a.v[e] = binary_op<T>(nd.op, a.v[e], b.v[e]);
            st.set(nd.slot, a);
        }
    }
    return st.get(0);
}

template <typename T, int V>
__global__ void __launch_bounds__(256) ew_chain_kernel(const EwProgram p, T *__restrict__ out) {
    const int64_t nvec = p.numel / V;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
        const int64_t flat = v * V;
        const Vec<T, V> r = run_program<T, V>(p, flat);
        if constexpr (V * sizeof(T) == 16) {
            f32x4_t raw;
            __builtin_memcpy(&raw, &r, 16);
            __builtin_nontemporal_store(raw, (f32x4_t *)(out + flat));
        } else {
#pragma unroll
            for (int e = 0; e < V; e++) out[flat + e] = r.v[e];
        }
    }
    // tail (numel % V elements), one element per thread of block 0
    if (blockIdx.x == 0) {
        const int64_t t = nvec * V + threadIdx.x;
        // with V == 1 every leaf mode loads the single element at its
        // affine or general offset, so the same program serves the tail
        if (t < p.numel) out[t] = run_program<T, 1>(p, t).v[0];
    }
}

// block-wide reduction of one value per thread (256 threads)
template <typename T>
__device__ __forceinline__ T block_reduce(int op, T v, T *smem) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = red_apply<T>(op, v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    if (l == 0) smem[w] = v;
    __syncthreads();
    T r = red_ident<T>(op);
    if (threadIdx.x == 0) {
        for (int i = 0; i < (int)(blockDim.x / 64); i++) r = red_apply<T>(op, r, smem[i]);
    }
    __syncthreads();
    return r;
}

// Reduce-all, stage 1: each block reduces a grid-stride share of the chain.
template <typename T, int V>
__global__ void __launch_bounds__(256) ew_reduce_all_kernel(const EwProgram p, int op,
                                                            T *__restrict__ partials) {
    __shared__ T smem[4];
    T acc = red_ident<T>(op);
    const int64_t nvec = p.numel / V;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
        const Vec<T, V> r = run_program<T, V>(p, v * V);
#pragma unroll
        for (int e = 0; e < V; e++) acc = red_apply<T>(op, acc, r.v[e]);
    }
    if (blockIdx.x == 0) {
        const int64_t t = nvec * V + threadIdx.x;
        if (t < p.numel) acc = red_apply<T>(op, acc, run_program<T, 1>(p, t).v[0]);
    }
    const T r = block_reduce<T>(op, acc, smem);
    if (threadIdx.x == 0) partials[blockIdx.x] = r;
}

// Reduce-all, stage 2: one block folds the partials; mean divides by n.
template <typename T>
__global__ void __launch_bounds__(256) ew_reduce_finish_kernel(const T *__restrict__ partials, int n,
                                                               int op, int64_t count,
                                                               T *__restrict__ out, int64_t out_numel) {
    __shared__ T smem[4];
    T acc = red_ident<T>(op);
    for (int i = threadIdx.x; i < n; i += blockDim.x) acc = red_apply<T>(op, acc, partials[i]);
    T r = block_reduce<T>(op, acc, smem);
    if (threadIdx.x == 0 && op == TZH_OP_MEAN) r = r / (T)count;
    if (threadIdx.x == 0) smem[0] = r;
    __syncthreads();
    r = smem[0];
    for (int64_t i = threadIdx.x; i < out_numel; i += blockDim.x) out[i] = r;
}

// Reduce over the last axis (inner == 1): one wave per output row.
template <typename T>
__global__ void __launch_bounds__(256) ew_reduce_rows_kernel(const EwProgram p, int op, int64_t outer,
                                                             int64_t rsz, T *__restrict__ out) {
    const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (row >= outer) return;
    T acc = red_ident<T>(op);
    for (int64_t r = lane; r < rsz; r += 64) acc = red_apply<T>(op, acc, run_program<T, 1>(p, row * rsz + r).v[0]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc = red_apply<T>(op, acc, __shfl_xor(acc, o, 64));
    if (lane == 0) out[row] = (op == TZH_OP_MEAN) ? acc / (T)rsz : acc;
}

// Reduce over a middle/leading axis: one thread per (outer, inner) column.
template <typename T>
__global__ void __launch_bounds__(256) ew_reduce_cols_kernel(const EwProgram p, int op, int64_t outer,
                                                             int64_t rsz, int64_t inner,
                                                             T *__restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= outer * inner) return;
    const int64_t o = idx / inner, i = idx % inner;
    T acc = red_ident<T>(op);
    for (int64_t r = 0; r < rsz; r++) acc = red_apply<T>(op, acc, run_program<T, 1>(p, (o * rsz + r) * inner + i).v[0]);
    out[idx] = (op == TZH_OP_MEAN) ? acc / (T)rsz : acc;
}

// ------------------------------------------------------------------------
// Softmax, LayerNorm and transpose nodes (executor.zig:363-535).  Their
// inputs are contiguous buffers: leaf tensors or materialised children.
// ------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_max_t(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}
template <typename T>
__device__ __forceinline__ T wave_sum_t(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float exp_t(float x) { return expf(x); }
__device__ __forceinline__ double exp_t(double x) { return exp(x); }
__device__ __forceinline__ float sqrt_t(float x) { return sqrtf(x); }
__device__ __forceinline__ double sqrt_t(double x) { return sqrt(x); }

template <typename T, int V>
struct alignas(sizeof(T) * V) RowVec {
    T v[V];
};

// softmaxRow (softmax.zig:38-137): max, exp(x - max) summed, then
// exp(x - max) * (1 / sum) stored (recomputed rather than stored and
// re-read: the same values, one pass less over memory).  One wave per row
// of the last axis, V consecutive elements per lane and access.
template <typename T, int V>
__global__ void __launch_bounds__(256) ew_softmax_rows_kernel(const T *__restrict__ x, T *__restrict__ y,
                                                              int64_t rows, int64_t n) {
    const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (r >= rows) return;
    const RowVec<T, V> *xr = (const RowVec<T, V> *)(x + r * n);
    RowVec<T, V> *yr = (RowVec<T, V> *)(y + r * n);
    const int64_t nv = n / V;
    T m = -INFINITY;
    for (int64_t c = lane; c < nv; c += 64) {
        const RowVec<T, V> a = xr[c];
#pragma unroll
        for (int k = 0; k < V; k++) m = fmax(m, a.v[k]);
    }
    m = wave_max_t(m);
    T s = 0;
    for (int64_t c = lane; c < nv; c += 64) {
        const RowVec<T, V> a = xr[c];
#pragma unroll
        for (int k = 0; k < V; k++) s += exp_t(a.v[k] - m);
    }
    const T inv = (T)1 / wave_sum_t(s);
    for (int64_t c = lane; c < nv; c += 64) {
        const RowVec<T, V> a = xr[c];
        RowVec<T, V> o;
#pragma unroll
        for (int k = 0; k < V; k++) o.v[k] = exp_t(a.v[k] - m) * inv;
        yr[c] = o;
    }
}

// softmaxAxis general case (softmax.zig:172-213): one thread per
// (outer, inner) column of a middle or leading axis.
template <typename T>
__global__ void __launch_bounds__(256) ew_softmax_cols_kernel(const T *__restrict__ x, T *__restrict__ y,
                                                              int64_t outer, int64_t n, int64_t inner) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= outer * inner) return;
    const int64_t base = (idx / inner) * n * inner + idx % inner;
    T m = -INFINITY;
    for (int64_t a = 0; a < n; a++) m = fmax(m, x[base + a * inner]);
    T s = 0;
    for (int64_t a = 0; a < n; a++) {
        const T e = exp_t(x[base + a * inner] - m);
        y[base + a * inner] = e;
        s += e;
    }
    const T inv = (T)1 / s;
    for (int64_t a = 0; a < n; a++) y[base + a * inner] = y[base + a * inner] * inv;
}

// layerNorm (layernorm.zig:123-185): mean = sum * (1/N), variance = sum of
// squared deviations * (1/N), 1 / sqrt(variance + eps), then
// (x - mean) * inv_std * gamma + beta.  One wave per instance, V
// consecutive elements per lane and access.
template <typename T, int V>
__global__ void __launch_bounds__(256) ew_layernorm_kernel(const T *__restrict__ x, const T *__restrict__ g,
                                                           const T *__restrict__ b, T *__restrict__ y,
                                                           int64_t rows, int64_t n, T eps) {
    const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (r >= rows) return;
    using RV = RowVec<T, V>;
    const RV *xr = (const RV *)(x + r * n);
    RV *yr = (RV *)(y + r * n);
    const int64_t nv = n / V;
    const T inv_n = (T)1 / (T)n;
    T s = 0;
    for (int64_t c = lane; c < nv; c += 64) {
        const RV a = xr[c];
#pragma unroll
        for (int k = 0; k < V; k++) s += a.v[k];
    }
    const T mean = wave_sum_t(s) * inv_n;
    T var = 0;
    for (int64_t c = lane; c < nv; c += 64) {
        const RV a = xr[c];
#pragma unroll
        for (int k = 0; k < V; k++) {
            const T d = a.v[k] - mean;
            var += d * d;
        }
    }
    const T inv_std = (T)1 / sqrt_t(wave_sum_t(var) * inv_n + eps);
    for (int64_t c = lane; c < nv; c += 64) {
        const RV a = xr[c], gg = ((const RV *)g)[c], bb = ((const RV *)b)[c];
        RV o;
#pragma unroll
        for (int k = 0; k < V; k++) o.v[k] = ((a.v[k] - mean) * inv_std) * gg.v[k] + bb.v[k];
        yr[c] = o;
    }
}

// gather (gather.zig:4-39): output row r is table row indices[r]; a row
// whose index lies outside [0, vocab) is NaN.
template <typename T, typename I>
__global__ void __launch_bounds__(256) ew_gather_kernel(const T *__restrict__ table, const I *__restrict__ idx,
                                                        T *__restrict__ y, int64_t vocab, int64_t embed,
                                                        int64_t numel) {
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= numel) return;
    const int64_t row = o / embed, j = o % embed;
    const I k = idx[row];
    bool ok;
    if constexpr (std::is_signed<I>::value) ok = k >= 0 && (int64_t)k < vocab;
    else ok = (uint64_t)k < (uint64_t)vocab;
    y[o] = ok ? table[(int64_t)k * embed + j] : (T)NAN;
}

// matmul (executor.zig:199-326, matmul.zig): C[b] = A[b] B[b] over
// broadcast batch dimensions, computed by the matrix-core GEMM of
// gemm_fp.hip; these are the batch strides and sizes the planner derives.
struct MatmulArgs {
    int32_t nb;  // batch dimensions of the output
    int64_t batch_shape[TZH_MAX_RANK];
    int64_t a_stride[TZH_MAX_RANK], b_stride[TZH_MAX_RANK];  // 0 where broadcast
    int64_t m, k, n;
};

// transpose (transpose.zig): output element o at multi-index i reads the
// input at sum_k i[k] * in_stride[perm[k]].
struct TransposeArgs {
    int32_t ndim;
    int64_t out_shape[TZH_MAX_RANK];
    int64_t src_stride[TZH_MAX_RANK];  // input stride of the axis that output axis k reads
};

// Transposes that move the last axis: 32 x 32 tiles of (output last axis,
// output axis that reads the input's last axis) through LDS, so that both
// the reads and the writes run along a contiguous axis.
struct TileTransposeArgs {
    int32_t nrest;  // output axes other than the two tiled ones
    int64_t rest_shape[TZH_MAX_RANK], rest_src[TZH_MAX_RANK], rest_dst[TZH_MAX_RANK];
    int64_t n_l, n_q;  // extents of the output's last axis and of axis q
    int64_t src_l;     // input stride of the axis the output's last axis reads
    int64_t dst_q;     // output stride of axis q
    int64_t nz;        // product of rest_shape
};

template <typename T>
__global__ void __launch_bounds__(256) ew_transpose_tiled_kernel(const T *__restrict__ x, T *__restrict__ y,
                                                                 const TileTransposeArgs a) {
    __shared__ T tile[32][33];
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;
    const int64_t l0 = (int64_t)blockIdx.x * 32, q0 = (int64_t)blockIdx.y * 32;
    for (int64_t z = blockIdx.z; z < a.nz; z += gridDim.z) {
        int64_t rem = z, sb = 0, db = 0;
        for (int d = a.nrest - 1; d >= 0; d--) {
            const int64_t i = rem % a.rest_shape[d];
            rem /= a.rest_shape[d];
            sb += i * a.rest_src[d];
            db += i * a.rest_dst[d];
        }
        for (int j = ty; j < 32; j += 8) {
            const int64_t l = l0 + j, q = q0 + tx;
            if (l < a.n_l && q < a.n_q) tile[j][tx] = x[sb + l * a.src_l + q];
        }
        __syncthreads();
        for (int j = ty; j < 32; j += 8) {
            const int64_t q = q0 + j, l = l0 + tx;
            if (l < a.n_l && q < a.n_q) y[db + q * a.dst_q + l] = tile[tx][j];
        }
        __syncthreads();
    }
}

template <typename T>
__global__ void __launch_bounds__(256) ew_transpose_kernel(const T *__restrict__ x, T *__restrict__ y,
                                                           const TransposeArgs a, int64_t numel) {
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= numel) return;
    int64_t rem = o, src = 0;
    for (int k = a.ndim - 1; k >= 0; k--) {
        const int64_t i = rem % a.out_shape[k];
        rem /= a.out_shape[k];
        src += i * a.src_stride[k];
    }
    y[o] = x[src];
}

// ------------------------------------------------------------------------
// host planner
// ------------------------------------------------------------------------
using tzh_ew::unary_ok;

bool binary_ok(int op) {
    switch (op) {
    case TZH_OP_ADD: case TZH_OP_SUB: case TZH_OP_MUL: case TZH_OP_DIV: case TZH_OP_POW:
    case TZH_OP_MAX: case TZH_OP_MIN:
        return true;
    default:
        return false;
    }
}

bool reduce_ok(int op) {
    switch (op) {
    case TZH_OP_SUM: case TZH_OP_MEAN: case TZH_OP_PROD: case TZH_OP_REDUCE_MAX:
    case TZH_OP_REDUCE_MIN:
        return true;
    default:
        return false;
    }
}

int64_t numel_of(int32_t nd, const int64_t *s) {
    int64_t n = 1;
    for (int i = 0; i < nd; i++) n *= s[i];
    return n;
}

struct Planner {
    tzh_ctx *ctx;
    const tzh_node *tape;
    int32_t n_nodes;
    const tzh_leaf *leaves;
    int32_t n_leaves;
    int32_t dtype;
    size_t es;
    // Temporaries come from the stream-ordered allocator (hipMallocAsync on
    // the context's stream) and go back to it after the kernels that read
    // them, so an evaluation never waits on the host; where that allocator
    // is unavailable, from hipMalloc, freed after one synchronisation.
    std::vector<void *> temps, sync_temps;
    bool no_async = false;

    ~Planner() {
        for (void *t : temps) hipFreeAsync(t, ctx->stream);
        if (sync_temps.empty()) return;
        hipStreamSynchronize(ctx->stream);
        for (void *t : sync_temps) hipFree(t);
    }

    int temporary(size_t bytes, void **out) {
        void *t = nullptr;
        if (!no_async) {
            if (hipMallocAsync(&t, bytes ? bytes : es, ctx->stream) == hipSuccess) {
                temps.push_back(t);
                *out = t;
                return TZH_OK;
            }
            (void)hipGetLastError();
            no_async = true;
        }
        if (hipMalloc(&t, bytes ? bytes : es) != hipSuccess) {
            (void)hipGetLastError();
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "temporary of %zu bytes failed", bytes);
        }
        sync_temps.push_back(t);
        *out = t;
        return TZH_OK;
    }

    int validate(int32_t idx) {
        if (idx < 0 || idx >= n_nodes) return tzh_fail(TZH_ERR_INVALID_ARGS, "node index %d out of range", idx);
        const tzh_node &n = tape[idx];
        if (n.ndim < 0 || n.ndim > TZH_MAX_RANK) return tzh_fail(TZH_ERR_SHAPE, "node %d: rank %d", idx, n.ndim);
        for (int i = 0; i < n.ndim; i++)
            if (n.shape[i] < 0) return tzh_fail(TZH_ERR_SHAPE, "node %d: negative dim", idx);
        switch (n.kind) {
        case TZH_NODE_TENSOR: {
            if (n.leaf < 0 || n.leaf >= n_leaves) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: leaf %d out of range", idx, n.leaf);
            const tzh_leaf &lf = leaves[n.leaf];
            if (lf.ndim != n.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: leaf rank mismatch", idx);
            for (int i = 0; i < n.ndim; i++)
                if (lf.shape[i] != n.shape[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: leaf shape mismatch", idx);
            if (!lf.data && numel_of(lf.ndim, lf.shape) > 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "leaf %d: null data", n.leaf);
            if (is_index_dtype(lf.dtype)) {
                if (!index_leaf_read_by_gather(idx))
                    return tzh_fail(TZH_ERR_WRONG_DTYPE, "leaf %d: integer tensors are only gather indices", n.leaf);
            } else if (lf.dtype != 0 && lf.dtype != dtype) {
                return tzh_fail(TZH_ERR_WRONG_DTYPE, "leaf %d: dtype %d is not the expression's element type %d",
                                n.leaf, lf.dtype, dtype);
            }
            return TZH_OK;
        }
        case TZH_NODE_CONSTANT:
            return TZH_OK;
        case TZH_NODE_UNARY: {
            if (!unary_ok(n.op)) return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "Unsupported unary operation: tag %d", n.op);
            if (n.lhs < 0 || n.lhs >= idx) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad input index", idx);
            const tzh_node &c = tape[n.lhs];
            if (c.ndim != n.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: unary shape mismatch", idx);
            for (int i = 0; i < n.ndim; i++)
                if (c.shape[i] != n.shape[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: unary shape mismatch", idx);
            return validate(n.lhs);
        }
        case TZH_NODE_BINARY: {
            if (!binary_ok(n.op)) return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "Unsupported binary operation: tag %d", n.op);
            if (n.lhs < 0 || n.lhs >= idx || n.rhs < 0 || n.rhs >= idx)
                return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad operand index", idx);
            const tzh_node &l = tape[n.lhs], &r = tape[n.rhs];
            const int nd = l.ndim > r.ndim ? l.ndim : r.ndim;
            if (n.ndim != nd) return tzh_fail(TZH_ERR_SHAPE, "Shapes not broadcast compatible (node %d)", idx);
            for (int i = 0; i < nd; i++) {
                const int li = i - (nd - l.ndim), ri = i - (nd - r.ndim);
                const int64_t a = li >= 0 ? l.shape[li] : 1, b = ri >= 0 ? r.shape[ri] : 1;
                if (a != b && a != 1 && b != 1) return tzh_fail(TZH_ERR_SHAPE, "Shapes not broadcast compatible (node %d)", idx);
                if (n.shape[i] != (a > b ? a : b)) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong broadcast result shape", idx);
                // shape.zig:196-200 takes @max, so an empty dimension against
                // a 1 gives a result of extent 1 whose element would be read
                // from the empty operand (the reference's slice access panics
                // there in a safe build): refuse it instead of reading past
                // an empty buffer.
                if ((a == 0 || b == 0) && n.shape[i] != 0)
                    return tzh_fail(TZH_ERR_SHAPE, "node %d: broadcast reads an element of an empty operand", idx);
            }
            TZH_TRY(validate(n.lhs));
            return validate(n.rhs);
        }
        case TZH_NODE_REDUCE: {
            if (!reduce_ok(n.op)) return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "Unsupported reduction: tag %d", n.op);
            if (n.lhs < 0 || n.lhs >= idx) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad input index", idx);
            const tzh_node &c = tape[n.lhs];
            if (n.axis < -1 || n.axis >= c.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: axis %d out of range", idx, n.axis);
            // shape.zig:279-320 ReduceShape
            int64_t want[TZH_MAX_RANK];
            int wn = 0;
            if (n.axis < 0) {
                if (n.keepdims) { wn = c.ndim; for (int i = 0; i < wn; i++) want[i] = 1; }
            } else {
                for (int i = 0; i < c.ndim; i++) {
                    if (i == n.axis) { if (n.keepdims) want[wn++] = 1; }
                    else want[wn++] = c.shape[i];
                }
            }
            if (n.ndim != wn) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong reduce result rank", idx);
            for (int i = 0; i < wn; i++)
                if (n.shape[i] != want[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong reduce result shape", idx);
            return validate(n.lhs);
        }
        case TZH_NODE_SOFTMAX: {
            if (n.lhs < 0 || n.lhs >= idx) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad input index", idx);
            TZH_TRY(same_shape(idx, n.lhs));
            if (n.axis < 0 || n.axis >= n.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: softmax axis %d", idx, n.axis);
            return validate(n.lhs);
        }
        case TZH_NODE_LAYERNORM: {
            if (n.lhs < 0 || n.lhs >= idx || n.rhs < 0 || n.rhs >= idx || n.aux < 0 || n.aux >= idx)
                return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad operand index", idx);
            TZH_TRY(same_shape(idx, n.lhs));
            if (n.axis < 1 || n.axis > n.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: norm_dims %d", idx, n.axis);
            for (int32_t pi : {n.rhs, n.aux}) {  // expr.zig:705-735: gamma/beta are the last norm_dims dims
                const tzh_node &q = tape[pi];
                if (q.ndim != n.axis)
                    return tzh_fail(TZH_ERR_SHAPE, "Gamma/beta rank must equal normalized_dims (node %d)", idx);
                for (int i = 0; i < n.axis; i++)
                    if (q.shape[i] != n.shape[n.ndim - n.axis + i])
                        return tzh_fail(TZH_ERR_SHAPE, "Gamma/beta shape must match last dimensions of input (node %d)", idx);
            }
            TZH_TRY(validate(n.lhs));
            TZH_TRY(validate(n.rhs));
            return validate(n.aux);
        }
        case TZH_NODE_TRANSPOSE: {
            if (n.lhs < 0 || n.lhs >= idx) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad input index", idx);
            const tzh_node &c = tape[n.lhs];
            if (c.ndim != n.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: transpose rank mismatch", idx);
            bool seen[TZH_MAX_RANK] = {};
            for (int i = 0; i < n.ndim; i++) {  // expr.zig:932-952
                const int p = n.perm[i];
                if (p < 0 || p >= n.ndim || seen[p])
                    return tzh_fail(TZH_ERR_SHAPE, "Invalid transpose permutation (node %d)", idx);
                seen[p] = true;
                if (n.shape[i] != c.shape[p]) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong transpose shape", idx);
            }
            return validate(n.lhs);
        }
        case TZH_NODE_MATMUL: {  // numpy matmul shape rules (executor.zig:199-326)
            if (n.lhs < 0 || n.lhs >= idx || n.rhs < 0 || n.rhs >= idx)
                return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad operand index", idx);
            MatmulArgs ma;
            int64_t want[TZH_MAX_RANK];
            int wn = 0;
            TZH_TRY(matmul_plan(idx, ma, want, &wn));
            if (n.ndim != wn) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong matmul result rank", idx);
            for (int i = 0; i < wn; i++)
                if (n.shape[i] != want[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong matmul result shape", idx);
            TZH_TRY(validate(n.lhs));
            return validate(n.rhs);
        }
        case TZH_NODE_GATHER: {  // expr.zig:775-830
            if (n.lhs < 0 || n.lhs >= idx || n.rhs < 0 || n.rhs >= idx)
                return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad operand index", idx);
            const tzh_node &t = tape[n.lhs], &ix = tape[n.rhs];
            if (t.ndim != 2) return tzh_fail(TZH_ERR_SHAPE, "Gather table must be 2D [vocab, embed] (node %d)", idx);
            if (ix.kind != TZH_NODE_TENSOR || ix.leaf < 0 || ix.leaf >= n_leaves || !is_index_dtype(leaves[ix.leaf].dtype))
                return tzh_fail(TZH_ERR_WRONG_DTYPE, "Gather indices must be an integer tensor (node %d)", idx);
            if (n.ndim != ix.ndim + 1 || n.shape[n.ndim - 1] != t.shape[1])
                return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong gather result shape", idx);
            for (int i = 0; i < ix.ndim; i++)
                if (n.shape[i] != ix.shape[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: wrong gather result shape", idx);
            TZH_TRY(validate(n.lhs));
            return validate(n.rhs);
        }
        case TZH_NODE_RESHAPE: {
            if (n.lhs < 0 || n.lhs >= idx) return tzh_fail(TZH_ERR_INVALID_ARGS, "node %d: bad input index", idx);
            const tzh_node &c = tape[n.lhs];
            if (numel_of(c.ndim, c.shape) != numel_of(n.ndim, n.shape))
                return tzh_fail(TZH_ERR_SHAPE, "node %d: reshape changes the element count", idx);
            return validate(n.lhs);
        }
        default:
            return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "node kind %d is not evaluated by this backend", n.kind);
        }
    }

    // Batch strides, m/k/n and the result shape of a matmul node: a 1-D lhs
    // is a row [1, k] and a 1-D rhs a column [k, 1] whose unit dimension
    // the result drops; batch dimensions broadcast.
    int matmul_plan(int32_t idx, MatmulArgs &ma, int64_t *out_shape, int *out_nd) const {
        const tzh_node &n = tape[idx], &l = tape[n.lhs], &r = tape[n.rhs];
        if (l.ndim < 1 || r.ndim < 1) return tzh_fail(TZH_ERR_SHAPE, "node %d: matmul of a scalar", idx);
        std::memset(&ma, 0, sizeof ma);
        const int64_t m = l.ndim == 1 ? 1 : l.shape[l.ndim - 2], k = l.shape[l.ndim - 1];
        const int64_t k2 = r.ndim == 1 ? r.shape[0] : r.shape[r.ndim - 2], nn = r.ndim == 1 ? 1 : r.shape[r.ndim - 1];
        if (k != k2) return tzh_fail(TZH_ERR_SHAPE, "Matmul inner dimensions differ (node %d)", idx);
        const int lb = l.ndim > 2 ? l.ndim - 2 : 0, rb = r.ndim > 2 ? r.ndim - 2 : 0;
        const int nb = lb > rb ? lb : rb;
        ma.nb = nb;
        ma.m = m;
        ma.k = k;
        ma.n = nn;
        int64_t as = m * k, bs = k * nn;
        for (int i = nb - 1; i >= 0; i--) {
            const int li = i - (nb - lb), ri = i - (nb - rb);
            const int64_t ld = li >= 0 ? l.shape[li] : 1, rd = ri >= 0 ? r.shape[ri] : 1;
            if (ld != rd && ld != 1 && rd != 1) return tzh_fail(TZH_ERR_SHAPE, "Matmul batch dimensions not broadcast compatible (node %d)", idx);
            ma.batch_shape[i] = ld > rd ? ld : rd;
            ma.a_stride[i] = ld == 1 ? 0 : as;
            ma.b_stride[i] = rd == 1 ? 0 : bs;
            if (li >= 0) as *= ld;
            if (ri >= 0) bs *= rd;
        }
        int w = 0;
        for (int i = 0; i < nb; i++) out_shape[w++] = ma.batch_shape[i];
        if (l.ndim > 1) out_shape[w++] = m;
        if (r.ndim > 1) out_shape[w++] = nn;
        *out_nd = w;
        return TZH_OK;
    }

    static bool is_index_dtype(int32_t d) { return d == TZH_I32 || d == TZH_U32 || d == TZH_I64 || d == TZH_U64; }

    // An integer leaf node may be read only as a gather's indices.
    bool index_leaf_read_by_gather(int32_t leaf_node) const {
        bool read = false;
        for (int32_t i = leaf_node + 1; i < n_nodes; i++) {
            const tzh_node &t = tape[i];
            const bool as_indices = t.kind == TZH_NODE_GATHER && t.rhs == leaf_node;
            const bool other = (t.lhs == leaf_node) || (t.rhs == leaf_node && !as_indices) ||
                               (t.kind == TZH_NODE_LAYERNORM && t.aux == leaf_node);
            if (other) return false;
            read = read || as_indices;
        }
        return read;
    }

    int same_shape(int32_t a, int32_t b) const {
        const tzh_node &x = tape[a], &y = tape[b];
        if (x.ndim != y.ndim) return tzh_fail(TZH_ERR_SHAPE, "node %d: shape mismatch with its input", a);
        for (int i = 0; i < x.ndim; i++)
            if (x.shape[i] != y.shape[i]) return tzh_fail(TZH_ERR_SHAPE, "node %d: shape mismatch with its input", a);
        return TZH_OK;
    }

    // Nodes computed by a kernel of their own, read by chains as leaves.
    static bool materialised_kind(int k) {
        return k == TZH_NODE_REDUCE || k == TZH_NODE_SOFTMAX || k == TZH_NODE_LAYERNORM || k == TZH_NODE_TRANSPOSE ||
               k == TZH_NODE_RESHAPE || k == TZH_NODE_GATHER || k == TZH_NODE_MATMUL;
    }

    // Nodes evaluated into a temporary before the program that reads them
    // (reductions, and subtrees cut to fit the kernel's limits).
    std::vector<char> cut;

    bool is_leafish(int32_t idx) const {
        const int k = tape[idx].kind;
        return cut[(size_t)idx] || k == TZH_NODE_TENSOR || k == TZH_NODE_CONSTANT || materialised_kind(k);
    }
    // value-stack depth to evaluate idx inline (Sethi-Ullman for a stack machine)
    int depth(int32_t idx) const {
        if (is_leafish(idx)) return 1;
        const tzh_node &n = tape[idx];
        if (n.kind == TZH_NODE_UNARY) return depth(n.lhs);
        const int a = depth(n.lhs), b = depth(n.rhs) + 1;
        return a > b ? a : b;
    }
    // program nodes and leaves to evaluate idx inline
    int count(int32_t idx, int *leaves_out) const {
        if (is_leafish(idx)) {
            if (tape[idx].kind != TZH_NODE_CONSTANT) (*leaves_out)++;
            return 1;
        }
        const tzh_node &n = tape[idx];
        if (n.kind == TZH_NODE_UNARY) return 1 + count(n.lhs, leaves_out);
        return 1 + count(n.lhs, leaves_out) + count(n.rhs, leaves_out);
    }
    bool fits(int32_t idx) const {
        int nl = 0;
        const int nn = count(idx, &nl);
        return depth(idx) <= kMaxDepth && nn <= kMaxNodes && nl <= kMaxLeaves;
    }
    // Candidate cut points: elementwise nodes strictly below `root` and not
    // already inside a cut subtree.  `rhs_only` restricts to right operands
    // (the only place stack depth grows).
    void candidates(int32_t idx, bool is_root, bool is_rhs, bool rhs_only, std::vector<int32_t> &out) const {
        if (!is_root && is_leafish(idx)) return;
        const tzh_node &n = tape[idx];
        if (n.kind != TZH_NODE_UNARY && n.kind != TZH_NODE_BINARY) return;
        if (!is_root && (!rhs_only || is_rhs)) out.push_back(idx);
        candidates(n.lhs, false, false, rhs_only, out);
        if (n.kind == TZH_NODE_BINARY) candidates(n.rhs, false, true, rhs_only, out);
    }
    // Cut subtrees below `root` until the inline program fits; each cut
    // subtree is later compiled as a program of its own (and split again if
    // it is still too large), so every program root is evaluated inline.
    void choose_cuts(int32_t root) {
        while (!fits(root)) {
            const bool deep = depth(root) > kMaxDepth;
            std::vector<int32_t> cand;
            candidates(root, true, false, deep, cand);
            if (cand.empty()) candidates(root, true, false, false, cand);
            int32_t best = -1, best_score = -1;
            bool best_fits = false;
            for (int32_t c : cand) {
                int nl = 0;
                const int score = deep ? depth(c) : count(c, &nl);
                const bool f = fits(c);
                if ((f && !best_fits) || (f == best_fits && score > best_score)) {
                    best = c;
                    best_score = score;
                    best_fits = f;
                }
            }
            if (best < 0) break;  // nothing left to cut: root's own operands are leaves
            cut[(size_t)best] = 1;
        }
    }

    int add_leaf(EwProgram &p, const void *ptr, int32_t lnd, const int64_t *lshape, int vec, int *leaf_idx) {
        if (p.n_leaves >= kMaxLeaves) return tzh_fail(TZH_ERR_INVALID_ARGS, "internal: too many leaves");
        // every element of the program's output reads every leaf once, so a
        // leaf with no elements can back only an empty program
        if (p.numel > 0 && numel_of(lnd, lshape) == 0)
            return tzh_fail(TZH_ERR_SHAPE, "internal: a non-empty program reads an empty operand");
        EwLeaf &lf = p.leaves[p.n_leaves];
        std::memset(&lf, 0, sizeof lf);
        lf.ptr = ptr;
        // broadcast strides onto the program's output index space (strides.zig:92-121)
        int64_t cs[TZH_MAX_RANK];
        int64_t s = 1;
        for (int i = lnd - 1; i >= 0; i--) { cs[i] = s; s *= lshape[i]; }
        int first = -1, last = -1;
        for (int i = 0; i < p.ndim; i++) {
            const int si = i - (p.ndim - lnd);
            lf.strides[i] = (si >= 0 && lshape[si] != 1) ? cs[si] : 0;
            if (lf.strides[i] != 0) { if (first < 0) first = i; last = i; }
        }
        bool contiguous_run = true;
        for (int i = first; first >= 0 && i <= last; i++)
            if (lf.strides[i] == 0 && p.shape[i] != 1) contiguous_run = false;
        if (first < 0) {  // scalar
            lf.general = 0; lf.div = 1; lf.mod = 1;
        } else if (contiguous_run) {
            int64_t div = 1, mod = 1;
            for (int i = last + 1; i < p.ndim; i++) div *= p.shape[i];
            for (int i = first; i <= last; i++) mod *= p.shape[i];
            lf.general = 0; lf.div = div; lf.mod = mod;
        } else {
            lf.general = 1; lf.div = 1; lf.mod = 1;
        }
        lf.fdiv = make_fastdiv((uint64_t)lf.div);
        lf.fmod = make_fastdiv((uint64_t)lf.mod);
        // (flat / div) < numel <= mod: the modulo never wraps, skip it
        const bool wraps = lf.mod < p.numel;
        const bool aligned = ((uintptr_t)ptr % 16) == 0;
        if (!lf.general && lf.div == 1 && (!wraps || lf.mod % vec == 0) && aligned) lf.vec = VEC_CONTIG;
        else if (!lf.general && lf.div % vec == 0) lf.vec = VEC_SPLAT;
        else lf.vec = VEC_PER_ELEM;
        if (!wraps) lf.mod = INT64_MAX;
        *leaf_idx = p.n_leaves++;
        return TZH_OK;
    }

    int push(EwProgram &p, int16_t kind, int16_t op, int16_t slot, int16_t arg, double cval) {
        if (p.n_nodes >= kMaxNodes) return tzh_fail(TZH_ERR_INVALID_ARGS, "internal: program too long");
        EwNode &nd = p.nodes[p.n_nodes++];
        nd.kind = kind; nd.op = op; nd.slot = slot; nd.arg = arg; nd.pad0 = nd.pad1 = 0; nd.cval = cval;
        return TZH_OK;
    }

    // Materialise node idx into a fresh device temporary.
    int materialise(int32_t idx, void **buf) {
        const tzh_node &n = tape[idx];
        const size_t bytes = (size_t)numel_of(n.ndim, n.shape) * es;
        void *t = nullptr;
        TZH_TRY(temporary(bytes, &t));
        TZH_TRY(eval_into(idx, t));
        *buf = t;
        return TZH_OK;
    }

    int emit(EwProgram &p, int32_t idx, int sp, int vec, bool is_root) {
        const tzh_node &n = tape[idx];
        if (sp >= kMaxDepth) return tzh_fail(TZH_ERR_INVALID_ARGS, "internal: value stack overflow");
        if (n.kind == TZH_NODE_RESHAPE && tape[n.lhs].kind == TZH_NODE_TENSOR) {
            // a reshaped leaf is the same contiguous data under another shape
            int li;
            TZH_TRY(add_leaf(p, leaves[tape[n.lhs].leaf].data, n.ndim, n.shape, vec, &li));
            return push(p, EK_LEAF, 0, (int16_t)sp, (int16_t)li, 0.0);
        }
        // (a reduction's input program may itself be rooted at such a node)
        if (materialised_kind(n.kind) || (!is_root && cut[(size_t)idx])) {
            void *buf = nullptr;
            TZH_TRY(materialise(idx, &buf));
            int li;
            TZH_TRY(add_leaf(p, buf, n.ndim, n.shape, vec, &li));
            return push(p, EK_LEAF, 0, (int16_t)sp, (int16_t)li, 0.0);
        }
        switch (n.kind) {
        case TZH_NODE_TENSOR: {
            int li;
            TZH_TRY(add_leaf(p, leaves[n.leaf].data, n.ndim, n.shape, vec, &li));
            return push(p, EK_LEAF, 0, (int16_t)sp, (int16_t)li, 0.0);
        }
        case TZH_NODE_CONSTANT:
            return push(p, EK_CONST, 0, (int16_t)sp, 0, n.value);
        case TZH_NODE_UNARY:
            TZH_TRY(emit(p, n.lhs, sp, vec, false));
            return push(p, EK_UNARY, (int16_t)n.op, (int16_t)sp, 0, 0.0);
        case TZH_NODE_BINARY:
            TZH_TRY(emit(p, n.lhs, sp, vec, false));
            TZH_TRY(emit(p, n.rhs, sp + 1, vec, false));
            return push(p, EK_BINARY, (int16_t)n.op, (int16_t)sp, 0, 0.0);
        default:
            return tzh_fail(TZH_ERR_UNSUPPORTED_OP, "node kind %d", n.kind);
        }
    }

    int compile(int32_t idx, EwProgram &p, int vec) {
        std::memset(&p, 0, sizeof p);
        if (cut.size() != (size_t)n_nodes) cut.assign((size_t)n_nodes, 0);
        const tzh_node &n = tape[idx];
        p.ndim = n.ndim;
        for (int i = 0; i < n.ndim; i++) p.shape[i] = n.shape[i];
        p.numel = numel_of(n.ndim, n.shape);
        p.small = p.numel < ((int64_t)1 << 32) ? 1 : 0;
        for (int i = 0; i < n.ndim; i++) p.fshape[i] = make_fastdiv((uint64_t)n.shape[i]);
        // a cut node being materialised is this program's root: evaluate it inline
        const char was_cut = cut[(size_t)idx];
        cut[(size_t)idx] = 0;
        choose_cuts(idx);
        int rc = fits(idx) ? emit(p, idx, 0, vec, true)
                           : tzh_fail(TZH_ERR_INVALID_ARGS, "internal: expression cannot be split to fit");
        cut[(size_t)idx] = was_cut;
        return rc;
    }

    // One work item per thread: measured on MI355X (config 2, 2^26 vectors)
    // a grid that covers every item once streams at 6.1 TB/s, while
    // grid-stride loops over 16 to 512 blocks per CU reached 4.5 to 5.4.
    // The cap only keeps the block count bounded for very large tensors.
    int grid_for(int64_t work_items) const {
        int64_t g = (work_items + 255) / 256;
        const int64_t cap = (int64_t)ctx->num_cus * 4096;
        if (g > cap) g = cap;
        if (g < 1) g = 1;
        return (int)g;
    }

    template <typename T, int V>
    int launch_chain(int32_t idx, T *out) {
        EwProgram p;
        TZH_TRY(compile(idx, p, V));
        if (p.numel == 0) return TZH_OK;
        const int g = grid_for(p.numel / V);
        if constexpr (kHaveJit) {
            if (!ctx->ew_interpreter) return jit_chain_launch(ctx, p, sizeof(T) == 8, V, g, out);
        }
        hipLaunchKernelGGL((ew_chain_kernel<T, V>), dim3(g), dim3(256), 0, ctx->stream, p, out);
        TZH_LAUNCHED("ew_chain_kernel");
        return TZH_OK;
    }

    template <typename T, int V>
    int launch_reduce(int32_t idx, T *out) {
        const tzh_node &n = tape[idx];
        const tzh_node &c = tape[n.lhs];
        EwProgram p;
        const int64_t out_numel = numel_of(n.ndim, n.shape);
        if (n.axis < 0) {
            TZH_TRY(compile(n.lhs, p, V));
            const int g = grid_for(p.numel / V);
            void *partials = nullptr;
            TZH_TRY(tzh_ctx_scratch(ctx, sizeof(T) * (size_t)g, &partials));
            hipLaunchKernelGGL((ew_reduce_all_kernel<T, V>), dim3(g), dim3(256), 0, ctx->stream, p, n.op, (T *)partials);
            TZH_LAUNCHED("ew_reduce_all_kernel");
            hipLaunchKernelGGL((ew_reduce_finish_kernel<T>), dim3(1), dim3(256), 0, ctx->stream, (const T *)partials, g,
                               n.op, p.numel, out, out_numel);
            TZH_LAUNCHED("ew_reduce_finish_kernel");
            return TZH_OK;
        }
        TZH_TRY(compile(n.lhs, p, 1));
        int64_t outer = 1, inner = 1;
        const int64_t rsz = c.shape[n.axis];
        for (int i = 0; i < n.axis; i++) outer *= c.shape[i];
        for (int i = n.axis + 1; i < c.ndim; i++) inner *= c.shape[i];
        if (outer * inner == 0) return TZH_OK;
        if (inner == 1) {
            const int64_t blocks = (outer + 3) / 4;
            hipLaunchKernelGGL((ew_reduce_rows_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, p, n.op,
                               outer, rsz, out);
            TZH_LAUNCHED("ew_reduce_rows_kernel");
        } else {
            const int64_t blocks = (outer * inner + 255) / 256;
            hipLaunchKernelGGL((ew_reduce_cols_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, p, n.op,
                               outer, rsz, inner, out);
            TZH_LAUNCHED("ew_reduce_cols_kernel");
        }
        return TZH_OK;
    }

    // Contiguous data of node idx: a leaf's own buffer, else a temporary.
    int input_data(int32_t idx, const void **out) {
        const tzh_node &n = tape[idx];
        if (n.kind == TZH_NODE_TENSOR) {
            *out = leaves[n.leaf].data;
            return TZH_OK;
        }
        void *buf = nullptr;
        TZH_TRY(materialise(idx, &buf));
        *out = buf;
        return TZH_OK;
    }

    template <typename T>
    int launch_structural(int32_t idx, T *out) {
        const tzh_node &n = tape[idx];
        const int64_t numel = numel_of(n.ndim, n.shape);
        if (n.kind == TZH_NODE_RESHAPE) return eval_into(n.lhs, out);  // executor.zig:481-495
        const void *x = nullptr;
        TZH_TRY(input_data(n.lhs, &x));
        if (numel == 0) return TZH_OK;
        if (n.kind == TZH_NODE_SOFTMAX) {
            int64_t outer = 1, inner = 1;
            const int64_t len = n.shape[n.axis];
            for (int i = 0; i < n.axis; i++) outer *= n.shape[i];
            for (int i = n.axis + 1; i < n.ndim; i++) inner *= n.shape[i];
            if (inner == 1) return softmax_rows<T>((const T *)x, out, outer, len);
            if (outer * inner >= 65536) {  // enough columns for one thread each
                hipLaunchKernelGGL((ew_softmax_cols_kernel<T>), dim3((unsigned)((outer * inner + 255) / 256)), dim3(256),
                                   0, ctx->stream, (const T *)x, out, outer, len, inner);
                TZH_LAUNCHED("ew_softmax_cols_kernel");
                return TZH_OK;
            }
            // few long columns: [outer, len, inner] -> [outer, inner, len],
            // softmax along rows, and back, through two stream-ordered
            // temporaries
            const size_t bytes = (size_t)numel * sizeof(T);
            void *t1 = nullptr, *t2 = nullptr;
            TZH_TRY(temporary(bytes, &t1));
            TZH_TRY(temporary(bytes, &t2));
            const int64_t s3[3] = {outer, len, inner}, s3t[3] = {outer, inner, len};
            const int p021[3] = {0, 2, 1};
            TZH_TRY(launch_transpose<T>((const T *)x, (T *)t1, 3, s3, p021));
            TZH_TRY(softmax_rows<T>((const T *)t1, (T *)t2, outer * inner, len));
            return launch_transpose<T>((const T *)t2, out, 3, s3t, p021);
        }
        if (n.kind == TZH_NODE_LAYERNORM) {
            const void *g = nullptr, *b = nullptr;
            TZH_TRY(input_data(n.rhs, &g));
            TZH_TRY(input_data(n.aux, &b));
            int64_t len = 1;
            for (int i = n.ndim - n.axis; i < n.ndim; i++) len *= n.shape[i];
            const int64_t rows = numel / len;
            // layernorm.zig:15: default_eps is the f32 1e-5, widened for f64
            constexpr int V = 16 / sizeof(T);
            const dim3 grid((unsigned)((rows + 3) / 4));
            if (len % V == 0 && aligned16(x) && aligned16(g) && aligned16(b) && aligned16(out))
                hipLaunchKernelGGL((ew_layernorm_kernel<T, V>), grid, dim3(256), 0, ctx->stream, (const T *)x,
                                   (const T *)g, (const T *)b, out, rows, len, (T)1e-5f);
            else
                hipLaunchKernelGGL((ew_layernorm_kernel<T, 1>), grid, dim3(256), 0, ctx->stream, (const T *)x,
                                   (const T *)g, (const T *)b, out, rows, len, (T)1e-5f);
            TZH_LAUNCHED("ew_layernorm_kernel");
            return TZH_OK;
        }
        if (n.kind == TZH_NODE_MATMUL) return launch_matmul(idx, nullptr, 0, out);
        if (n.kind == TZH_NODE_GATHER) {
            const tzh_node &t = tape[n.lhs];
            const tzh_leaf &il = leaves[tape[n.rhs].leaf];
            const dim3 grid((unsigned)((numel + 255) / 256));
            const T *tab = (const T *)x;
            switch (il.dtype) {
            case TZH_I32: hipLaunchKernelGGL((ew_gather_kernel<T, int32_t>), grid, dim3(256), 0, ctx->stream, tab, (const int32_t *)il.data, out, t.shape[0], t.shape[1], numel); break;
            case TZH_U32: hipLaunchKernelGGL((ew_gather_kernel<T, uint32_t>), grid, dim3(256), 0, ctx->stream, tab, (const uint32_t *)il.data, out, t.shape[0], t.shape[1], numel); break;
            case TZH_I64: hipLaunchKernelGGL((ew_gather_kernel<T, int64_t>), grid, dim3(256), 0, ctx->stream, tab, (const int64_t *)il.data, out, t.shape[0], t.shape[1], numel); break;
            default: hipLaunchKernelGGL((ew_gather_kernel<T, uint64_t>), grid, dim3(256), 0, ctx->stream, tab, (const uint64_t *)il.data, out, t.shape[0], t.shape[1], numel); break;
            }
            TZH_LAUNCHED("ew_gather_kernel");
            return TZH_OK;
        }
        // TZH_NODE_TRANSPOSE
        const tzh_node &c = tape[n.lhs];
        return launch_transpose<T>((const T *)x, out, n.ndim, c.shape, n.perm);
    }

    static bool aligned16(const void *p) { return ((uintptr_t)p % 16) == 0; }

    template <typename T>
    int softmax_rows(const T *x, T *y, int64_t rows, int64_t len) {
        constexpr int V = 16 / sizeof(T);
        const dim3 grid((unsigned)((rows + 3) / 4));
        if (len % V == 0 && aligned16(x) && aligned16(y))
            hipLaunchKernelGGL((ew_softmax_rows_kernel<T, V>), grid, dim3(256), 0, ctx->stream, x, y, rows, len);
        else
            hipLaunchKernelGGL((ew_softmax_rows_kernel<T, 1>), grid, dim3(256), 0, ctx->stream, x, y, rows, len);
        TZH_LAUNCHED("ew_softmax_rows_kernel");
        return TZH_OK;
    }

    // y = x with its axes permuted: output axis i is input axis perm[i]
    template <typename T>
    int launch_transpose(const T *x, T *y, int nd, const int64_t *in_shape, const int32_t *perm) {
        TransposeArgs a;
        std::memset(&a, 0, sizeof a);
        a.ndim = nd;
        int64_t in_stride[TZH_MAX_RANK];
        int64_t st = 1, numel = 1;
        for (int i = nd - 1; i >= 0; i--) {
            in_stride[i] = st;
            st *= in_shape[i];
        }
        for (int i = 0; i < nd; i++) {
            a.out_shape[i] = in_shape[perm[i]];
            a.src_stride[i] = in_stride[perm[i]];
            numel *= in_shape[i];
        }
        if (numel == 0) return TZH_OK;
        int q = -1;
        for (int i = 0; i < nd; i++)
            if (perm[i] == nd - 1) q = i;
        if (nd >= 2 && q != nd - 1) {  // the last axis moves: tiles through LDS
            TileTransposeArgs t;
            std::memset(&t, 0, sizeof t);
            int64_t out_stride[TZH_MAX_RANK], os = 1;
            for (int i = nd - 1; i >= 0; i--) {
                out_stride[i] = os;
                os *= a.out_shape[i];
            }
            t.n_l = a.out_shape[nd - 1];
            t.n_q = a.out_shape[q];
            t.src_l = a.src_stride[nd - 1];
            t.dst_q = out_stride[q];
            t.nz = 1;
            for (int i = 0; i < nd - 1; i++) {
                if (i == q) continue;
                t.rest_shape[t.nrest] = a.out_shape[i];
                t.rest_src[t.nrest] = a.src_stride[i];
                t.rest_dst[t.nrest] = out_stride[i];
                t.nz *= a.out_shape[i];
                t.nrest++;
            }
            const int64_t gx = (t.n_l + 31) / 32, gy = (t.n_q + 31) / 32;
            if (gx <= 0x7fffffff && gy <= 65535) {
                const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)(t.nz < 65535 ? t.nz : 65535));
                hipLaunchKernelGGL((ew_transpose_tiled_kernel<T>), grid, dim3(256), 0, ctx->stream, x, y, t);
                TZH_LAUNCHED("ew_transpose_tiled_kernel");
                return TZH_OK;
            }
        }
        hipLaunchKernelGGL((ew_transpose_kernel<T>), dim3((unsigned)((numel + 255) / 256)), dim3(256), 0, ctx->stream,
                           x, y, a, numel);
        TZH_LAUNCHED("ew_transpose_kernel");
        return TZH_OK;
    }

    // Matmul node `mm` on the matrix cores (gemm_fp.hip), with `n_ops` fused
    // epilogue ops (bias adds read `bias` as a row vector over the last axis).
    int launch_matmul(int32_t mm, const void *bias, int n_ops, void *out, const int32_t *ops = nullptr) {
        const tzh_node &n = tape[mm];
        const void *adat = nullptr, *bdat = nullptr;
        TZH_TRY(input_data(n.lhs, &adat));
        TZH_TRY(input_data(n.rhs, &bdat));
        MatmulArgs ma;
        int64_t shp[TZH_MAX_RANK];
        int nd = 0;
        TZH_TRY(matmul_plan(mm, ma, shp, &nd));
        tzh_gemm_desc d;
        d.m = ma.m, d.n = ma.n, d.k = ma.k, d.lda = ma.k, d.ldb = ma.n, d.ldy = ma.n;
        d.nb = ma.nb;
        for (int i = 0; i < ma.nb; i++) {
            d.batch_shape[i] = ma.batch_shape[i];
            d.a_bstride[i] = ma.a_stride[i];
            d.b_bstride[i] = ma.b_stride[i];
        }
        d.y_bstride = ma.m * ma.n;
        d.bias = bias;
        d.n_ops = n_ops;
        for (int o = 0; o < n_ops; o++) d.ops[o] = ops[o];
        return tzh_gemm_fp_launch(ctx->stream, dtype, false, false, adat, bdat, out, d);
    }

    // A row vector over the last axis of a result of rank nd: a leaf whose
    // dimensions are all 1 but the last, which is n.
    bool is_row_bias(int32_t idx, int nd, int64_t n) const {
        const tzh_node &b = tape[idx];
        if (b.kind != TZH_NODE_TENSOR || b.ndim < 1 || b.ndim > nd || b.shape[b.ndim - 1] != n) return false;
        for (int i = 0; i < b.ndim - 1; i++)
            if (b.shape[i] != 1) return false;
        return true;
    }

    // FusedMatmulEpilogueKernel (fusion/codegen.zig:78-147; the plan of
    // analyzer.zig:106-153, 268-297): a root that is unary ops and adds of
    // one bias row vector over a matmul of its own shape is evaluated by the
    // matmul kernel, the ops applied in order (innermost first) to each
    // output.  *fused = false (nothing launched) when the root has another
    // form.
    int try_fused_matmul(int32_t idx, void *out, bool *fused) {
        *fused = false;
        const tzh_node &root = tape[idx];
        int32_t chain[8];
        int len = 0;
        int32_t cur = idx, bias_node = -1;
        while (len < 8) {
            const tzh_node &n = tape[cur];
            if (n.kind == TZH_NODE_MATMUL) break;
            if (n.ndim != root.ndim) return TZH_OK;
            for (int i = 0; i < n.ndim; i++)
                if (n.shape[i] != root.shape[i]) return TZH_OK;
            if (n.kind == TZH_NODE_UNARY && unary_ok(n.op)) {
                chain[len++] = cur;
                cur = n.lhs;
            } else if (n.kind == TZH_NODE_BINARY && n.op == TZH_OP_ADD && root.ndim >= 1) {
                const int64_t last = root.shape[root.ndim - 1];
                int32_t next, b;
                if (is_row_bias(n.rhs, root.ndim, last)) next = n.lhs, b = n.rhs;
                else if (is_row_bias(n.lhs, root.ndim, last)) next = n.rhs, b = n.lhs;
                else return TZH_OK;
                if (bias_node >= 0 && leaves[tape[bias_node].leaf].data != leaves[tape[b].leaf].data) return TZH_OK;
                bias_node = b;
                chain[len++] = cur;
                cur = next;
            } else {
                return TZH_OK;
            }
        }
        const tzh_node &mm = tape[cur];
        if (mm.kind != TZH_NODE_MATMUL || len == 0 || len > 4 || mm.ndim != root.ndim) return TZH_OK;
        for (int i = 0; i < mm.ndim; i++)
            if (mm.shape[i] != root.shape[i]) return TZH_OK;
        if (numel_of(root.ndim, root.shape) == 0) return TZH_OK;  // nothing to compute: the chain path returns
        int32_t ops[4];
        for (int o = 0; o < len; o++) {
            const tzh_node &n = tape[chain[len - 1 - o]];
            ops[o] = n.kind == TZH_NODE_UNARY ? n.op : TZH_OP_ADD;
        }
        *fused = true;
        return launch_matmul(cur, bias_node >= 0 ? leaves[tape[bias_node].leaf].data : nullptr, len, out, ops);
    }

    int eval_into(int32_t idx, void *out) {
        const tzh_node &n = tape[idx];
        const bool is64 = dtype == TZH_F64;
        if ((n.kind == TZH_NODE_UNARY || n.kind == TZH_NODE_BINARY) && !ctx->ew_interpreter) {
            bool fused = false;
            TZH_TRY(try_fused_matmul(idx, out, &fused));
            if (fused) return TZH_OK;
        }
        if (n.kind != TZH_NODE_REDUCE && materialised_kind(n.kind))
            return is64 ? launch_structural<double>(idx, (double *)out) : launch_structural<float>(idx, (float *)out);
        if (n.kind == TZH_NODE_REDUCE)
            return is64 ? launch_reduce<double, 2>(idx, (double *)out) : launch_reduce<float, 4>(idx, (float *)out);
        return is64 ? launch_chain<double, 2>(idx, (double *)out) : launch_chain<float, 4>(idx, (float *)out);
    }
};

}  // namespace

extern "C" int tzh_eval_into(tzh_ctx *ctx, const tzh_node *tape, int32_t n_nodes, const tzh_leaf *leaves,
                             int32_t n_leaves, int32_t dtype, void *out) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!tape || n_nodes <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "empty expression");
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad leaves");
    if (dtype != TZH_F32 && dtype != TZH_F64)
        return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "eval supports F32 and F64 element types (got %d)", dtype);
    Planner pl{ctx, tape, n_nodes, leaves, n_leaves, dtype, dtype == TZH_F64 ? 8u : 4u, {}};
    TZH_TRY(pl.validate(n_nodes - 1));
    const tzh_node &root = tape[n_nodes - 1];
    if (numel_of(root.ndim, root.shape) > 0 && !out) return tzh_fail(TZH_ERR_INVALID_ARGS, "null output");
    return pl.eval_into(n_nodes - 1, out);
}
