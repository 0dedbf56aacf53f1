// tenzor.hpp — C++17 host API over libtenzor_hip (include/tenzor_hip.h).
//
// Mirrors the reference's Zig surfaces for this path with the same names and
// argument meaning, so code and tests read like the reference's:
//
//   using Vec = tenzor::Tensor<float, 4>;                      // Tensor(f32, .{4})   tensor.zig:28
//   auto a = Vec::fromSlice(ctx, {1, 2, 3, 4});                 // Tensor.fromSlice    tensor.zig:84
//   auto e = tenzor::BinaryExpr<tenzor::OpTag::add, Vec, Vec>::init(a, b).mul(c).exp();  // expr.zig:352
//   auto r = tenzor::eval(ctx, e);                              // executor.eval       executor.zig:29
//   tenzor::evalInto(ctx, e, out);                              // executor.evalInto   executor.zig:49
//
//   auto w = tenzor::arctic::ModelWeights::fromSafeTensors(ctx, "model.safetensors");  // arctic.zig:113
//   tenzor::arctic::forwardBatch(outputs, ids, lengths, stride, w);                    // arctic.zig:902-1013
//   tenzor::arctic::feedForward(output, input, w, layer, seq_len);                     // arctic.zig:760-811
//   tenzor::io::Tokenizer tok; tok.loadVocab("vocab.txt");                             // tokenizer.zig:17-51
//   tenzor::arctic::embedDocuments(outputs, docs, tok.handle(), w);                    // main.zig:786-933
//
// Shapes are template parameters, as comptime shapes are in Zig: element
// types and broadcast compatibility are checked at compile time
// (expr.zig:358-376, shape.zig:168-204) with static_assert, where Zig uses
// @compileError.  Run-time failures throw tenzor::Error carrying the
// library's status code, whose names are the Zig error names.
#pragma once

#include <array>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/tenzor_hip.h"

namespace tenzor {

// ---------------------------------------------------------------- errors
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &msg) : std::runtime_error(msg), code(c) {}
};

inline void check(int rc) {
    if (rc != TZH_OK) throw Error(rc, tzh_last_error());
}

// --------------------------------------------------------------- context
// One device + one stream; not thread-safe (one per thread), like
// arctic.InferenceContext (arctic.zig:407-482).
class Context {
  public:
    explicit Context(int device = 0, void *stream = nullptr) { check(tzh_init(device, stream, &h_)); }
    ~Context() {
        if (h_) tzh_destroy(h_);
    }
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;
    void sync() { check(tzh_sync(h_)); }
    tzh_ctx *handle() const { return h_; }

  private:
    tzh_ctx *h_ = nullptr;
};

// ------------------------------------------------------------- op tags
// ops.OpTag (expr.zig:19-91); values are the C-ABI's TZH_OP_* ordinals.
enum class OpTag : int32_t {
    neg = TZH_OP_NEG, abs = TZH_OP_ABS, exp = TZH_OP_EXP, log = TZH_OP_LOG, sqrt = TZH_OP_SQRT,
    rsqrt = TZH_OP_RSQRT, sin = TZH_OP_SIN, cos = TZH_OP_COS, tanh = TZH_OP_TANH, sigmoid = TZH_OP_SIGMOID,
    relu = TZH_OP_RELU, gelu = TZH_OP_GELU, silu = TZH_OP_SILU, softplus = TZH_OP_SOFTPLUS,
    ceil = TZH_OP_CEIL, floor = TZH_OP_FLOOR, round = TZH_OP_ROUND,
    add = TZH_OP_ADD, sub = TZH_OP_SUB, mul = TZH_OP_MUL, div = TZH_OP_DIV, pow = TZH_OP_POW,
    max = TZH_OP_MAX, min = TZH_OP_MIN,
    sum = TZH_OP_SUM, prod = TZH_OP_PROD, reduce_max = TZH_OP_REDUCE_MAX, reduce_min = TZH_OP_REDUCE_MIN,
    mean = TZH_OP_MEAN,
};

// NodeKind (expr.zig:137-149)
enum class NodeKind : int32_t { tensor = TZH_NODE_TENSOR, constant = TZH_NODE_CONSTANT, unary = TZH_NODE_UNARY,
                                binary = TZH_NODE_BINARY, matmul = TZH_NODE_MATMUL, reduce = TZH_NODE_REDUCE,
                                reshape = TZH_NODE_RESHAPE, transpose = TZH_NODE_TRANSPOSE,
                                softmax = TZH_NODE_SOFTMAX, layernorm = TZH_NODE_LAYERNORM };

template <typename T>
constexpr int32_t dtype_of() {
    static_assert(std::is_same<T, float>::value || std::is_same<T, double>::value,
                  "the GPU evaluator supports f32 and f64 expressions");
    return std::is_same<T, float>::value ? TZH_F32 : TZH_F64;
}

// ----------------------------------------------------------- shape algebra
template <size_t N>
using Shape = std::array<int64_t, N>;

template <size_t N>
constexpr int64_t numel(const Shape<N> &s) {
    int64_t n = 1;
    for (size_t i = 0; i < N; i++) n *= s[i];
    return n;
}

// BroadcastShape (shape.zig:168-204): NumPy rules, right-aligned.
template <size_t A, size_t B>
constexpr bool broadcast_compatible(const Shape<A> &a, const Shape<B> &b) {
    constexpr size_t n = A > B ? A : B;
    for (size_t i = 0; i < n; i++) {
        const int64_t da = i < n - A ? 1 : a[i - (n - A)];
        const int64_t db = i < n - B ? 1 : b[i - (n - B)];
        if (da != db && da != 1 && db != 1) return false;
    }
    return true;
}

template <size_t A, size_t B>
constexpr Shape<(A > B ? A : B)> broadcast_shape(const Shape<A> &a, const Shape<B> &b) {
    constexpr size_t n = A > B ? A : B;
    Shape<n> out{};
    for (size_t i = 0; i < n; i++) {
        const int64_t da = i < n - A ? 1 : a[i - (n - A)];
        const int64_t db = i < n - B ? 1 : b[i - (n - B)];
        out[i] = da > db ? da : db;
    }
    return out;
}

// ------------------------------------------------------------------- tape
struct Tape {
    std::vector<tzh_node> nodes;
    std::vector<tzh_leaf> leaves;
    std::vector<const void *> leaf_ptrs;

    template <size_t N>
    static tzh_node node_of(NodeKind kind, const Shape<N> &shape) {
        tzh_node n;
        std::memset(&n, 0, sizeof n);
        n.kind = (int32_t)kind;
        n.lhs = n.rhs = n.leaf = -1;
        n.axis = -1;
        n.ndim = (int32_t)N;
        for (size_t i = 0; i < N; i++) n.shape[i] = shape[i];
        return n;
    }

    int32_t push(const tzh_node &n) {
        nodes.push_back(n);
        return (int32_t)nodes.size() - 1;
    }

    // one leaf per distinct tensor (the same tensor used twice is read twice
    // through one leaf, as the reference's evalInto reads it twice)
    template <size_t N>
    int32_t leaf(const void *data, const Shape<N> &shape) {
        for (size_t i = 0; i < leaf_ptrs.size(); i++)
            if (leaf_ptrs[i] == data && leaves[i].ndim == (int32_t)N) {
                bool same = true;
                for (size_t d = 0; d < N; d++) same = same && leaves[i].shape[d] == shape[d];
                if (same) return (int32_t)i;
            }
        tzh_leaf l;
        std::memset(&l, 0, sizeof l);
        l.data = data;
        l.ndim = (int32_t)N;
        for (size_t i = 0; i < N; i++) l.shape[i] = shape[i];
        leaves.push_back(l);
        leaf_ptrs.push_back(data);
        return (int32_t)leaves.size() - 1;
    }
};

// -------------------------------------------------------- expression nodes
template <OpTag op, typename Input> struct UnaryExpr;
template <OpTag op, typename Lhs, typename Rhs> struct BinaryExpr;
template <typename T> struct ScalarExpr;
template <typename Input, int Axis> struct SoftmaxExpr;
template <typename Input, int... Perm> struct TransposeExpr;
template <typename Input, int64_t... Dims> struct ReshapeExpr;
template <typename Lhs, typename Rhs> struct MatmulExpr;

// Methods every expression has (expr.zig:236-316): unary ops, binary ops
// with an expression or a scalar, reductions.
template <typename Self>
struct ExprMethods {
    const Self &self() const { return static_cast<const Self &>(*this); }
#define TZH_UNARY(name) \
    UnaryExpr<OpTag::name, Self> name() const { return UnaryExpr<OpTag::name, Self>::init(self()); }
    TZH_UNARY(neg) TZH_UNARY(abs) TZH_UNARY(exp) TZH_UNARY(log) TZH_UNARY(sqrt) TZH_UNARY(rsqrt) TZH_UNARY(sin)
    TZH_UNARY(cos) TZH_UNARY(tanh) TZH_UNARY(sigmoid) TZH_UNARY(relu) TZH_UNARY(gelu) TZH_UNARY(silu)
    TZH_UNARY(softplus) TZH_UNARY(floor) TZH_UNARY(ceil) TZH_UNARY(round)
#undef TZH_UNARY
#define TZH_BINARY(name, tag)                                                                         \
    template <typename R>                                                                             \
    auto name(const R &rhs) const {                                                                   \
        if constexpr (std::is_arithmetic<R>::value) {                                                 \
            using S = ScalarExpr<typename Self::ElementType>;                                         \
            return BinaryExpr<OpTag::tag, Self, S>::init(self(), S::init((typename Self::ElementType)rhs)); \
        } else {                                                                                      \
            return BinaryExpr<OpTag::tag, Self, R>::init(self(), rhs);                                \
        }                                                                                             \
    }
    TZH_BINARY(add, add) TZH_BINARY(sub, sub) TZH_BINARY(mul, mul) TZH_BINARY(div, div) TZH_BINARY(pow, pow)
    TZH_BINARY(maximum, max) TZH_BINARY(minimum, min)
#undef TZH_BINARY
    // softmax(axis) (expr.zig:657-659); a negative axis counts from the end
    template <int Axis>
    SoftmaxExpr<Self, Axis> softmax() const { return SoftmaxExpr<Self, Axis>::init(self()); }
    // transpose(perm) (expr.zig:914-916)
    template <int... Perm>
    TransposeExpr<Self, Perm...> transpose() const { return TransposeExpr<Self, Perm...>::init(self()); }
    // reshape(target_shape) (expr.zig:918-920)
    template <int64_t... Dims>
    ReshapeExpr<Self, Dims...> reshape() const { return ReshapeExpr<Self, Dims...>::init(self()); }
    // matmul(other) (expr.zig:290-294)
    template <typename R>
    MatmulExpr<Self, R> matmul(const R &rhs) const { return MatmulExpr<Self, R>::init(self(), rhs); }
};

// A concrete tensor: Tensor(T, shape) (tensor.zig:28-249) with device data.
template <typename T, int64_t... Dims>
class Tensor : public ExprMethods<Tensor<T, Dims...>> {
  public:
    using ElementType = T;
    static constexpr NodeKind kind = NodeKind::tensor;
    static constexpr size_t ndim = sizeof...(Dims);
    static constexpr Shape<sizeof...(Dims)> shape = {Dims...};
    static constexpr int64_t count = numel(Shape<sizeof...(Dims)>{Dims...});

    Tensor() = default;
    // borrow a device buffer of `count` elements (owns_data = false)
    explicit Tensor(T *device_data) : data_(device_data), owns_(false) {}
    Tensor(Tensor &&o) noexcept : data_(o.data_), owns_(o.owns_), ctx_(o.ctx_) { o.owns_ = false; }
    Tensor &operator=(Tensor &&o) noexcept {
        if (this != &o) {
            deinit();
            data_ = o.data_;
            owns_ = o.owns_;
            ctx_ = o.ctx_;
            o.owns_ = false;
        }
        return *this;
    }
    // copies share the data without owning it (expressions hold tensors by value)
    Tensor(const Tensor &o) : data_(o.data_), owns_(false), ctx_(o.ctx_) {}
    Tensor &operator=(const Tensor &o) {
        if (this != &o) {
            deinit();
            data_ = o.data_;
            owns_ = false;
            ctx_ = o.ctx_;
        }
        return *this;
    }
    ~Tensor() { deinit(); }

    // Tensor.init: uninitialised device storage
    static Tensor init(Context &ctx) {
        Tensor t;
        void *p = nullptr;
        check(tzh_malloc(ctx.handle(), (size_t)count * sizeof(T), &p));
        t.data_ = (T *)p;
        t.owns_ = true;
        t.ctx_ = &ctx;
        return t;
    }
    // Tensor.fromSlice: copy host values (tensor.zig:84-95)
    static Tensor fromSlice(Context &ctx, const std::vector<T> &values) {
        if ((int64_t)values.size() != count) throw Error(TZH_ERR_SHAPE, "fromSlice: wrong element count");
        Tensor t = init(ctx);
        check(tzh_memcpy_h2d(ctx.handle(), t.data_, values.data(), values.size() * sizeof(T)));
        return t;
    }
    // Tensor.slice, copied back to the host
    std::vector<T> slice(Context &ctx) const {
        std::vector<T> out((size_t)count);
        check(tzh_memcpy_d2h(ctx.handle(), out.data(), data_, out.size() * sizeof(T)));
        return out;
    }
    void deinit() {
        if (owns_ && data_ && ctx_) tzh_free(ctx_->handle(), data_);
        owns_ = false;
        data_ = nullptr;
    }
    T *data() const { return data_; }

    int32_t emit(Tape &tape) const {
        tzh_node n = Tape::node_of(kind, shape);
        n.leaf = tape.leaf(data_, shape);
        return tape.push(n);
    }

  private:
    T *data_ = nullptr;
    bool owns_ = false;
    Context *ctx_ = nullptr;
};

// ScalarExpr (expr.zig:1010-1035): a rank-0 constant.
template <typename T>
struct ScalarExpr : ExprMethods<ScalarExpr<T>> {
    using ElementType = T;
    static constexpr NodeKind kind = NodeKind::constant;
    static constexpr Shape<0> shape = {};
    T value;
    static ScalarExpr init(T v) {
        ScalarExpr s;
        s.value = v;
        return s;
    }
    int32_t emit(Tape &tape) const {
        tzh_node n = Tape::node_of(kind, shape);
        n.value = (double)value;
        return tape.push(n);
    }
};

// UnaryExpr(op, Input) (expr.zig:212-349)
template <OpTag op, typename Input>
struct UnaryExpr : ExprMethods<UnaryExpr<op, Input>> {
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::unary;
    static constexpr OpTag operation = op;
    static constexpr auto shape = Input::shape;
    Input input;
    static UnaryExpr init(const Input &in) {
        UnaryExpr e;
        e.input = in;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.op = (int32_t)op;
        n.lhs = a;
        return tape.push(n);
    }
};

// BinaryExpr(op, Lhs, Rhs) (expr.zig:352-512): same element type, shapes
// broadcast.
template <OpTag op, typename Lhs, typename Rhs>
struct BinaryExpr : ExprMethods<BinaryExpr<op, Lhs, Rhs>> {
    static_assert(std::is_same<typename Lhs::ElementType, typename Rhs::ElementType>::value,
                  "BinaryExpr requires both operands to have the same element type");
    static_assert(broadcast_compatible(Lhs::shape, Rhs::shape), "Shapes not broadcast compatible");
    using ElementType = typename Lhs::ElementType;
    static constexpr NodeKind kind = NodeKind::binary;
    static constexpr OpTag operation = op;
    static constexpr auto shape = broadcast_shape(Lhs::shape, Rhs::shape);
    Lhs lhs;
    Rhs rhs;
    static BinaryExpr init(const Lhs &l, const Rhs &r) {
        BinaryExpr e;
        e.lhs = l;
        e.rhs = r;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = lhs.emit(tape);
        const int32_t b = rhs.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.op = (int32_t)op;
        n.lhs = a;
        n.rhs = b;
        return tape.push(n);
    }
};

// ReduceExpr(op, Input, axes, keepdims) (expr.zig:606-661): all axes
// (Axis = -1, `.{}` in Zig) or one axis.
template <size_t N, int Axis, bool KeepDims>
constexpr auto reduce_shape(const Shape<N> &s) {
    if constexpr (Axis < 0) {
        if constexpr (KeepDims) {
            Shape<N> out{};
            for (size_t i = 0; i < N; i++) out[i] = 1;
            return out;
        } else {
            return Shape<0>{};
        }
    } else {
        static_assert(Axis < (int)N, "reduction axis out of range");
        if constexpr (KeepDims) {
            Shape<N> out = s;
            out[Axis] = 1;
            return out;
        } else {
            Shape<N - 1> out{};
            for (size_t i = 0, j = 0; i < N; i++)
                if ((int)i != Axis) out[j++] = s[i];
            return out;
        }
    }
}

template <OpTag op, typename Input, int Axis = -1, bool KeepDims = false>
struct ReduceExpr : ExprMethods<ReduceExpr<op, Input, Axis, KeepDims>> {
    static_assert(op == OpTag::sum || op == OpTag::prod || op == OpTag::reduce_max || op == OpTag::reduce_min ||
                      op == OpTag::mean,
                  "Unsupported reduce operation");
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::reduce;
    static constexpr OpTag operation = op;
    static constexpr auto shape = reduce_shape<Input::shape.size(), Axis, KeepDims>(Input::shape);
    Input input;
    static ReduceExpr init(const Input &in) {
        ReduceExpr e;
        e.input = in;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.op = (int32_t)op;
        n.lhs = a;
        n.axis = Axis;
        n.keepdims = KeepDims ? 1 : 0;
        return tape.push(n);
    }
};

// SoftmaxExpr(Input, axis) (expr.zig:665-696)
template <typename Input, int Axis>
struct SoftmaxExpr : ExprMethods<SoftmaxExpr<Input, Axis>> {
    static constexpr int ndim = (int)Input::shape.size();
    static_assert(Axis >= -ndim && Axis < ndim, "softmax axis out of range");
    static constexpr int softmax_axis = Axis < 0 ? Axis + ndim : Axis;  // shape.normalizeAxis
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::softmax;
    static constexpr auto shape = Input::shape;
    Input input;
    static SoftmaxExpr init(const Input &in) {
        SoftmaxExpr e;
        e.input = in;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.lhs = a;
        n.axis = softmax_axis;
        return tape.push(n);
    }
};

template <size_t N>
constexpr bool is_permutation(const std::array<int, N> &p) {
    for (size_t i = 0; i < N; i++) {
        if (p[i] < 0 || p[i] >= (int)N) return false;
        for (size_t j = 0; j < i; j++)
            if (p[j] == p[i]) return false;
    }
    return true;
}

// TransposeExpr(Input, perm) (expr.zig:925-990): output axis i is input
// axis perm[i].
template <typename Input, int... Perm>
struct TransposeExpr : ExprMethods<TransposeExpr<Input, Perm...>> {
    static constexpr std::array<int, sizeof...(Perm)> perm{Perm...};
    static_assert(sizeof...(Perm) == Input::shape.size(), "Permutation length must match rank");
    static_assert(is_permutation(perm), "Invalid transpose permutation");
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::transpose;
    static constexpr Shape<sizeof...(Perm)> shape{Input::shape[Perm]...};
    Input input;
    static TransposeExpr init(const Input &in) {
        TransposeExpr e;
        e.input = in;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.lhs = a;
        for (size_t i = 0; i < perm.size(); i++) n.perm[i] = perm[i];
        return tape.push(n);
    }
};

// matmulCompatible / MatmulShape (shape.zig:206-274): the contracting
// dimensions agree; [K] @ [K] is a scalar, [K] @ [K, N] is [N], [M, K] @ [K]
// is [M], [M, K] @ [K, N] is [M, N]; otherwise both operands are matrices
// with broadcast batch dimensions in front.
template <size_t A, size_t B>
constexpr bool matmul_compatible(const Shape<A> &a, const Shape<B> &b) {
    if (A < 1 || B < 1) return false;
    return a[A - 1] == (B >= 2 ? b[B - 2] : b[0]);
}

template <size_t A, size_t B>
constexpr size_t matmul_rank() {
    return (A == 1 && B == 1) ? 0 : (A == 1 || B == 1) && A + B == 3 ? 1 : (A > B ? A : B);
}

template <size_t A, size_t B>
constexpr bool matmul_batch_ok(const Shape<A> &a, const Shape<B> &b) {
    if (A < 2 || B < 2) return A + B <= 3;  // a vector operand only with a matrix or a vector
    constexpr size_t nb = (A > B ? A : B) - 2;
    for (size_t i = 0; i < nb; i++) {
        const int64_t da = i < nb - (A - 2) ? 1 : a[i - (nb - (A - 2))];
        const int64_t db = i < nb - (B - 2) ? 1 : b[i - (nb - (B - 2))];
        if (da != db && da != 1 && db != 1) return false;
    }
    return true;
}

template <size_t A, size_t B>
constexpr Shape<matmul_rank<A, B>()> matmul_shape(const Shape<A> &a, const Shape<B> &b) {
    Shape<matmul_rank<A, B>()> out{};
    if constexpr (A == 1 && B == 2) {
        out[0] = b[1];
    } else if constexpr (A == 2 && B == 1) {
        out[0] = a[0];
    } else if constexpr (A >= 2 && B >= 2) {
        constexpr size_t nb = (A > B ? A : B) - 2;
        for (size_t i = 0; i < nb; i++) {
            const int64_t da = i < nb - (A - 2) ? 1 : a[i - (nb - (A - 2))];
            const int64_t db = i < nb - (B - 2) ? 1 : b[i - (nb - (B - 2))];
            out[i] = da > db ? da : db;
        }
        out[nb] = a[A - 2];
        out[nb + 1] = b[B - 1];
    }
    return out;
}

// MatmulExpr(Lhs, Rhs) (expr.zig:515-560): same element type, the shape
// rules above as compile-time errors.  Evaluated on the matrix cores; a
// bias add and unary ops directly above it run in its epilogue.
template <typename Lhs, typename Rhs>
struct MatmulExpr : ExprMethods<MatmulExpr<Lhs, Rhs>> {
    static_assert(std::is_same<typename Lhs::ElementType, typename Rhs::ElementType>::value,
                  "MatmulExpr requires both operands to have the same element type");
    static_assert(matmul_compatible(Lhs::shape, Rhs::shape), "Shapes not compatible for matmul");
    static_assert(matmul_batch_ok(Lhs::shape, Rhs::shape), "Batch dimensions not broadcastable in matmul");
    using ElementType = typename Lhs::ElementType;
    static constexpr NodeKind kind = NodeKind::matmul;
    static constexpr auto shape = matmul_shape(Lhs::shape, Rhs::shape);
    Lhs lhs;
    Rhs rhs;
    static MatmulExpr init(const Lhs &l, const Rhs &r) {
        MatmulExpr e;
        e.lhs = l;
        e.rhs = r;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = lhs.emit(tape);
        const int32_t b = rhs.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.lhs = a;
        n.rhs = b;
        return tape.push(n);
    }
};

// ReshapeExpr(Input, target_shape): the same elements under another shape.
template <typename Input, int64_t... Dims>
struct ReshapeExpr : ExprMethods<ReshapeExpr<Input, Dims...>> {
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::reshape;
    static constexpr Shape<sizeof...(Dims)> shape{Dims...};
    static_assert(numel(shape) == numel(Input::shape), "Reshape must preserve the element count");
    Input input;
    static ReshapeExpr init(const Input &in) {
        ReshapeExpr e;
        e.input = in;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.lhs = a;
        return tape.push(n);
    }
};

// LayerNormExpr(Input, Gamma, Beta, norm_dims) (expr.zig:705-760)
template <typename Input, typename Gamma, typename Beta, int NormDims = 1>
struct LayerNormExpr : ExprMethods<LayerNormExpr<Input, Gamma, Beta, NormDims>> {
    static constexpr int ndim = (int)Input::shape.size();
    static_assert(NormDims >= 1 && NormDims <= ndim, "norm_dims out of range");
    static_assert((int)Gamma::shape.size() == NormDims && (int)Beta::shape.size() == NormDims,
                  "Gamma/beta rank must equal normalized_dims");
    static constexpr bool params_match() {
        for (int i = 0; i < NormDims; i++)
            if (Gamma::shape[i] != Input::shape[ndim - NormDims + i] || Beta::shape[i] != Gamma::shape[i])
                return false;
        return true;
    }
    static_assert(params_match(), "Gamma/beta shape must match last dimensions of input");
    using ElementType = typename Input::ElementType;
    static constexpr NodeKind kind = NodeKind::layernorm;
    static constexpr auto shape = Input::shape;
    Input input;
    Gamma gamma;
    Beta beta;
    static LayerNormExpr init(const Input &in, const Gamma &g, const Beta &b) {
        LayerNormExpr e;
        e.input = in;
        e.gamma = g;
        e.beta = b;
        return e;
    }
    int32_t emit(Tape &tape) const {
        const int32_t a = input.emit(tape), g = gamma.emit(tape), b = beta.emit(tape);
        tzh_node n = Tape::node_of(kind, shape);
        n.lhs = a;
        n.rhs = g;
        n.aux = b;
        n.axis = NormDims;
        return tape.push(n);
    }
};

// ---------------------------------------------------------- evaluation
template <typename T, typename ShapeArr, size_t... I>
auto tensor_type_for(std::index_sequence<I...>) -> Tensor<T, ShapeArr::value[I]...>;

template <typename Expr>
struct ShapeOf {
    static constexpr auto value = Expr::shape;
};

// Tensor type of an expression's result (Tensor(Expr.ElementType, Expr.shape))
template <typename Expr>
using ResultTensor = decltype(tensor_type_for<typename Expr::ElementType, ShapeOf<Expr>>(
    std::make_index_sequence<Expr::shape.size()>{}));

// executor.evalInto (executor.zig:49-54): out is device memory of the
// expression's shape.
template <typename Expr>
void evalInto(Context &ctx, const Expr &expr, typename Expr::ElementType *out) {
    Tape tape;
    expr.emit(tape);
    check(tzh_eval_into(ctx.handle(), tape.nodes.data(), (int32_t)tape.nodes.size(),
                        tape.leaves.empty() ? nullptr : tape.leaves.data(), (int32_t)tape.leaves.size(),
                        dtype_of<typename Expr::ElementType>(), out));
}

// executor.eval (executor.zig:29-45): allocate the result, evalInto it.
template <typename Expr>
ResultTensor<Expr> eval(Context &ctx, const Expr &expr) {
    auto out = ResultTensor<Expr>::init(ctx);
    evalInto(ctx, expr, out.data());
    return out;
}

// ------------------------------------------------------------- Arctic
namespace arctic {

// arctic.Config (arctic.zig:29-42)
inline tzh_arctic_config default_config() {
    tzh_arctic_config c;
    c.hidden_size = 384;
    c.num_hidden_layers = 6;
    c.num_attention_heads = 12;
    c.intermediate_size = 1536;
    c.vocab_size = 30522;
    c.max_position_embeddings = 512;
    c.type_vocab_size = 2;
    c.layer_norm_eps = 1e-12f;
    return c;
}

// arctic.ModelWeights (arctic.zig:100-178), resident in HBM.
class ModelWeights {
  public:
    ModelWeights() = default;
    ModelWeights(ModelWeights &&o) noexcept : h_(o.h_) { o.h_ = nullptr; }
    ModelWeights &operator=(ModelWeights &&o) noexcept {
        if (this != &o) {
            deinit();
            h_ = o.h_;
            o.h_ = nullptr;
        }
        return *this;
    }
    ModelWeights(const ModelWeights &) = delete;
    ~ModelWeights() { deinit(); }

    static ModelWeights fromSafeTensors(Context &ctx, const std::string &path,
                                        const tzh_arctic_config &config = default_config()) {
        ModelWeights w;
        check(tzh_arctic_load_safetensors(ctx.handle(), path.c_str(), &config, &w.h_));
        return w;
    }
    static ModelWeights fromHost(Context &ctx, const tzh_arctic_weights &host) {
        ModelWeights w;
        check(tzh_arctic_upload(ctx.handle(), &host, &w.h_));
        return w;
    }
    void deinit() {
        if (h_) tzh_arctic_free(h_);
        h_ = nullptr;
    }
    tzh_model *handle() const { return h_; }

  private:
    tzh_model *h_ = nullptr;
};

// arctic.forward (arctic.zig:874-898): one sequence of device ids ->
// L2-normalised CLS embedding (device f32 [hidden]).
inline void forward(float *output, const uint32_t *token_ids, int64_t seq_len, const ModelWeights &weights) {
    check(tzh_arctic_forward(weights.handle(), output, token_ids, seq_len));
}

// arctic.forwardBatchParallel (arctic.zig:959-1013): ragged batch.  ids are
// device u32, packed (stride 0) or padded [batch, stride]; lengths on the
// host; outputs device f32 [batch, hidden].
inline void forwardBatch(float *outputs, const uint32_t *ids, const std::vector<int32_t> &lengths, int64_t stride,
                         const ModelWeights &weights) {
    check(tzh_arctic_forward_batch(weights.handle(), outputs, ids, lengths.data(), (int32_t)lengths.size(), stride));
}

// arctic.feedForward (arctic.zig:760-811) of encoder layer `layer`: device
// f32 input and output [seq_len, hidden] (distinct buffers), f32 arithmetic.
inline void feedForward(float *output, const float *input, const ModelWeights &weights, int32_t layer,
                        int64_t seq_len) {
    check(tzh_arctic_feed_forward(weights.handle(), layer, input, output, seq_len));
}

// The embed command's document path (main.zig:786-933) for several
// documents: outputs device f32 [texts.size(), hidden]; returns each
// document's chunk count.
inline std::vector<int32_t> embedDocuments(float *outputs, const std::vector<std::string> &texts,
                                           const tzh_tokenizer *tok, const ModelWeights &weights) {
    std::vector<const char *> ptrs;
    std::vector<int64_t> lens;
    for (const auto &t : texts) {
        ptrs.push_back(t.data());
        lens.push_back((int64_t)t.size());
    }
    std::vector<int32_t> counts(texts.size());
    check(tzh_arctic_embed_documents(weights.handle(), tok, ptrs.data(), lens.data(), (int32_t)texts.size(), outputs,
                                     counts.data()));
    return counts;
}

}  // namespace arctic

namespace io {

// io/tokenizer.Tokenizer (tokenizer.zig:9-285).
class Tokenizer {
  public:
    static constexpr uint32_t unk_id = 100, cls_id = 101, sep_id = 102;

    Tokenizer() { check(tzh_tokenizer_create(&h_)); }  // Tokenizer.init
    Tokenizer(const Tokenizer &) = delete;
    ~Tokenizer() { tzh_tokenizer_free(h_); }

    void loadVocab(const std::string &path) { check(tzh_tokenizer_load_vocab(h_, path.c_str())); }
    void loadVocabFromBytes(const std::string &data) {
        check(tzh_tokenizer_load_vocab_bytes(h_, data.data(), (int64_t)data.size()));
    }
    // vocab.put(token, id), as the reference's tests build vocabularies
    void put(const std::string &token, uint32_t id) {
        check(tzh_tokenizer_put(h_, token.data(), (int64_t)token.size(), id));
    }
    // [CLS] ... [SEP] into output (size >= 2); returns the id count
    size_t encode(const std::string &text, uint32_t *output, size_t capacity) const {
        int64_t n = 0;
        check(tzh_tokenizer_encode(h_, text.data(), (int64_t)text.size(), output, (int64_t)capacity, &n));
        return (size_t)n;
    }
    std::vector<uint32_t> encodeRaw(const std::string &text) const {
        int64_t n = 0;
        const int rc = tzh_tokenizer_encode_raw(h_, text.data(), (int64_t)text.size(), nullptr, 0, &n);
        if (rc != TZH_OK && rc != TZH_ERR_TOO_LARGE) check(rc);
        std::vector<uint32_t> out((size_t)n);
        check(tzh_tokenizer_encode_raw(h_, text.data(), (int64_t)text.size(), out.data(), n, &n));
        return out;
    }
    const tzh_tokenizer *handle() const { return h_; }

  private:
    tzh_tokenizer *h_ = nullptr;
};

}  // namespace io
}  // namespace tenzor
