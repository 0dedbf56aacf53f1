// Programs of the elementwise engine (K1): the descriptor the interpreter
// kernels in ew.hip execute and the chain-kernel generator (ew_jit.cpp)
// specialises into straight-line code.
#pragma once

#include "common.h"

namespace tzh_ew {

constexpr int kMaxNodes = 32;  // analyzer.zig:13 MAX_ELEMENTWISE_OPS
constexpr int kMaxLeaves = 12;
constexpr int kMaxDepth = 4;   // value stack slots per thread

enum : int16_t { EK_LEAF = 0, EK_CONST = 1, EK_UNARY = 2, EK_BINARY = 3 };
enum : int32_t { VEC_PER_ELEM = 0, VEC_CONTIG = 1, VEC_SPLAT = 2 };

#define TZH_EW_SHARED(...) __VA_ARGS__
#include "ew_shared.inc"
#undef TZH_EW_SHARED

static_assert(TZH_MAX_RANK == 8 && kMaxNodes == 32 && kMaxLeaves == 12,
              "array bounds in ew_shared.inc are written as literals");
static_assert(sizeof(EwProgram) < 3800, "kernel argument block too large");

FastDiv make_fastdiv(uint64_t d);

// The unary ops unary_op<T> implements (simd.zig:107-315).
inline bool unary_ok(int op) {
    switch (op) {
    case TZH_OP_NEG: case TZH_OP_ABS: case TZH_OP_EXP: case TZH_OP_LOG: case TZH_OP_SQRT:
    case TZH_OP_RSQRT: case TZH_OP_SIN: case TZH_OP_COS: case TZH_OP_TANH: case TZH_OP_SIGMOID:
    case TZH_OP_RELU: case TZH_OP_GELU: case TZH_OP_SILU: case TZH_OP_SOFTPLUS:
    case TZH_OP_FLOOR: case TZH_OP_CEIL: case TZH_OP_ROUND:
        return true;
    default:
        return false;
    }
}

// Launch the generated single-pass kernel for chain program p (no reduce
// node) writing p.numel elements of type f64 ? double : float to out, with
// V outputs per thread and `grid` blocks of 256 threads; kernels are
// compiled on first use of a program shape and cached per device.
int jit_chain_launch(tzh_ctx *ctx, const EwProgram &p, bool f64, int V, int grid, void *out);

}  // namespace tzh_ew
