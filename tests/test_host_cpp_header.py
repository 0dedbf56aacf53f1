"""The C++ host API header (tenzor_amd/host/tenzor.hpp) on the CPU: it
compiles, and the compile-time checks the reference makes with
@compileError (expr.zig:358-376: same element type, broadcastable shapes;
reduce axis in range) are compile errors here too."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "tenzor_amd", "host", "tenzor.hpp")

PRELUDE = f'#include "{HDR}"\nusing namespace tenzor;\n'


def compile_snippet(body: str, tmp_path):
    src = tmp_path / "snippet.cpp"
    src.write_text(PRELUDE + "void f(Context &ctx) {\n" + body + "\n}\n")
    return subprocess.run(["g++", "-std=c++17", "-fsyntax-only", str(src)], capture_output=True, text=True)


def test_header_compiles_with_the_reference_surface(tmp_path):
    res = compile_snippet("""
        using Mat = Tensor<float, 4, 8>;
        using Row = Tensor<float, 8>;
        auto a = Mat::fromSlice(ctx, std::vector<float>(32, 1.0f));
        auto b = Row::fromSlice(ctx, std::vector<float>(8, 2.0f));
        auto e = BinaryExpr<OpTag::add, Mat, Row>::init(a, b).mul(a).exp().relu().add(1.0);
        static_assert(decltype(e)::shape.size() == 2 && decltype(e)::shape[1] == 8, "shape");
        auto r = eval(ctx, e);
        auto s = eval(ctx, ReduceExpr<OpTag::sum, decltype(e), 1, true>::init(e));
        static_assert(decltype(s)::shape[0] == 4 && decltype(s)::shape[1] == 1, "reduced shape");
        evalInto(ctx, e, r.data());
        // MatmulShape (shape.zig:221-274) at compile time
        Tensor<float, 8, 5> bm;
        auto mm = a.matmul(bm).add(Tensor<float, 5>{}).relu();
        static_assert(decltype(mm)::shape.size() == 2 && decltype(mm)::shape[0] == 4 && decltype(mm)::shape[1] == 5, "mm");
        Tensor<float, 3, 1, 4, 8> ba;
        Tensor<float, 2, 8, 6> bb;
        auto bmm = ba.matmul(bb);
        constexpr auto bs = decltype(bmm)::shape;
        static_assert(bs.size() == 4 && bs[0] == 3 && bs[1] == 2 && bs[2] == 4 && bs[3] == 6, "batched matmul shape");
        auto mv = a.matmul(b);
        static_assert(decltype(mv)::shape.size() == 1 && decltype(mv)::shape[0] == 4, "matrix-vector shape");
        auto vv = b.matmul(b);
        static_assert(decltype(vv)::shape.size() == 0, "vector-vector is a scalar");
        auto w = arctic::ModelWeights::fromSafeTensors(ctx, "m.safetensors");
        std::vector<int32_t> lengths{3};
        arctic::forwardBatch(nullptr, nullptr, lengths, 0, w);
    """, tmp_path)
    assert res.returncode == 0, res.stderr


@pytest.mark.parametrize("body,message", [
    ("Tensor<float, 2, 3> a; Tensor<float, 4> b; auto e = a.add(b); (void)e;", "Shapes not broadcast compatible"),
    ("Tensor<float, 3> a; Tensor<double, 3> b; auto e = BinaryExpr<OpTag::add, Tensor<float, 3>, Tensor<double, 3>>"
     "::init(a, b); (void)e;", "same element type"),
    ("Tensor<float, 2, 3> a; auto e = ReduceExpr<OpTag::sum, Tensor<float, 2, 3>, 2>::init(a); (void)e;",
     "reduction axis out of range"),
    ("Tensor<float, 3> a; auto e = ReduceExpr<OpTag::add, Tensor<float, 3>>::init(a); (void)e;",
     "Unsupported reduce operation"),
    # expr.zig:932-952 and 705-735
    ("Tensor<float, 2, 3> a; auto e = a.transpose<0, 0>(); (void)e;", "Invalid transpose permutation"),
    ("Tensor<float, 2, 3> a; auto e = a.transpose<1, 0, 2>(); (void)e;", "Permutation length must match rank"),
    ("Tensor<float, 2, 3> a; Tensor<float, 4> g; auto e = LayerNormExpr<Tensor<float, 2, 3>, Tensor<float, 4>, "
     "Tensor<float, 4>, 1>::init(a, g, g); (void)e;", "Gamma/beta shape must match last dimensions of input"),
    ("Tensor<float, 2, 3> a; auto e = a.softmax<2>(); (void)e;", "softmax axis out of range"),
    ("Tensor<float, 2, 3> a; auto e = a.reshape<4, 2>(); (void)e;", "Reshape must preserve the element count"),
    # shape.zig:206-216, 256-261
    ("Tensor<float, 2, 3> a; Tensor<float, 4, 5> b; auto e = a.matmul(b); (void)e;", "Shapes not compatible for matmul"),
    ("Tensor<float, 2, 4, 3> a; Tensor<float, 3, 3, 5> b; auto e = a.matmul(b); (void)e;",
     "Batch dimensions not broadcastable in matmul"),
    ("Tensor<float, 4, 3> a; Tensor<double, 3, 5> b; auto e = MatmulExpr<Tensor<float, 4, 3>, Tensor<double, 3, 5>>"
     "::init(a, b); (void)e;", "same element type"),
])
def test_compile_time_errors_mirror_comptime_errors(tmp_path, body, message):
    res = compile_snippet(body, tmp_path)
    assert res.returncode != 0
    assert message in res.stderr, res.stderr[-2000:]
