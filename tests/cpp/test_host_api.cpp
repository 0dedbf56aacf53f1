// GPU parity of the C++ host API (tenzor_amd/host/tenzor.hpp), written as
// the reference writes its tests: the executor known answers
// (executor.zig:605-740), broadcasting and scalars (elementwise.zig:339-460),
// reductions (reduce.zig:241-350), config-2 chains against the oracle, and
// the Arctic integration flow (arctic_integration_test.zig: safetensors +
// token file -> embeddings) against expected embeddings computed by the
// oracle.  Test infrastructure: links the CPU oracle as the checker.
//
//   test_host_api [fixture_dir]     (fixture_dir: model.safetensors, ids.bin,
//                                    lengths.bin, expected.bin)
#include <cmath>
#include <cstdio>
#include <fstream>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "../../oracle/oracle.h"
#include "../../tenzor_amd/host/tenzor.hpp"

using namespace tenzor;

static int g_failed = 0;

#define EXPECT(cond)                                                                                 \
    do {                                                                                             \
        if (!(cond)) throw std::runtime_error(std::string("expectation failed: ") + #cond + " line " + \
                                              std::to_string(__LINE__));                             \
    } while (0)

static void run(const char *name, const std::function<void()> &fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception &e) {
        std::printf("FAIL %s: %s\n", name, e.what());
        g_failed++;
    }
    std::fflush(stdout);
}

static int64_t ulp_diff(float a, float b) {
    int32_t ia, ib;
    std::memcpy(&ia, &a, 4);
    std::memcpy(&ib, &b, 4);
    int64_t x = ia < 0 ? (int64_t)INT32_MIN - ia : ia;
    int64_t y = ib < 0 ? (int64_t)INT32_MIN - ib : ib;
    return x > y ? x - y : y - x;
}

template <typename T>
static std::vector<T> read_file(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    f.seekg(0, std::ios::end);
    const size_t n = (size_t)f.tellg() / sizeof(T);
    f.seekg(0);
    std::vector<T> v(n);
    f.read((char *)v.data(), (std::streamsize)(n * sizeof(T)));
    return v;
}

int main(int argc, char **argv) {
    Context ctx(0);

    run("eval tensor passthrough", [&] {  // executor.zig:605-614
        using Vec = Tensor<float, 4>;
        auto input = Vec::fromSlice(ctx, {1, 2, 3, 4});
        auto result = eval(ctx, input);
        EXPECT(result.slice(ctx) == input.slice(ctx));
    });

    run("eval unary relu", [&] {  // executor.zig:616-631
        using Vec = Tensor<float, 4>;
        auto input = Vec::fromSlice(ctx, {-2, -1, 1, 2});
        auto expr = UnaryExpr<OpTag::relu, Vec>::init(input);
        auto result = eval(ctx, expr).slice(ctx);
        const float expected[] = {0, 0, 1, 2};
        for (int i = 0; i < 4; i++) EXPECT(std::fabs(result[i] - expected[i]) <= 1e-6f);
    });

    run("eval binary add", [&] {  // executor.zig:633-650
        using Vec = Tensor<float, 4>;
        auto a = Vec::fromSlice(ctx, {1, 2, 3, 4});
        auto b = Vec::fromSlice(ctx, {10, 20, 30, 40});
        auto expr = BinaryExpr<OpTag::add, Vec, Vec>::init(a, b);
        EXPECT((eval(ctx, expr).slice(ctx) == std::vector<float>{11, 22, 33, 44}));
    });

    run("eval chained expression", [&] {  // executor.zig:652-673
        using Vec = Tensor<float, 4>;
        auto a = Vec::fromSlice(ctx, {-1, 2, -3, 4});
        auto b = Vec::fromSlice(ctx, {1, 1, 1, 1});
        using AddExpr = BinaryExpr<OpTag::add, Vec, Vec>;
        auto relu_expr = UnaryExpr<OpTag::relu, AddExpr>::init(AddExpr::init(a, b));
        EXPECT((eval(ctx, relu_expr).slice(ctx) == std::vector<float>{0, 3, 0, 5}));
    });

    run("eval reduce sum", [&] {  // executor.zig:694-706
        using Vec = Tensor<float, 4>;
        auto input = Vec::fromSlice(ctx, {1, 2, 3, 4});
        auto s = eval(ctx, ReduceExpr<OpTag::sum, Vec>::init(input)).slice(ctx);
        EXPECT(s.size() == 1 && s[0] == 10.0f);
    });

    run("reduce along an axis", [&] {  // reduce.zig:283-300
        using Mat = Tensor<float, 2, 3>;
        auto m = Mat::fromSlice(ctx, {1, 2, 3, 4, 5, 6});
        EXPECT((eval(ctx, ReduceExpr<OpTag::sum, Mat, 1>::init(m)).slice(ctx) == std::vector<float>{6, 15}));
        EXPECT((eval(ctx, ReduceExpr<OpTag::sum, Mat, 0>::init(m)).slice(ctx) == std::vector<float>{5, 7, 9}));
        EXPECT((eval(ctx, ReduceExpr<OpTag::mean, Mat, 1, true>::init(m)).slice(ctx) == std::vector<float>{2, 5}));
        EXPECT((eval(ctx, ReduceExpr<OpTag::reduce_max, Mat, 0>::init(m)).slice(ctx) ==
                std::vector<float>{4, 5, 6}));
    });

    run("broadcast row and column", [&] {  // strides.zig:92-121 stride-0 rule
        using Mat = Tensor<float, 2, 3>;
        using Row = Tensor<float, 3>;
        using Col = Tensor<float, 2, 1>;
        auto m = Mat::fromSlice(ctx, {1, 2, 3, 4, 5, 6});
        auto r = Row::fromSlice(ctx, {10, 20, 30});
        auto c = Col::fromSlice(ctx, {100, 200});
        auto e = m.add(r).add(c);
        static_assert(decltype(e)::shape[0] == 2 && decltype(e)::shape[1] == 3, "broadcast shape");
        EXPECT((eval(ctx, e).slice(ctx) == std::vector<float>{111, 122, 133, 214, 225, 236}));
    });

    run("scalar operands", [&] {  // ScalarExpr, expr.zig:1010-1063
        using Vec = Tensor<float, 5>;
        auto x = Vec::fromSlice(ctx, {-2, -0.5f, 0, 0.5f, 2});
        auto r = eval(ctx, x.mul(2.5).add(-1.0).maximum(0.0)).slice(ctx);
        const float expected[] = {0, 0, 0, 0.25f, 4.0f};
        for (int i = 0; i < 5; i++) EXPECT(r[i] == expected[i]);
    });

    run("matmul with a fused bias + relu epilogue", [&] {  // codegen.zig:330-347
        using Mat = Tensor<float, 2, 2>;
        using Row = Tensor<float, 2>;
        auto a = Mat::fromSlice(ctx, {1, 2, 3, 4});
        auto eye = Mat::fromSlice(ctx, {1, 0, 0, 1});
        auto bias = Row::fromSlice(ctx, {-10, 10});
        EXPECT((eval(ctx, a.matmul(eye).add(bias).relu()).slice(ctx) == std::vector<float>{0, 12, 0, 14}));
    });

    run("batched and vector matmul shapes", [&] {  // shape.zig:206-274
        using Batch = Tensor<float, 2, 1, 3>;
        using Mat = Tensor<float, 3, 2>;
        using Vec = Tensor<float, 3>;
        auto a = Batch::fromSlice(ctx, {1, 2, 3, 4, 5, 6});
        auto b = Mat::fromSlice(ctx, {1, 0, 0, 1, 1, 1});
        auto v = Vec::fromSlice(ctx, {1, 1, 1});
        auto ab = a.matmul(b);
        static_assert(decltype(ab)::shape.size() == 3 && decltype(ab)::shape[0] == 2 &&
                          decltype(ab)::shape[1] == 1 && decltype(ab)::shape[2] == 2,
                      "batched shape");
        EXPECT((eval(ctx, ab).slice(ctx) == std::vector<float>{4, 5, 10, 11}));
        auto vb = v.matmul(b);  // [3] @ [3, 2] -> [2]
        EXPECT((eval(ctx, vb).slice(ctx) == std::vector<float>{2, 2}));
        auto vv = eval(ctx, v.matmul(v)).slice(ctx);  // [3] @ [3] -> scalar
        EXPECT(vv.size() == 1 && vv[0] == 3.0f);
    });

    run("config-2 chain exp((A + b) * c) vs oracle", [&] {
        constexpr int64_t R = 512, C = 4096;
        using Mat = Tensor<float, R, C>;
        using Row = Tensor<float, C>;
        std::mt19937 gen(11);
        std::uniform_real_distribution<float> u(-1.0f, 1.0f);
        std::vector<float> ha(R * C), hb(C), hc(R * C), ref(R * C), t1(R * C), t2(R * C);
        for (auto &v : ha) v = u(gen);
        for (auto &v : hb) v = u(gen);
        for (auto &v : hc) v = u(gen);
        auto a = Mat::fromSlice(ctx, ha);
        auto b = Row::fromSlice(ctx, hb);
        auto c = Mat::fromSlice(ctx, hc);
        auto out = eval(ctx, BinaryExpr<OpTag::add, Mat, Row>::init(a, b).mul(c).exp()).slice(ctx);
        orc_chain_add_mul_exp(ha.data(), hb.data(), hc.data(), ref.data(), R, C, t1.data(), t2.data());
        int64_t worst = 0;
        for (size_t i = 0; i < out.size(); i++) worst = std::max(worst, ulp_diff(out[i], ref[i]));
        EXPECT(worst <= 2);
    });

    run("f64 chain vs oracle executor", [&] {
        using Mat = Tensor<double, 17, 31>;
        using Row = Tensor<double, 31>;
        std::mt19937 gen(7);
        std::normal_distribution<double> n01;
        std::vector<double> ha(17 * 31), hb(31);
        for (auto &v : ha) v = n01(gen);
        for (auto &v : hb) v = n01(gen);
        auto a = Mat::fromSlice(ctx, ha);
        auto b = Row::fromSlice(ctx, hb);
        auto e = BinaryExpr<OpTag::add, Mat, Row>::init(a, b).exp().mul(a);
        auto got = eval(ctx, e).slice(ctx);
        // the oracle evaluates the same tape over host copies of the leaves
        Tape tape;
        e.emit(tape);
        std::vector<tzh_leaf> host = tape.leaves;
        host[0].data = ha.data();
        host[1].data = hb.data();
        std::vector<double> ref(got.size());
        EXPECT(orc_eval(tape.nodes.data(), (int32_t)tape.nodes.size(), host.data(), (int32_t)host.size(), TZH_F64,
                        ref.data()) == 0);
        for (size_t i = 0; i < got.size(); i++) EXPECT(std::fabs(got[i] - ref[i]) <= 1e-14 * std::fabs(ref[i]) + 1e-15);
    });

    run("errors carry the reference's error names", [&] {
        using Vec = Tensor<float, 4>;
        auto x = Vec::fromSlice(ctx, {1, 2, 3, 4});
        try {
            evalInto(ctx, x.exp(), (float *)nullptr);
            EXPECT(false);
        } catch (const Error &e) {
            EXPECT(e.code == TZH_ERR_INVALID_ARGS);
        }
        try {
            (void)arctic::ModelWeights::fromSafeTensors(ctx, "/nonexistent/model.safetensors");
            EXPECT(false);
        } catch (const Error &e) {
            EXPECT(e.code == TZH_ERR_IO);
        }
    });

    run("softmax, transpose, reshape, layernorm nodes", [&] {  // executor.zig:876-1030
        using Mat = Tensor<float, 2, 3>;
        auto x = Mat::fromSlice(ctx, {1, 2, 3, 0, 0, 0});
        const auto s = eval(ctx, x.softmax<-1>()).slice(ctx);
        EXPECT(std::fabs(s[0] + s[1] + s[2] - 1.0f) < 1e-5f && std::fabs(s[3] - 1.0f / 3.0f) < 1e-5f);
        const auto t = eval(ctx, x.transpose<1, 0>()).slice(ctx);
        EXPECT(t == std::vector<float>({1, 0, 2, 0, 3, 0}));
        const auto r = eval(ctx, x.reshape<3, 2>().add(1.0f)).slice(ctx);
        EXPECT(r == std::vector<float>({2, 3, 4, 1, 1, 1}));
        using Row = Tensor<float, 3>;
        auto g = Row::fromSlice(ctx, {1, 1, 1});
        auto b = Row::fromSlice(ctx, {0, 0, 0});
        auto y = Mat::fromSlice(ctx, {1, 2, 3, 10, 20, 30});
        const auto l = eval(ctx, LayerNormExpr<Mat, Row, Row, 1>::init(y, g, b)).slice(ctx);
        EXPECT(std::fabs(l[0] + l[1] + l[2]) < 1e-5f && std::fabs(l[0] - l[3]) < 1e-5f);
    });

    // the reference's tokenizer tests (tokenizer.zig:291-437): vocabulary
    // entries put directly, output capacity 32
    run("tokenizer: the reference's known answers", [&] {
        struct Case {
            std::vector<std::pair<std::string, uint32_t>> vocab;
            std::string text;
            std::vector<uint32_t> expected;
        };
        const std::vector<std::pair<std::string, uint32_t>> special = {{"[UNK]", 100}, {"[CLS]", 101}, {"[SEP]", 102}};
        std::vector<Case> cases = {
            {{{"[PAD]", 0}, {"hello", 7592}, {"world", 2088}, {"##ing", 2075}, {"test", 3231}, {"##s", 1055}},
             "hello world", {101, 7592, 2088, 102}},
            {{{"test", 3231}, {"##ing", 2075}}, "testing", {101, 3231, 2075, 102}},
            {{{"hello", 7592}}, "xyz", {101, 100, 102}},
            {{{"hello", 7592}, {",", 1010}, {"world", 2088}}, "hello, world", {101, 7592, 1010, 2088, 102}},
            {{{"hello", 7592}}, "HELLO", {101, 7592, 102}},
        };
        for (const auto &c : cases) {
            io::Tokenizer tok;
            for (const auto &e : special) tok.put(e.first, e.second);
            for (const auto &e : c.vocab) tok.put(e.first, e.second);
            uint32_t out[32];
            const size_t n = tok.encode(c.text, out, 32);
            EXPECT(std::vector<uint32_t>(out, out + n) == c.expected);
            const auto raw = tok.encodeRaw(c.text);
            EXPECT(std::vector<uint32_t>(c.expected.begin() + 1, c.expected.end() - 1) == raw);
        }
    });

    if (argc > 1) {
        const std::string dir = argv[1];
        run("embed documents: vocab.txt + text -> pooled chunk embeddings", [&] {  // main.zig:786-933
            auto weights = arctic::ModelWeights::fromSafeTensors(ctx, dir + "/model.safetensors");
            io::Tokenizer tok;
            tok.loadVocab(dir + "/vocab.txt");
            const auto text = read_file<char>(dir + "/doc.txt");
            const std::string doc(text.begin(), text.end());
            const auto chunk_ids = read_file<uint32_t>(dir + "/chunk_ids.bin");   // the oracle's chunks
            const auto chunk_lens = read_file<int32_t>(dir + "/chunk_lens.bin");
            const size_t nc = chunk_lens.size();
            EXPECT(nc >= 2);
            // the library's own tokenizer gives the oracle's pieces
            const auto pieces = tok.encodeRaw(doc);
            int64_t planned = 0;
            check(tzh_embed_chunk_count((int64_t)pieces.size(), &planned));
            EXPECT(planned == (int64_t)nc);
            EXPECT(std::vector<uint32_t>(chunk_ids.begin() + 1, chunk_ids.begin() + chunk_lens[0] - 1) ==
                   std::vector<uint32_t>(pieces.begin(), pieces.begin() + chunk_lens[0] - 2));
            void *d_out = nullptr, *d_ids = nullptr, *d_chunks = nullptr;
            check(tzh_malloc(ctx.handle(), 384 * 4, &d_out));
            check(tzh_malloc(ctx.handle(), chunk_ids.size() * 4, &d_ids));
            check(tzh_malloc(ctx.handle(), nc * 384 * 4, &d_chunks));
            const auto counts = arctic::embedDocuments((float *)d_out, {doc}, tok.handle(), weights);
            EXPECT(counts.size() == 1 && (size_t)counts[0] == nc);
            std::vector<float> got(384), emb(nc * 384);
            check(tzh_memcpy_d2h(ctx.handle(), got.data(), d_out, 384 * 4));
            check(tzh_memcpy_h2d(ctx.handle(), d_ids, chunk_ids.data(), chunk_ids.size() * 4));
            arctic::forwardBatch((float *)d_chunks, (const uint32_t *)d_ids, chunk_lens, 0, weights);
            check(tzh_memcpy_d2h(ctx.handle(), emb.data(), d_chunks, emb.size() * 4));
            tzh_free(ctx.handle(), d_out);
            tzh_free(ctx.handle(), d_ids);
            tzh_free(ctx.handle(), d_chunks);
            // main.zig:908-923 in its order, on the same chunk embeddings
            float mean[384] = {}, norm = 0.0f;
            for (size_t c = 0; c < nc; c++)
                for (int j = 0; j < 384; j++) mean[j] += emb[c * 384 + j];
            const float scale = 1.0f / (float)nc;
            for (int j = 0; j < 384; j++) mean[j] *= scale;
            for (int j = 0; j < 384; j++) {
                const float sq = mean[j] * mean[j];
                norm += sq;
            }
            norm = std::sqrt(norm);
            for (int j = 0; j < 384; j++) EXPECT(got[j] == (norm > 0 ? mean[j] / norm : mean[j]));
        });
        run("arctic integration: safetensors + tokens -> embeddings", [&] {  // arctic_integration_test.zig
            auto weights = arctic::ModelWeights::fromSafeTensors(ctx, dir + "/model.safetensors");
            const auto ids = read_file<uint32_t>(dir + "/ids.bin");
            const auto lengths = read_file<int32_t>(dir + "/lengths.bin");
            const auto expected = read_file<float>(dir + "/expected.bin");
            const size_t batch = lengths.size();
            EXPECT(expected.size() == batch * 384);
            void *d_ids = nullptr, *d_out = nullptr;
            check(tzh_malloc(ctx.handle(), ids.size() * 4, &d_ids));
            check(tzh_malloc(ctx.handle(), expected.size() * 4, &d_out));
            check(tzh_memcpy_h2d(ctx.handle(), d_ids, ids.data(), ids.size() * 4));
            arctic::forwardBatch((float *)d_out, (const uint32_t *)d_ids, lengths, 0, weights);
            std::vector<float> got(expected.size());
            check(tzh_memcpy_d2h(ctx.handle(), got.data(), d_out, got.size() * 4));
            // single-sequence entry point on the first sequence
            std::vector<float> one(384);
            arctic::forward((float *)d_out, (const uint32_t *)d_ids, lengths[0], weights);
            check(tzh_memcpy_d2h(ctx.handle(), one.data(), d_out, 384 * 4));
            tzh_free(ctx.handle(), d_ids);
            tzh_free(ctx.handle(), d_out);
            double max_abs = 0, min_cos = 1;
            for (size_t b = 0; b < batch; b++) {
                double dot = 0, ng = 0, nr = 0;
                for (int j = 0; j < 384; j++) {
                    const double g = got[b * 384 + j], r = expected[b * 384 + j];
                    max_abs = std::max(max_abs, std::fabs(g - r));
                    dot += g * r;
                    ng += g * g;
                    nr += r * r;
                }
                min_cos = std::min(min_cos, dot / std::sqrt(ng * nr));
            }
            std::printf("  arctic: %zu sequences, max-abs %.3g, min cosine %.7f\n", batch, max_abs, min_cos);
            EXPECT(max_abs <= 1e-3 && min_cos >= 0.9999);
            for (int j = 0; j < 384; j++) EXPECT(one[j] == got[j]);  // same kernels, same sums
        });
        run("arctic feed-forward: one kernel = the GEMM pair to f32 rounding", [&] {  // arctic.zig:760-811
            auto weights = arctic::ModelWeights::fromSafeTensors(ctx, dir + "/model.safetensors");
            const int64_t n = 100;
            std::vector<float> x((size_t)n * 384);
            for (size_t i = 0; i < x.size(); i++) x[i] = std::sin(0.37f * (float)i) * 1.5f;
            void *d_x = nullptr, *d_y = nullptr, *d_z = nullptr;
            check(tzh_malloc(ctx.handle(), x.size() * 4, &d_x));
            check(tzh_malloc(ctx.handle(), x.size() * 4, &d_y));
            check(tzh_malloc(ctx.handle(), x.size() * 4, &d_z));
            check(tzh_memcpy_h2d(ctx.handle(), d_x, x.data(), x.size() * 4));
            arctic::feedForward((float *)d_y, (const float *)d_x, weights, 0, n);
            check(tzh_arctic_set_ffn_fusion(weights.handle(), 0));
            arctic::feedForward((float *)d_z, (const float *)d_x, weights, 0, n);
            check(tzh_arctic_set_ffn_fusion(weights.handle(), 1));
            std::vector<float> y(x.size()), z(x.size());
            check(tzh_memcpy_d2h(ctx.handle(), y.data(), d_y, y.size() * 4));
            check(tzh_memcpy_d2h(ctx.handle(), z.data(), d_z, z.size() * 4));
            tzh_free(ctx.handle(), d_x);
            tzh_free(ctx.handle(), d_y);
            tzh_free(ctx.handle(), d_z);
            double max_abs = 0;
            bool finite = true;
            for (size_t i = 0; i < y.size(); i++) {
                finite = finite && std::isfinite(y[i]) && std::isfinite(z[i]);
                max_abs = std::max(max_abs, (double)std::fabs(y[i] - z[i]));
            }
            std::printf("  feed-forward: fused vs GEMM pair max-abs %.3g\n", max_abs);
            EXPECT(finite && max_abs <= 2e-5);
        });
    }

    std::printf(g_failed ? "FAILED %d\n" : "ALL PASSED\n", g_failed);
    return g_failed ? 1 : 0;
}
