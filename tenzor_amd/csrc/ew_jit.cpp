// Generated single-pass chain kernels (K1 fast path).
//
// The reference fuses an elementwise chain at compile time into one loop
// (codegen.zig:15-205 FusedElementwiseKernel: the ops of the chain applied
// in post-order per element, patterns.zig:43-63).  Here the same happens at
// run time: a chain program (ew_program.h) is turned into straight-line HIP
// source - every leaf loaded up front through its broadcast projection with
// the projection kind baked in, every op inlined with its tag as a
// constant - compiled once per program shape with hipRTC for the device's
// architecture, and cached.  Pointers, shapes, divisors and constant values
// stay run-time kernel arguments (the EwProgram struct itself), so programs
// that differ only in those share one kernel.
//
// The op semantics and the program layout are the exact text the
// interpreter kernels are compiled from (ew_shared.inc, stringified below).
#include "ew_program.h"

#ifndef TZH_EMULATION
#include <hip/hiprtc.h>
#else
#include <dlfcn.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#endif

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace tzh_ew {
namespace {

#define TZH_EW_SHARED(...) #__VA_ARGS__
const char kSharedSrc[] =
#include "ew_shared.inc"
    ;
#undef TZH_EW_SHARED

#define TZH_JIT_OPS(X)                                                                                    \
    X(TZH_OP_NEG) X(TZH_OP_ABS) X(TZH_OP_EXP) X(TZH_OP_LOG) X(TZH_OP_SQRT) X(TZH_OP_RSQRT) X(TZH_OP_SIN)   \
    X(TZH_OP_COS) X(TZH_OP_TANH) X(TZH_OP_SIGMOID) X(TZH_OP_RELU) X(TZH_OP_GELU) X(TZH_OP_SILU)           \
    X(TZH_OP_SOFTPLUS) X(TZH_OP_FLOOR) X(TZH_OP_CEIL) X(TZH_OP_ROUND) X(TZH_OP_ADD) X(TZH_OP_SUB)         \
    X(TZH_OP_MUL) X(TZH_OP_DIV) X(TZH_OP_POW) X(TZH_OP_MAX) X(TZH_OP_MIN) X(TZH_OP_PROD)                  \
    X(TZH_OP_REDUCE_MAX) X(TZH_OP_REDUCE_MIN)

std::string prelude() {
    std::string s = "typedef float tzh_f32x4 __attribute__((ext_vector_type(4)));\n"
                    "typedef double tzh_f64x2 __attribute__((ext_vector_type(2)));\n"
                    "enum {";
#define TZH_JIT_ENUM(name) s += std::string(#name) + " = " + std::to_string((int)name) + ", ";
    TZH_JIT_OPS(TZH_JIT_ENUM)
#undef TZH_JIT_ENUM
    s += "};\n";
    s += kSharedSrc;
    s += "\n";
    return s;
}

// Offset expression of leaf j for the flat output index held in `var`.
std::string offset_fn(const EwProgram &p, int j) {
    const EwLeaf &lf = p.leaves[j];
    const std::string L = "p.leaves[" + std::to_string(j) + "]";
    std::string b = "__device__ __forceinline__ long long off" + std::to_string(j) +
                    "(const EwProgram &p, long long flat) {\n";
    if (p.small) {
        b += "    unsigned f = (unsigned)flat;\n";
        if (!lf.general) {
            if (lf.div != 1) b += "    f = fast_div(" + L + ".fdiv, f);\n";
            if (lf.mod <= (long long)0xffffffff) b += "    f = f - fast_div(" + L + ".fmod, f) * " + L + ".fmod.d;\n";
            b += "    return f;\n";
        } else {
            b += "    unsigned off = 0, rem = f, q;\n";
            for (int d = p.ndim - 1; d >= 0; d--) {
                const std::string D = std::to_string(d);
                b += "    q = fast_div(p.fshape[" + D + "], rem);\n";
                if (lf.strides[d] != 0)
                    b += "    off += (rem - q * p.fshape[" + D + "].d) * (unsigned)" + L + ".strides[" + D + "];\n";
                b += "    rem = q;\n";
            }
            b += "    return off;\n";
        }
    } else {
        if (!lf.general) {
            b += "    return (flat / " + L + ".div) % " + L + ".mod;\n";
        } else {
            b += "    long long off = 0, rem = flat;\n";
            for (int d = p.ndim - 1; d >= 0; d--) {
                const std::string D = std::to_string(d);
                if (lf.strides[d] != 0) b += "    off += (rem % p.shape[" + D + "]) * " + L + ".strides[" + D + "];\n";
                b += "    rem /= p.shape[" + D + "];\n";
            }
            b += "    return off;\n";
        }
    }
    b += "}\n";
    return b;
}

// Leaf loads for outputs flat .. flat+W-1 into L<j><sfx>[W].  `flat` is the
// name of the index expression in the generated code.
std::string loads(const EwProgram &p, const char *T, int W, bool vec16, const std::string &sfx,
                  const std::string &flat) {
    std::string b;
    const std::string WS = std::to_string(W);
    for (int j = 0; j < p.n_leaves; j++) {
        const std::string J = std::to_string(j), LJ = "L" + J + sfx;
        const std::string ptr = "((const " + std::string(T) + " *)p.leaves[" + J + "].ptr)";
        b += "        " + std::string(T) + " " + LJ + "[" + WS + "];\n";
        const int mode = W == 1 ? VEC_PER_ELEM : p.leaves[j].vec;
        if (mode == VEC_CONTIG && vec16) {
            const std::string VT = std::string(T) == "float" ? "tzh_f32x4" : "tzh_f64x2";
            b += "        { const " + VT + " raw = *(const " + VT + " *)(" + ptr + " + off" + J + "(p, " + flat + "));\n";
            for (int e = 0; e < W; e++) b += "          " + LJ + "[" + std::to_string(e) + "] = raw[" + std::to_string(e) + "];\n";
            b += "        }\n";
        } else if (mode == VEC_CONTIG) {
            b += "        { const long long o = off" + J + "(p, " + flat + ");\n";
            for (int e = 0; e < W; e++)
                b += "          " + LJ + "[" + std::to_string(e) + "] = " + ptr + "[o + " + std::to_string(e) + "];\n";
            b += "        }\n";
        } else if (mode == VEC_SPLAT) {
            b += "        { const " + std::string(T) + " x = " + ptr + "[off" + J + "(p, " + flat + ")];\n";
            for (int e = 0; e < W; e++) b += "          " + LJ + "[" + std::to_string(e) + "] = x;\n";
            b += "        }\n";
        } else {
            for (int e = 0; e < W; e++)
                b += "        " + LJ + "[" + std::to_string(e) + "] = " + ptr + "[off" + J + "(p, " + flat + " + " +
                     std::to_string(e) + ")];\n";
        }
    }
    return b;
}

// The stack program run symbolically (slot -> expression name) on the
// loaded leaves: r<sfx>[0..W).
std::string compute(const EwProgram &p, const char *T, int W, const std::string &sfx) {
    std::string b;
    for (int e = 0; e < W; e++) {
        const std::string E = std::to_string(e);
        std::string slot[kMaxDepth + 1];
        for (int i = 0; i < p.n_nodes; i++) {
            const EwNode &nd = p.nodes[i];
            const std::string v = "v" + std::to_string(i) + "_" + E + sfx;
            const std::string I = std::to_string(i);
            switch (nd.kind) {
            case EK_LEAF:
                slot[nd.slot] = "L" + std::to_string(nd.arg) + sfx + "[" + E + "]";
                break;
            case EK_CONST:
                b += "        const " + std::string(T) + " " + v + " = (" + T + ")p.nodes[" + I + "].cval;\n";
                slot[nd.slot] = v;
                break;
            case EK_UNARY:
                b += "        const " + std::string(T) + " " + v + " = unary_op<" + T + ">(" + std::to_string(nd.op) +
                     ", " + slot[nd.slot] + ");\n";
                slot[nd.slot] = v;
                break;
            default:
                b += "        const " + std::string(T) + " " + v + " = binary_op<" + T + ">(" + std::to_string(nd.op) +
                     ", " + slot[nd.slot] + ", " + slot[nd.slot + 1] + ");\n";
                slot[nd.slot] = v;
                break;
            }
        }
        b += "        r" + sfx + "[" + E + "] = " + slot[0] + ";\n";
    }
    return b;
}

// Store of r<sfx>[0..W) at out + flat (16-byte nontemporal when whole).
std::string store(const char *T, int W, bool vec16, bool f64, const std::string &sfx, const std::string &flat) {
    std::string b;
    if (vec16) {
        const std::string VT = f64 ? "tzh_f64x2" : "tzh_f32x4";
        b += "        { " + VT + " o;\n";
        for (int e = 0; e < W; e++) b += "          o[" + std::to_string(e) + "] = r" + sfx + "[" + std::to_string(e) + "];\n";
        b += "          __builtin_nontemporal_store(o, (" + VT + " *)(out + " + flat + ")); }\n";
    } else {
        for (int e = 0; e < W; e++)
            b += "        out[" + flat + " + " + std::to_string(e) + "] = r" + sfx + "[" + std::to_string(e) + "];\n";
    }
    return b;
}

// Grid-stride kernel over numel / V vectors of V outputs.  Each thread
// takes kUnroll vectors (one grid stride apart) per trip: all their leaf
// loads are issued before any arithmetic, which doubles the bytes in flight
// per thread.  Leftover vectors run one per trip; the numel % V tail
// elements run one per thread of block 0.
constexpr int kUnroll = 2;

std::string chain_source(const EwProgram &p, bool f64, int V) {
    const char *T = f64 ? "double" : "float";
    const bool vec16 = V * (f64 ? 8 : 4) == 16;
    std::string s = prelude();
    for (int j = 0; j < p.n_leaves; j++) s += offset_fn(p, j);
    const std::string VS = std::to_string(V);
    s += "extern \"C\" __global__ void __launch_bounds__(256) tzh_chain(const EwProgram p, " + std::string(T) +
         " *__restrict__ out) {\n";
    s += "    const long long nvec = p.numel / " + VS + ";\n";
    s += "    const long long stride = (long long)gridDim.x * blockDim.x;\n";
    s += "    long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n";
    s += "    for (; v + " + std::to_string(kUnroll - 1) + " * stride < nvec; v += " + std::to_string(kUnroll) +
         " * stride) {\n";
    for (int u = 0; u < kUnroll; u++) {
        const std::string U = "_" + std::to_string(u);
        s += "        const long long flat" + U + " = (v + " + std::to_string(u) + " * stride) * " + VS + ";\n";
        s += loads(p, T, V, vec16, U, "flat" + U);
    }
    for (int u = 0; u < kUnroll; u++) {
        const std::string U = "_" + std::to_string(u);
        s += "        " + std::string(T) + " r" + U + "[" + VS + "];\n";
        s += compute(p, T, V, U);
        s += store(T, V, vec16, f64, U, "flat" + U);
    }
    s += "    }\n";
    s += "    for (; v < nvec; v += stride) {\n";
    s += "        const long long flat = v * " + VS + ";\n";
    s += loads(p, T, V, vec16, "", "flat");
    s += "        " + std::string(T) + " r[" + VS + "];\n";
    s += compute(p, T, V, "");
    s += store(T, V, vec16, f64, "", "flat");
    s += "    }\n";
    // tail (numel % V elements): one element per thread of block 0
    s += "    if (blockIdx.x == 0) {\n";
    s += "        const long long flat = nvec * " + VS + " + threadIdx.x;\n";
    s += "        if (flat < p.numel) {\n";
    s += loads(p, T, 1, false, "", "flat");
    s += "        " + std::string(T) + " r[1];\n";
    s += compute(p, T, 1, "");
    s += "        out[flat] = r[0];\n";
    s += "        }\n    }\n}\n";
    return s;
}

#ifdef TZH_EMULATION
// CPU emulation build (tests/cpu_emu; test infrastructure only): the same
// generated text is compiled as C++ against the emulated runtime header,
// with AddressSanitizer, into a shared object linked to the emulation
// library, and its kernel is run on the emulator's fibers.  The compiler
// and header directory are fixed when the emulation library is built.
using EmuLaunch = void (*)(unsigned grid, const void *p, void *out);

std::mutex g_mu;
std::unordered_map<std::string, EmuLaunch> g_cache;  // key: source
std::string g_dir;

int emu_compile(const std::string &src, bool f64, EmuLaunch *out) {
    if (g_dir.empty()) {
        char tmpl[] = "/tmp/tzh_emu_jit_XXXXXX";
        if (!mkdtemp(tmpl)) return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: mkdtemp failed");
        g_dir = tmpl;
    }
    Dl_info info{};
    if (!dladdr((const void *)&jit_chain_launch, &info) || !info.dli_fname)
        return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: cannot locate the emulation library");
    const std::string stem = g_dir + "/k" + std::to_string(g_cache.size());
    const char *T = f64 ? "double" : "float";
    std::string text = "#include \"hip/hip_runtime.h\"\n" + src;
    text += "extern \"C\" void tzh_chain_emu_launch(unsigned grid, const void *p, void *out) {\n"
            "    emu::launch_kernel(\"tzh_chain (generated)\", tzh_chain, dim3(grid), dim3(256),\n"
            "                       *(const EwProgram *)p, (" + std::string(T) + " *)out);\n}\n";
    FILE *f = std::fopen((stem + ".cpp").c_str(), "w");
    if (!f) return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: cannot write %s.cpp", stem.c_str());
    std::fwrite(text.data(), 1, text.size(), f);
    std::fclose(f);
    const std::string cmd = std::string(TZH_EMU_CXX) + " -x c++ -std=c++17 -O1 -g -fPIC -shared -fsanitize=address" +
                            " -ffp-contract=off -Wno-unused-result -I" + TZH_EMU_INC + " " + stem + ".cpp -x none " +
                            info.dli_fname + " -o " + stem + ".so > " + stem + ".log 2>&1";
    if (std::system(cmd.c_str()) != 0)
        return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: compile failed (see %s.log)", stem.c_str());
    void *h = dlopen((stem + ".so").c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: %s", dlerror());
    *out = (EmuLaunch)dlsym(h, "tzh_chain_emu_launch");
    if (!*out) return tzh_fail(TZH_ERR_DEVICE, "emulated chain kernel: no launcher");
    return TZH_OK;
}

}  // namespace

int jit_chain_launch(tzh_ctx *ctx, const EwProgram &p, bool f64, int V, int grid, void *out) {
    (void)ctx;
    const std::string src = chain_source(p, f64, V);
    EmuLaunch fn = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_cache.find(src);
        if (it == g_cache.end()) {
            TZH_TRY(emu_compile(src, f64, &fn));
            g_cache.emplace(src, fn);
        } else {
            fn = it->second;
        }
    }
    fn((unsigned)grid, &p, out);
    return TZH_OK;
}

#else
struct Compiled {
    hipModule_t module;
    hipFunction_t fn;
};

std::mutex g_mu;
std::unordered_map<std::string, Compiled> g_cache;  // key: device id + source

int compile(int device, const std::string &src, Compiled *out) {
    hipDeviceProp_t prop;
    TZH_HIP(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    arch = arch.substr(0, arch.find(':'));
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src.c_str(), "tzh_chain.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return tzh_fail(TZH_ERR_DEVICE, "hiprtcCreateProgram failed");
    const std::string arch_opt = "--offload-arch=" + arch;
    // same floating-point contract as the library build: no contraction, no
    // packed f32 instructions
    const char *opts[] = {arch_opt.c_str(), "-O3", "-std=c++17", "-ffp-contract=off",
                          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
    const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n + 1, '\0');
        hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return tzh_fail(TZH_ERR_DEVICE, "chain kernel compilation failed (%s): %.1500s", hiprtcGetErrorString(rc),
                        log.c_str());
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    std::vector<char> code(n);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    TZH_HIP(hipModuleLoadData(&out->module, code.data()));
    TZH_HIP(hipModuleGetFunction(&out->fn, out->module, "tzh_chain"));
    return TZH_OK;
}

}  // namespace

int jit_chain_launch(tzh_ctx *ctx, const EwProgram &p, bool f64, int V, int grid, void *out) {
    const std::string src = chain_source(p, f64, V);
    const std::string key = std::to_string(ctx->device) + "\n" + src;
    Compiled k{};
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_cache.find(key);
        if (it == g_cache.end()) {
            TZH_TRY(compile(ctx->device, src, &k));
            g_cache.emplace(key, k);
        } else {
            k = it->second;
        }
    }
    EwProgram arg = p;
    void *args[] = {&arg, &out};
    TZH_HIP(hipModuleLaunchKernel(k.fn, (unsigned)grid, 1, 1, 256, 1, 1, 0, ctx->stream, args, nullptr));
    return TZH_OK;
}

#endif

}  // namespace tzh_ew
