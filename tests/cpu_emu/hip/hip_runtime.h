// TEST INFRASTRUCTURE ONLY: a CPU emulation of the subset of HIP that
// libtenzor_hip's sources use, so the same kernel sources can be compiled
// for the host (with AddressSanitizer) and every launch executed on the CPU
// with its real grid/block shape.  Each lane is a fiber; wave-wide operations
// (shuffles, MFMA) and __syncthreads are barriers over the wave / block.  A
// barrier that can never complete (divergent __syncthreads, a lane that
// never reaches a shuffle) aborts with the kernel and thread named, which is
// how a GPU hang would show up here.
//
// MFMA operand/result layouts follow the CDNA register layouts the kernels
// assume: v_mfma_f32_32x32x16_f16 (A: row = lane%32, k = 8*(lane/32)+i;
// B: col = lane%32, same k; D element e of lane l: row 8*(e/4) + 4*(l/32) +
// e%4, col l%32) and v_mfma_f32_16x16x32_f16 (A/B: row/col = lane%16,
// k = 8*(lane/16)+i; D element e: row 4*(l/16)+e, col l%16), and
// v_mfma_f32_16x16x4_f32 / v_mfma_f64_16x16x4_f64 (A/B: one value per lane,
// row/col = lane%16, k = lane/16; D element e: row 4*(l/16)+e in f32 and
// row l/16+4*e in f64, col l%16).
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))

struct dim3 {
    unsigned x = 1, y = 1, z = 1;
    dim3() = default;
    dim3(unsigned a, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

struct uint4 {
    unsigned x, y, z, w;
};
struct uint2 {
    unsigned x, y;
};
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return uint4{a, b, c, d}; }

namespace emu {
extern dim3 g_threadIdx, g_blockIdx, g_blockDim, g_gridDim;
void syncthreads();
void wave_barrier();
int lane_id();
int wave_id();
void *wave_slot(int lane);  // 256-byte exchange slot of `lane` in the caller's wave
void launch(const char *name, dim3 grid, dim3 block, void (*body)(void *), void *ctx);
// direct-to-LDS loads: queued per lane at issue, written to LDS when a
// vmcnt wait of that lane retires them (oldest first), so a stage read
// before its wait sees stale data and fails the parity checks
void dma16(const void *src, void *lds_dst);
void waitcnt_vm(int n);
void vmem_marker();  // a vector memory op with no LDS effect (a store or a register load), in issue order
// A value the hardware holds once per wave (an SGPR, M0): every live lane of
// the wave must pass the same v, or the emulation aborts naming `what` and
// the source line (on the GPU a divergent value would silently become one
// lane's).  Returns the value of the wave's first live lane.
uint64_t wave_uniform(uint64_t v, const char *what, const char *file, int line);
}  // namespace emu

// the hooks gemm_pipe.hip takes from its target: DMA issue and LDS barrier
#define TZH_EMULATION 1
// global_load_lds_dwordx4 takes its global base in an SGPR pair and its LDS
// base in M0: both must be wave-uniform
inline void emu_dma16(const char *sbase, uint32_t voff, char *lds_base, const char *file, int line) {
    emu::wave_uniform((uint64_t)(uintptr_t)sbase, "dma16 global base (SGPR operand)", file, line);
    emu::wave_uniform((uint64_t)(uintptr_t)lds_base, "dma16 LDS base (M0)", file, line);
    emu::dma16(sbase + voff, lds_base + 16 * emu::lane_id());
}
#define dma16(sbase, voff, lds_base) emu_dma16((sbase), (voff), (lds_base), __FILE__, __LINE__)
inline void lds_barrier_only() { emu::syncthreads(); }
inline void vmem_store_issued() { emu::vmem_marker(); }
inline void vmem_load_issued() { emu::vmem_marker(); }
// v_permlane32_swap_b32: lanes 32..63 of `lo` <-> lanes 0..31 of `hi`
inline void lane_swap32(uint32_t &lo, uint32_t &hi) {
    const int lane = emu::lane_id();
    const uint32_t mine[2] = {lo, hi};
    std::memcpy(emu::wave_slot(lane), mine, sizeof mine);
    emu::wave_barrier();
    uint32_t other[2];
    std::memcpy(other, emu::wave_slot(lane ^ 32), sizeof other);
    emu::wave_barrier();
    if (lane < 32)
        hi = other[0];  // the upper partner's lo
    else
        lo = other[1];  // the lower partner's hi
}
// v_permlane16_swap_b32: odd 16-lane rows of `a` <-> even rows of `b`
inline void lane_swap16(uint32_t &a, uint32_t &b) {
    const int lane = emu::lane_id();
    const uint32_t mine[2] = {a, b};
    std::memcpy(emu::wave_slot(lane), mine, sizeof mine);
    emu::wave_barrier();
    uint32_t other[2];
    std::memcpy(other, emu::wave_slot(lane ^ 16), sizeof other);
    emu::wave_barrier();
    if (lane & 16)
        a = other[1];  // the even-row partner's b
    else
        b = other[0];  // the odd-row partner's a
}
inline void wave_lds_order() { emu::wave_barrier(); }
// v_mov_b32 with a DPP lane pattern, every lane active and every row and
// bank enabled: quad_perm (ctrl < 0x100), row_mirror (0x140) and
// row_half_mirror (0x141); others abort
inline int __builtin_amdgcn_update_dpp(int, int src, int ctrl, int, int, bool) {
    const int lane = emu::lane_id();
    int from;
    if (ctrl < 0x100)
        from = (lane & ~3) | ((ctrl >> (2 * (lane & 3))) & 3);
    else if (ctrl == 0x140)
        from = (lane & ~15) | (15 - (lane & 15));
    else if (ctrl == 0x141)
        from = (lane & ~7) | (7 - (lane & 7));
    else
        __builtin_trap();
    std::memcpy(emu::wave_slot(lane), &src, sizeof src);
    emu::wave_barrier();
    int r;
    std::memcpy(&r, emu::wave_slot(from), sizeof r);
    emu::wave_barrier();
    return r;
}
inline bool wave_any(bool p) {  // every lane of the emulated wave is active
    const int lane = emu::lane_id();
    *(unsigned char *)emu::wave_slot(lane) = p ? 1 : 0;
    emu::wave_barrier();
    bool any = false;
    for (int l = 0; l < 64; l++) any = any || *(unsigned char *)emu::wave_slot(l);
    emu::wave_barrier();
    return any;
}
#define __builtin_amdgcn_s_waitcnt(imm) emu::waitcnt_vm(((imm)&15) | ((((imm) >> 14) & 3) << 4))
// v_readfirstlane_b32: the first live lane's value; the kernels use it only
// on values that are already wave-uniform, which the emulation checks
template <typename T>
inline T emu_readfirstlane(T x, const char *file, int line) {
    static_assert(sizeof(T) <= 8, "32/64-bit values only");
    uint64_t v = 0;
    std::memcpy(&v, &x, sizeof(T));
    v = emu::wave_uniform(v, "readfirstlane operand", file, line);
    T r;
    std::memcpy(&r, &v, sizeof(T));
    return r;
}
#define __builtin_amdgcn_readfirstlane(x) emu_readfirstlane((x), __FILE__, __LINE__)
#define __builtin_amdgcn_ldexpf(x, e) ldexpf((x), (e))
// v_frexp_exp_i32_f32: the exponent of frexp (x = f 2^e, f in [0.5, 1))
inline int __builtin_amdgcn_frexp_expf(float x) {
    int e = 0;
    (void)frexpf(x, &e);
    return e;
}

#define threadIdx (emu::g_threadIdx)
#define blockIdx (emu::g_blockIdx)
#define blockDim (emu::g_blockDim)
#define gridDim (emu::g_gridDim)

inline void __syncthreads() { emu::syncthreads(); }

template <typename T>
inline T __shfl_xor(T v, int mask, int width = 64) {
    static_assert(sizeof(T) <= 256, "slot too small");
    const int lane = emu::lane_id();
    std::memcpy(emu::wave_slot(lane), &v, sizeof(T));
    emu::wave_barrier();
    const int src = ((lane ^ mask) & (width - 1)) | (lane & ~(width - 1));
    T r;
    std::memcpy(&r, emu::wave_slot(src), sizeof(T));
    emu::wave_barrier();
    return r;
}

template <typename T>
inline T __shfl(T v, int src_lane, int width = 64) {
    static_assert(sizeof(T) <= 256, "slot too small");
    const int lane = emu::lane_id();
    std::memcpy(emu::wave_slot(lane), &v, sizeof(T));
    emu::wave_barrier();
    const int src = (src_lane & (width - 1)) | (lane & ~(width - 1));
    T r;
    std::memcpy(&r, emu::wave_slot(src), sizeof(T));
    emu::wave_barrier();
    return r;
}

template <typename T>
inline T atomicAdd(T *p, T v) {  // fibers are cooperative on one OS thread
    T old = *p;
    *p = old + v;
    return old;
}

template <typename T>
inline T atomicExch(T *p, T v) {
    T old = *p;
    *p = v;
    return old;
}

using std::max;
using std::min;
using std::sqrt;  // sqrt(float) in float, as HIP's overload computes it (not via double)
using std::isnan;
using std::isinf;
using std::isfinite;
inline unsigned __umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }

typedef _Float16 emu_half8 __attribute__((ext_vector_type(8)));
typedef float emu_f32x16 __attribute__((ext_vector_type(16)));
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));

namespace emu {
struct MfmaIn {
    emu_half8 a, b;
};

inline emu_f32x16 mfma_32x32x16(emu_half8 a, emu_half8 b, emu_f32x16 c) {
    const int lane = lane_id();
    MfmaIn in{a, b};
    std::memcpy(wave_slot(lane), &in, sizeof in);
    wave_barrier();
    emu_f32x16 d = c;
    for (int e = 0; e < 16; e++) {
        const int row = 8 * (e / 4) + 4 * (lane / 32) + e % 4, col = lane % 32;
        float acc = 0.0f;
        for (int k = 0; k < 16; k++) {
            MfmaIn ai, bi;
            std::memcpy(&ai, wave_slot(row + 32 * (k / 8)), sizeof ai);
            std::memcpy(&bi, wave_slot(col + 32 * (k / 8)), sizeof bi);
            acc += (float)ai.a[k % 8] * (float)bi.b[k % 8];
        }
        d[e] += acc;
    }
    wave_barrier();
    return d;
}

inline emu_f32x4 mfma_16x16x32(emu_half8 a, emu_half8 b, emu_f32x4 c) {
    const int lane = lane_id();
    MfmaIn in{a, b};
    std::memcpy(wave_slot(lane), &in, sizeof in);
    wave_barrier();
    emu_f32x4 d = c;
    for (int e = 0; e < 4; e++) {
        const int row = 4 * (lane / 16) + e, col = lane % 16;
        float acc = 0.0f;
        for (int k = 0; k < 32; k++) {
            MfmaIn ai, bi;
            std::memcpy(&ai, wave_slot(row + 16 * (k / 8)), sizeof ai);
            std::memcpy(&bi, wave_slot(col + 16 * (k / 8)), sizeof bi);
            acc += (float)ai.a[k % 8] * (float)bi.b[k % 8];
        }
        d[e] += acc;
    }
    wave_barrier();
    return d;
}

struct MfmaIn64 {
    double a, b;
};

// 16x16x4 with one f32 or f64 operand value per lane; T is the element type
template <typename T, typename V>
inline V mfma_16x16x4(T a, T b, V c) {
    const int lane = lane_id();
    MfmaIn64 in{(double)a, (double)b};
    std::memcpy(wave_slot(lane), &in, sizeof in);
    wave_barrier();
    V d = c;
    for (int e = 0; e < 4; e++) {
        const int row = sizeof(T) == 4 ? 4 * (lane / 16) + e : lane / 16 + 4 * e, col = lane % 16;
        T acc = 0;
        for (int k = 0; k < 4; k++) {
            MfmaIn64 ai, bi;
            std::memcpy(&ai, wave_slot(row + 16 * k), sizeof ai);
            std::memcpy(&bi, wave_slot(col + 16 * k), sizeof bi);
            acc += (T)ai.a * (T)bi.b;
        }
        d[e] += acc;
    }
    wave_barrier();
    return d;
}
}  // namespace emu

typedef double emu_f64x4 __attribute__((ext_vector_type(4)));
namespace emu {
inline emu_f32x4 mfma_f32_16x16x4_args(float a, float b, emu_f32x4 c, int, int, int) {
    return mfma_16x16x4<float, emu_f32x4>(a, b, c);
}
inline emu_f64x4 mfma_f64_16x16x4_args(double a, double b, emu_f64x4 c, int, int, int) {
    return mfma_16x16x4<double, emu_f64x4>(a, b, c);
}
inline emu_f32x16 mfma_32x32x16_args(emu_half8 a, emu_half8 b, emu_f32x16 c, int, int, int) {
    return mfma_32x32x16(a, b, c);
}
inline emu_f32x4 mfma_16x16x32_args(emu_half8 a, emu_half8 b, emu_f32x4 c, int, int, int) {
    return mfma_16x16x32(a, b, c);
}
}  // namespace emu
// variadic so that brace-initialised operands (which contain commas) pass through
#define __builtin_amdgcn_mfma_f32_32x32x16_f16(...) emu::mfma_32x32x16_args(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(...) emu::mfma_16x16x32_args(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f32_16x16x4f32(...) emu::mfma_f32_16x16x4_args(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f64_16x16x4f64(...) emu::mfma_f64_16x16x4_args(__VA_ARGS__)
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
// v_perm_b32: byte i of the result is byte sel[i] of {src0 (bytes 4..7), src1 (bytes 0..3)};
// 8..11 replicate a sign bit, 12 gives 0x00, 13.. give 0xff
inline uint32_t __builtin_amdgcn_perm(uint32_t src0, uint32_t src1, uint32_t sel) {
    const uint64_t in = ((uint64_t)src0 << 32) | src1;
    uint32_t r = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t s = (sel >> (8 * i)) & 0xffu;
        uint32_t b;
        if (s >= 13) b = 0xffu;
        else if (s == 12) b = 0u;
        else if (s >= 8) b = ((in >> (8 * (2 * (s - 8) + 1) + 7)) & 1u) ? 0xffu : 0u;
        else b = (uint32_t)(in >> (8 * s)) & 0xffu;
        r |= b << (8 * i);
    }
    return r;
}

// ---------------------------------------------------------------------------
// runtime API subset
// ---------------------------------------------------------------------------
typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2, hipErrorNoDevice = 100 };
typedef struct emu_stream *hipStream_t;
typedef struct emu_event *hipEvent_t;
enum hipMemcpyKind { hipMemcpyHostToHost, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice };
#define hipEventDisableTiming 2u
#define hipEventDisableSystemFence 0x20000000u
#define hipHostMallocDefault 0u
#define hipStreamNonBlocking 1u

struct hipDeviceProp_t {
    char gcnArchName[256];
    int multiProcessorCount;
};

hipError_t hipGetDeviceCount(int *n);
hipError_t hipSetDevice(int d);
hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int d);
hipError_t hipMalloc(void **p, size_t n);
hipError_t hipFree(void *p);
hipError_t hipMallocAsync(void **p, size_t n, hipStream_t s);
hipError_t hipFreeAsync(void *p, hipStream_t s);
hipError_t hipHostMalloc(void **p, size_t n, unsigned flags);
hipError_t hipHostFree(void *p);
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind k, hipStream_t st);
hipError_t hipMemset(void *p, int v, size_t n);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipDeviceSynchronize();
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned f);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned f);
hipError_t hipEventCreate(hipEvent_t *e);
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipGetLastError();
// device symbols are host arrays here: their address is the symbol itself
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void **p, const void *sym) {
    *p = const_cast<void *>(sym);
    return hipSuccess;
}
const char *hipGetErrorString(hipError_t e);

// hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...): every lane
// runs `kernel(args...)` in its own fiber.
#include <tuple>
#include <utility>
namespace emu {
template <typename F, typename Tup>
struct LaunchCtx {
    F f;
    Tup args;
};
template <typename F, typename Tup>
void launch_body(void *p) {
    auto *c = static_cast<LaunchCtx<F, Tup> *>(p);
    std::apply(c->f, c->args);
}
template <typename F, typename... A>
void launch_kernel(const char *name, F f, dim3 g, dim3 b, A &&...args) {
    using Tup = std::tuple<std::decay_t<A>...>;
    LaunchCtx<F, Tup> ctx{f, Tup(std::forward<A>(args)...)};
    launch(name, g, b, &launch_body<F, Tup>, &ctx);
}
}  // namespace emu

#define hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ...) \
    emu::launch_kernel(#kernel, (kernel), dim3(grid), dim3(block), __VA_ARGS__)
