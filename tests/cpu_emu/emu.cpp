// TEST INFRASTRUCTURE ONLY: fiber scheduler and runtime-API stubs behind
// tests/cpu_emu/hip/hip_runtime.h.  One OS thread runs every lane of a
// block as a ucontext fiber; blocks run one after another.
#include "hip/hip_runtime.h"

#undef dma16  // the kernels' hook (hip_runtime.h); emu::dma16 below is the queue behind it

#include <setjmp.h>
#include <ucontext.h>

#include <cstdio>
#include <cstdlib>
#include <deque>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#include <sanitizer/common_interface_defs.h>
#endif
#endif

namespace emu {

dim3 g_threadIdx, g_blockIdx, g_blockDim, g_gridDim;

namespace {
enum State { RUN, AT_BLOCK, AT_WAVE, DONE };
// A fiber starts on its own stack through makecontext/setcontext; every
// later switch is _setjmp/_longjmp, which (unlike swapcontext) saves no
// signal mask and so makes no system call.
struct Fiber {
    ucontext_t uc;
    jmp_buf jb;
    bool started;
    State st;
};
constexpr size_t kStack = 512 * 1024;
constexpr size_t kSlot = 256;
std::vector<Fiber> fibers;
std::vector<char *> stacks;
std::vector<unsigned char> slots;
struct PendingDma {
    char *dst;  // nullptr: a store marker (retires with no LDS effect)
    unsigned char data[16];
};
std::vector<std::deque<PendingDma>> dma_q;  // per lane of the running block
jmp_buf sched_jb;
int cur = -1;
void (*g_body)(void *) = nullptr;
void *g_ctx = nullptr;
const char *g_name = "";
#ifdef EMU_ASAN
const void *sched_bottom = nullptr;
size_t sched_size = 0;
#endif

void to_sched(bool dying) {
#ifdef EMU_ASAN
    void *fake = nullptr;
    __sanitizer_start_switch_fiber(dying ? nullptr : &fake, sched_bottom, sched_size);
    if (!_setjmp(fibers[(size_t)cur].jb)) _longjmp(sched_jb, 1);
    __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#else
    (void)dying;
    if (!_setjmp(fibers[(size_t)cur].jb)) _longjmp(sched_jb, 1);
#endif
}

void fiber_entry(int) {
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &sched_bottom, &sched_size);
#endif
    g_body(g_ctx);
    fibers[(size_t)cur].st = DONE;
    to_sched(true);
}

void switch_to(int i) {
    Fiber &f = fibers[(size_t)i];
    if (!_setjmp(sched_jb)) {
        if (f.started) _longjmp(f.jb, 1);
        f.started = true;
        setcontext(&f.uc);
    }
}

void run_fiber(int i) {
    cur = i;
    g_threadIdx = dim3((unsigned)i % g_blockDim.x, 0, 0);
#ifdef EMU_ASAN
    void *fake = nullptr;
    __sanitizer_start_switch_fiber(&fake, stacks[(size_t)i], kStack);
    switch_to(i);
    __sanitizer_finish_switch_fiber(fake, &sched_bottom, &sched_size);
#else
    switch_to(i);
#endif
}

[[noreturn]] void deadlock(int n) {
    std::fprintf(stderr, "EMU: kernel %s block (%u,%u,%u) cannot make progress (a barrier or wave operation "
                         "that not every live lane reaches):\n", g_name, g_blockIdx.x, g_blockIdx.y, g_blockIdx.z);
    for (int i = 0; i < n; i++)
        std::fprintf(stderr, "  thread %d state %d\n", i, (int)fibers[(size_t)i].st);
    std::abort();
}
}  // namespace

void syncthreads() {
    fibers[(size_t)cur].st = AT_BLOCK;
    to_sched(false);
}

void wave_barrier() {
    fibers[(size_t)cur].st = AT_WAVE;
    to_sched(false);
}

void dma16(const void *src, void *lds_dst) {
    PendingDma p;
    p.dst = (char *)lds_dst;
    std::memcpy(p.data, src, 16);  // the global read (bounds-checked here)
    dma_q[(size_t)cur].push_back(p);
}

void vmem_marker() {
    PendingDma p;
    p.dst = nullptr;
    dma_q[(size_t)cur].push_back(p);
}

void waitcnt_vm(int n) {
    std::deque<PendingDma> &q = dma_q[(size_t)cur];
    while ((int)q.size() > n) {
        if (q.front().dst) std::memcpy(q.front().dst, q.front().data, 16);  // the LDS write (bounds-checked here)
        q.pop_front();
    }
}

uint64_t wave_uniform(uint64_t v, const char *what, const char *file, int line) {
    const int lane = cur % 64, base = cur - lane;
    std::memcpy(wave_slot(lane), &v, sizeof v);
    wave_barrier();  // every live lane of the wave has written its value
    const int n = (int)fibers.size() - base < 64 ? (int)fibers.size() - base : 64;
    uint64_t first = v;
    bool have = false;
    for (int l = 0; l < n; l++) {
        if (fibers[(size_t)(base + l)].st == DONE) continue;  // exited lanes take no part
        uint64_t o;
        std::memcpy(&o, wave_slot(l), sizeof o);
        if (!have) {
            first = o;
            have = true;
        } else if (o != first) {
            std::fprintf(stderr,
                         "EMU: kernel %s block (%u,%u,%u) wave %d: %s is not wave-uniform at %s:%d "
                         "(lane %d has %#llx, the first live lane %#llx)\n",
                         g_name, g_blockIdx.x, g_blockIdx.y, g_blockIdx.z, cur / 64, what, file, line, l,
                         (unsigned long long)o, (unsigned long long)first);
            std::abort();
        }
    }
    wave_barrier();  // every lane has read the slots before they are reused
    return first;
}

int lane_id() { return cur % 64; }
int wave_id() { return cur / 64; }
void *wave_slot(int lane) { return &slots[((size_t)(cur / 64) * 64 + (size_t)lane) * kSlot]; }

void launch(const char *name, dim3 grid, dim3 block, void (*body)(void *), void *ctx) {
    if (block.y != 1 || block.z != 1 || block.x == 0 || block.x > 1024) {
        std::fprintf(stderr, "EMU: unsupported block shape for %s\n", name);
        std::abort();
    }
    const int n = (int)block.x;
    if (grid.x == 0) {
        std::fprintf(stderr, "EMU: kernel %s launched with an empty grid\n", name);
        std::abort();
    }
    while ((int)stacks.size() < n) stacks.push_back((char *)std::malloc(kStack));
    fibers.resize((size_t)n);
    dma_q.assign((size_t)n, {});
    slots.assign((size_t)((n + 63) / 64) * 64 * kSlot, 0);
    g_body = body;
    g_ctx = ctx;
    g_name = name;
    g_blockDim = block;
    g_gridDim = grid;
    for (unsigned bz = 0; bz < grid.z; bz++)
        for (unsigned by = 0; by < grid.y; by++)
            for (unsigned bx = 0; bx < grid.x; bx++) {
                g_blockIdx = dim3(bx, by, bz);
                for (int i = 0; i < n; i++) {
                    Fiber &f = fibers[(size_t)i];
                    getcontext(&f.uc);
                    f.uc.uc_stack.ss_sp = stacks[(size_t)i];
                    f.uc.uc_stack.ss_size = kStack;
                    f.uc.uc_link = nullptr;
                    makecontext(&f.uc, (void (*)())fiber_entry, 1, i);
                    f.started = false;
                    f.st = RUN;
                }
                for (;;) {
                    bool ran = false;
                    for (int i = 0; i < n; i++)
                        if (fibers[(size_t)i].st == RUN) {
                            run_fiber(i);
                            ran = true;
                        }
                    int live = 0, at_block = 0;
                    for (int i = 0; i < n; i++) {
                        live += fibers[(size_t)i].st != DONE;
                        at_block += fibers[(size_t)i].st == AT_BLOCK;
                    }
                    if (live == 0) break;
                    bool released = false;
                    for (int w = 0; w < (n + 63) / 64; w++) {
                        int wl = 0, wa = 0;
                        for (int i = w * 64; i < n && i < (w + 1) * 64; i++) {
                            wl += fibers[(size_t)i].st != DONE;
                            wa += fibers[(size_t)i].st == AT_WAVE;
                        }
                        if (wl > 0 && wa == wl) {
                            for (int i = w * 64; i < n && i < (w + 1) * 64; i++)
                                if (fibers[(size_t)i].st == AT_WAVE) fibers[(size_t)i].st = RUN;
                            released = true;
                        }
                    }
                    if (!released && at_block == live) {
                        for (int i = 0; i < n; i++)
                            if (fibers[(size_t)i].st == AT_BLOCK) fibers[(size_t)i].st = RUN;
                        released = true;
                    }
                    if (!ran && !released) deadlock(n);
                }
                for (int i = 0; i < n; i++) {
                    // trailing store markers may stay pending at exit; loads may not
                    while (!dma_q[(size_t)i].empty() && !dma_q[(size_t)i].back().dst) dma_q[(size_t)i].pop_back();
                    bool loads_pending = false;
                    for (const PendingDma &d : dma_q[(size_t)i]) loads_pending |= d.dst != nullptr;
                    if (!loads_pending) dma_q[(size_t)i].clear();
                }
                for (int i = 0; i < n; i++)
                    if (!dma_q[(size_t)i].empty()) {
                        std::fprintf(stderr, "EMU: kernel %s thread %d exited with %zu direct-to-LDS loads never "
                                             "waited for\n", name, i, dma_q[(size_t)i].size());
                        std::abort();
                    }
            }
    cur = -1;
}

}  // namespace emu

// ---------------------------------------------------------------------------
// runtime stubs: "device" memory is host memory with exact-size allocations
// (so AddressSanitizer's redzones sit right after every buffer)
// ---------------------------------------------------------------------------
struct emu_stream {};
struct emu_event {};

hipError_t hipGetDeviceCount(int *n) { *n = 1; return hipSuccess; }
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int) {
    std::memset(p, 0, sizeof *p);
    std::strcpy(p->gcnArchName, "gfx950:sramecc+:xnack-");
    const char *cus = getenv("TZH_EMU_CUS");
    p->multiProcessorCount = cus ? atoi(cus) : 16;
    return hipSuccess;
}
hipError_t hipMalloc(void **p, size_t n) {
    if (posix_memalign(p, 256, n ? n : 1)) return hipErrorOutOfMemory;
    std::memset(*p, 0xA5, n);  // poison: kernels must not rely on zeroed memory
    return hipSuccess;
}
hipError_t hipFree(void *p) { std::free(p); return hipSuccess; }
// launches run to completion when issued, so a stream-ordered free is an immediate one
hipError_t hipMallocAsync(void **p, size_t n, hipStream_t) { return hipMalloc(p, n); }
hipError_t hipFreeAsync(void *p, hipStream_t) { return hipFree(p); }
hipError_t hipHostMalloc(void **p, size_t n, unsigned) { return hipMalloc(p, n); }
hipError_t hipHostFree(void *p) { return hipFree(p); }
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) { std::memmove(d, s, n); return hipSuccess; }
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind k, hipStream_t) { return hipMemcpy(d, s, n, k); }
hipError_t hipMemset(void *p, int v, size_t n) { std::memset(p, v, n); return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) { *s = new emu_stream; return hipSuccess; }
hipError_t hipStreamDestroy(hipStream_t s) { delete s; return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { *e = new emu_event; return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t *e) { *e = new emu_event; return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) { *ms = 0.0f; return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t e) { delete e; return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipGetLastError() { return hipSuccess; }
const char *hipGetErrorString(hipError_t) { return "emulated HIP error"; }
