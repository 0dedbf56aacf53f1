// Context, memory and error plumbing of the C-ABI (include/tenzor_hip.h).
#include "common.h"

#include <cstdlib>
#include <cstring>
#include <new>

static thread_local std::string g_last_error;

int tzh_fail(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void tzh_clear_error() { g_last_error.clear(); }

extern "C" const char *tzh_last_error(void) { return g_last_error.c_str(); }

extern "C" int tzh_abi_version(void) { return TZH_ABI_VERSION; }

int tzh_ctx_enter(tzh_ctx *ctx) {
    if (!ctx) return tzh_fail(TZH_ERR_INVALID_ARGS, "null context");
    TZH_HIP(hipSetDevice(ctx->device));
    return TZH_OK;
}

int tzh_ctx_scratch(tzh_ctx *ctx, size_t bytes, void **out) {
    if (bytes > ctx->scratch_bytes) {
        if (ctx->scratch) {
            TZH_HIP(hipStreamSynchronize(ctx->stream));
            TZH_HIP(hipFree(ctx->scratch));
            ctx->scratch = nullptr;
            ctx->scratch_bytes = 0;
        }
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        if (hipMalloc(&ctx->scratch, want) != hipSuccess) {
            (void)hipGetLastError();
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "scratch allocation of %zu bytes failed", want);
        }
        ctx->scratch_bytes = want;
        ctx->scratch_allocs++;
    }
    *out = ctx->scratch;
    return TZH_OK;
}

extern "C" int tzh_ctx_scratch_info(tzh_ctx *ctx, int64_t *bytes, int64_t *allocs) {
    tzh_clear_error();
    if (!ctx || !bytes || !allocs) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *bytes = (int64_t)ctx->scratch_bytes;
    *allocs = ctx->scratch_allocs;
    return TZH_OK;
}

extern "C" int tzh_init(int device, void *stream, tzh_ctx **out) {
    tzh_clear_error();
    if (!out) return tzh_fail(TZH_ERR_INVALID_ARGS, "out is null");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        (void)hipGetLastError();
        return tzh_fail(TZH_ERR_DEVICE, "no HIP device available");
    }
    if (device < 0 || device >= count)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "device %d out of range (have %d)", device, count);
    TZH_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    TZH_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return tzh_fail(TZH_ERR_DEVICE, "device %d is %s; this library is built for gfx950 only",
                        device, prop.gcnArchName);
    tzh_ctx *ctx = new (std::nothrow) tzh_ctx();
    if (!ctx) return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "context allocation failed");
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    const char *interp = std::getenv("TZH_EW_INTERPRETER");
    ctx->ew_interpreter = interp && interp[0] == '1';
    // NULL is the device's default stream, as in every HIP/CUDA library API,
    // so callers on the default stream need no extra synchronisation.
    ctx->stream = (hipStream_t)stream;
    ctx->own_stream = false;
    *out = ctx;
    return TZH_OK;
}

int tzh_ctx_work_queue(tzh_ctx *ctx, unsigned **out) {
    if (!ctx->work_queue) {
        void *p = nullptr;
        if (hipMalloc(&p, 256) != hipSuccess) {
            (void)hipGetLastError();
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "work-queue allocation failed");
        }
        // zeroed and waited for here: the context's stream may be one that
        // does not wait for the default stream
        if (hipMemset(p, 0, 256) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
            (void)hipGetLastError();
            hipFree(p);
            return tzh_fail(TZH_ERR_DEVICE, "work-queue initialisation failed");
        }
        ctx->work_queue = (unsigned *)p;
    }
    *out = ctx->work_queue;
    return TZH_OK;
}

int tzh_ctx_upload_program(tzh_ctx *ctx, const void *src, size_t bytes, const void **dev_out) {
    if (bytes > tzh_ctx::kProgSlotBytes) return tzh_fail(TZH_ERR_INVALID_ARGS, "internal: program of %zu bytes", bytes);
    if (!ctx->prog_dev) {
        const size_t total = (size_t)tzh_ctx::kProgSlots * tzh_ctx::kProgSlotBytes;
        if (hipMalloc(&ctx->prog_dev, total) != hipSuccess) {
            (void)hipGetLastError();
            ctx->prog_dev = nullptr;
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "program ring allocation failed");
        }
        if (hipHostMalloc(&ctx->prog_host, total, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            ctx->prog_host = nullptr;
            return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "program staging allocation failed");
        }
        for (int i = 0; i < tzh_ctx::kProgSlots; i++)
            TZH_HIP(hipEventCreateWithFlags(&ctx->prog_ev[i], hipEventDisableTiming));
    }
    const int k = ctx->prog_next;
    ctx->prog_next = (k + 1) % tzh_ctx::kProgSlots;
    // the previous copy out of this staging slot has finished (events start
    // out complete, so the first round does not wait)
    TZH_HIP(hipEventSynchronize(ctx->prog_ev[k]));
    char *host = (char *)ctx->prog_host + (size_t)k * tzh_ctx::kProgSlotBytes;
    char *dev = (char *)ctx->prog_dev + (size_t)k * tzh_ctx::kProgSlotBytes;
    std::memcpy(host, src, bytes);
    TZH_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    TZH_HIP(hipEventRecord(ctx->prog_ev[k], ctx->stream));
    *dev_out = dev;
    return TZH_OK;
}

extern "C" int tzh_destroy(tzh_ctx *ctx) {
    if (!ctx) return TZH_OK;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (hipEvent_t e : ctx->prog_ev)
        if (e) hipEventDestroy(e);
    if (ctx->prog_dev) hipFree(ctx->prog_dev);
    if (ctx->prog_host) hipHostFree(ctx->prog_host);
    if (ctx->scratch) hipFree(ctx->scratch);
    if (ctx->work_queue) hipFree(ctx->work_queue);
    if (ctx->own_stream) hipStreamDestroy(ctx->stream);
    delete ctx;
    return TZH_OK;
}

extern "C" int tzh_sync(tzh_ctx *ctx) {
    TZH_TRY(tzh_ctx_enter(ctx));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    return TZH_OK;
}

extern "C" void *tzh_stream(tzh_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int tzh_malloc(tzh_ctx *ctx, size_t bytes, void **dptr) {
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!dptr) return tzh_fail(TZH_ERR_INVALID_ARGS, "dptr is null");
    if (hipMalloc(dptr, bytes ? bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        *dptr = nullptr;
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) failed", bytes);
    }
    return TZH_OK;
}

extern "C" int tzh_free(tzh_ctx *ctx, void *dptr) {
    TZH_TRY(tzh_ctx_enter(ctx));
    if (dptr) {
        TZH_HIP(hipStreamSynchronize(ctx->stream));
        TZH_HIP(hipFree(dptr));
    }
    return TZH_OK;
}

extern "C" int tzh_memcpy_h2d(tzh_ctx *ctx, void *dst, const void *src, size_t bytes) {
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!bytes) return TZH_OK;
    if (!dst || !src) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    TZH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    return TZH_OK;
}

extern "C" int tzh_memcpy_d2h(tzh_ctx *ctx, void *dst, const void *src, size_t bytes) {
    TZH_TRY(tzh_ctx_enter(ctx));
    if (!bytes) return TZH_OK;
    if (!dst || !src) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    TZH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    return TZH_OK;
}

// ---------------------------------------------------------------------------
// Host f16 helpers (IEEE round-to-nearest-even, as Zig's @floatCast).
// ---------------------------------------------------------------------------
uint16_t tzh_host_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t h = ((((ax >> 23) - 112u)) << 10) | ((ax & 0x7fffffu) >> 13);
        const uint32_t r = ax & 0x1fffu;
        if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t sh = 126u - e;
    uint32_t h = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float tzh_host_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            x = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}
