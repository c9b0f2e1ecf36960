// q8_bench.cpp -- host side of libq8bench.so (include/q8bench.h): launches
// the benchmark's measurement kernels (q8_probe.hip, a code object of their
// own embedded like the product's) on a stream the caller passes.  Bench-only:
// the product library neither links nor calls this.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/q8bench.h"
#include "../../include/q8mi.h"
#include "q8_bench_args.h"
#include "q8_bench_manifest.h"

extern "C" const unsigned char q8_bench_code_object[];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

enum Kernel {
    K_READ_2, K_READ_2_NT, K_READ_4, K_READ_4_NT, K_READ_8, K_READ_8_NT, K_READ_16, K_READ_16_NT,
    K_EMPTY, K_MFMA, K_VALU, K_MIX, K_MIX_F16, K_SPLIT_I8_VALU, K_SPLIT_I8_FMA, K_SPLIT_F32_VALU, K_COUNT
};
const char *const kNames[K_COUNT] = {
    "q8_probe_read_l2", "q8_probe_read_l2_nt", "q8_probe_read_l4", "q8_probe_read_l4_nt", "q8_probe_read_l8",
    "q8_probe_read_l8_nt", "q8_probe_read_l16", "q8_probe_read_l16_nt", "q8_probe_empty", "q8_probe_mfma",
    "q8_probe_valu", "q8_probe_mix", "q8_probe_mix_f16", "q8_probe_split_i8_valu", "q8_probe_split_i8_fma",
    "q8_probe_split_f32_valu",
};

}  // namespace

struct q8bench {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    unsigned *sink = nullptr;
};

namespace {

int launch(q8bench *b, Kernel k, unsigned grid, unsigned block, Q8ProbeArgs &a) {
    if (grid == 0) return Q8_OK;
    a.never = 0x7fc0dead;  // a NaN payload: no XOR of the data or float sum equals it by chance
    a.sink = b->sink;
    void *params[] = {&a};
    const hipError_t e = hipModuleLaunchKernel(b->fn[k], grid, 1, 1, block, 1, 1, 0, b->stream, params, nullptr);
    if (e != hipSuccess) return fail(Q8_ERR_HIP, "hip: launch of %s failed: %s", kNames[k], hipGetErrorString(e));
    return Q8_OK;
}

// A read probe: its arguments one by one, as the kernels declare them.
int launch_read(q8bench *b, Kernel k, unsigned grid, unsigned block, const uint8_t *src, long long bytes) {
    if (grid == 0) return Q8_OK;
    int threads = (int)block;
    unsigned never = 0x7fc0dead;
    unsigned *sink = b->sink;
    void *params[] = {&src, &bytes, &threads, &never, &sink};
    const hipError_t e = hipModuleLaunchKernel(b->fn[k], grid, 1, 1, block, 1, 1, 0, b->stream, params, nullptr);
    if (e != hipSuccess) return fail(Q8_ERR_HIP, "hip: launch of %s failed: %s", kNames[k], hipGetErrorString(e));
    return Q8_OK;
}

}  // namespace

extern "C" {

const char *q8bench_last_error(void) { return g_last_error.c_str(); }

const char *q8bench_build_info(void) { return Q8_BENCH_BUILD_INFO; }

int q8bench_open(void *hip_stream, q8bench **out) {
    if (!out) return fail(Q8_ERR_INVALID, "q8bench_open: null output");
    *out = nullptr;
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    int device = 0;
    hipError_t e = hipStreamGetDevice(stream, &device);
    if (e != hipSuccess) return fail(Q8_ERR_NO_DEVICE, "hip: hipStreamGetDevice failed: %s", hipGetErrorString(e));
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(Q8_ERR_NO_DEVICE, "hip: hipSetDevice failed: %s", hipGetErrorString(e));
    q8bench *b = new q8bench();
    b->device = device;
    b->stream = stream;
    int rc = Q8_OK;
    e = hipModuleLoadData(&b->module, q8_bench_code_object);
    if (e != hipSuccess) rc = fail(Q8_ERR_NO_DEVICE, "hip: hipModuleLoadData(probes) failed: %s", hipGetErrorString(e));
    for (int i = 0; i < K_COUNT && rc == Q8_OK; i++) {
        e = hipModuleGetFunction(&b->fn[i], b->module, kNames[i]);
        if (e != hipSuccess)
            rc = fail(Q8_ERR_NO_DEVICE, "hip: hipModuleGetFunction(%s) failed: %s", kNames[i], hipGetErrorString(e));
    }
    if (rc == Q8_OK) {
        e = hipMalloc(reinterpret_cast<void **>(&b->sink), 256);
        if (e != hipSuccess) rc = fail(Q8_ERR_OUT_OF_MEMORY, "hip: hipMalloc(sink) failed: %s", hipGetErrorString(e));
    }
    if (rc != Q8_OK) {
        q8bench_close(b);
        return rc;
    }
    *out = b;
    return Q8_OK;
}

void q8bench_close(q8bench *b) {
    if (!b) return;
    hipSetDevice(b->device);
    if (b->stream) hipStreamSynchronize(b->stream);
    if (b->sink) hipFree(b->sink);
    if (b->module) hipModuleUnload(b->module);
    delete b;
}

int q8bench_read(q8bench *b, uint64_t src, size_t bytes, int loads, int nontemporal, int threads) {
    if (!b) return fail(Q8_ERR_INVALID, "q8bench_read: null handle");
    if (bytes == 0 || bytes % 16 != 0 || src % 16 != 0)
        return fail(Q8_ERR_INVALID, "q8bench_read: a 16-byte aligned source and a multiple of 16 bytes");
    if (threads < 64 || threads > 1024 || threads % 64 != 0)
        return fail(Q8_ERR_INVALID, "q8bench_read: %d threads per workgroup", threads);
    const int idx = loads == 2 ? 0 : loads == 4 ? 2 : loads == 8 ? 4 : loads == 16 ? 6 : -1;
    if (idx < 0) return fail(Q8_ERR_INVALID, "q8bench_read: %d loads per lane (2, 4, 8 or 16)", loads);
    const unsigned long long per = (unsigned long long)threads * 16 * loads;
    const unsigned long long grid = (bytes + per - 1) / per;
    if (grid > 0x7fffffffULL) return fail(Q8_ERR_UNSUPPORTED, "q8bench_read: %zu bytes", bytes);
    return launch_read(b, static_cast<Kernel>(idx + (nontemporal ? 1 : 0)), (unsigned)grid, (unsigned)threads,
                       reinterpret_cast<const uint8_t *>(src), (long long)bytes);
}

int q8bench_probe(q8bench *b, int which, int iters, int workgroups, int mask) {
    if (!b) return fail(Q8_ERR_INVALID, "q8bench_probe: null handle");
    Q8ProbeArgs a{};
    if (which == Q8BENCH_EMPTY) return launch(b, K_EMPTY, 1, 64, a);
    if (iters < 2 || iters % 2 != 0 || workgroups < 1)
        return fail(Q8_ERR_INVALID, "q8bench_probe: iters must be even and >= 2, workgroups >= 1");
    a.iters = iters;
    a.mask = mask;
    switch (which) {
    case Q8BENCH_MFMA: return launch(b, K_MFMA, (unsigned)workgroups, 256, a);
    case Q8BENCH_VALU: return launch(b, K_VALU, (unsigned)workgroups, 256, a);
    case Q8BENCH_MIX: return launch(b, K_MIX, (unsigned)workgroups, 256, a);
    case Q8BENCH_MIX_F16: return launch(b, K_MIX_F16, (unsigned)workgroups, 256, a);
    case Q8BENCH_SPLIT_I8_VALU: return launch(b, K_SPLIT_I8_VALU, (unsigned)workgroups, 512, a);
    case Q8BENCH_SPLIT_I8_FMA: return launch(b, K_SPLIT_I8_FMA, (unsigned)workgroups, 512, a);
    case Q8BENCH_SPLIT_F32_VALU: return launch(b, K_SPLIT_F32_VALU, (unsigned)workgroups, 512, a);
    default: return fail(Q8_ERR_INVALID, "q8bench_probe: unknown probe %d", which);
    }
}

}  // extern "C"
