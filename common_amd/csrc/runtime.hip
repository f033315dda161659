// HIP data/compute context and memory provider behind the C-ABI.
//
// Plays the role of the reference's DataContext / ComputeContext / MemoryProvider trio
// (base/code/src/main/java/io/almostrealism/code/DataContext.java:81-88,
//  ComputeContext.java:89,133, MemoryProvider.java:60-188) for one GPU.
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "ar_hip_internal.h"

namespace {
thread_local char g_last_error[1024] = "";
}

thread_local LaunchTiming* g_launch_timing = nullptr;

// AR_HIP_LOG=1 (read once): every error message set for a caller is also written to stderr, the
// library's counterpart of the reference's verbose hardware logging flags (SystemUtils.getProperty
// over AR_* variables, base/io/src/main/java/org/almostrealism/io/SystemUtils.java:180-237).
static bool log_errors() {
    static const bool on = [] {
        const char* v = getenv("AR_HIP_LOG");
        return v && *v && strcmp(v, "0") != 0 && strcmp(v, "false") != 0;
    }();
    return on;
}

void ar_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    if (log_errors()) fprintf(stderr, "[ar_hip] %s\n", g_last_error);
}

void ar_log(const char* fmt, ...) {
    if (!log_errors()) return;
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    fprintf(stderr, "[ar_hip] %s\n", buf);
}

void ar_clear_error() { g_last_error[0] = '\0'; }

// AR_HIP_CHECK_PTRS=1 (read once): before the launches of the decode path, every device pointer
// argument is checked, with the extent its kernel reads or writes, against the HIP allocation that
// holds it (hipMemGetAddressRange); a pointer outside any allocation, or an extent past the end of
// its allocation, refuses the launch with AR_HIP_ERR_INVALID.  A debugging aid, off by default.
namespace {
std::atomic<unsigned long long> g_ptr_checks{0};
}

bool ar_check_ptrs_enabled() {
    static const bool on = [] {
        const char* v = getenv("AR_HIP_CHECK_PTRS");
        return v && *v && strcmp(v, "0") != 0 && strcmp(v, "false") != 0;
    }();
    return on;
}

int ar_check_range(const void* p, size_t bytes, const char* kernel, const char* what) {
    if (!ar_check_ptrs_enabled() || !p || !bytes) return AR_HIP_OK;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    const hipError_t e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
    g_ptr_checks.fetch_add(1, std::memory_order_relaxed);
    if (e != hipSuccess || !base) {
        ar_set_error("%s: %s %p is not inside a device allocation (%s)", kernel, what, p, hipGetErrorString(e));
        return AR_HIP_ERR_INVALID;
    }
    const uintptr_t b = reinterpret_cast<uintptr_t>(base), a = reinterpret_cast<uintptr_t>(p);
    if (a < b || a + bytes > b + size) {
        ar_set_error("%s: %s [%p, +%zu) leaves its allocation [%p, +%zu)", kernel, what, p, bytes, base, size);
        return AR_HIP_ERR_INVALID;
    }
    return AR_HIP_OK;
}

extern "C" int ar_hip_pointer_checks(unsigned long long* checked) {
    AR_CHECK_ARG(checked, "null argument");
    *checked = ar_check_ptrs_enabled() ? g_ptr_checks.load(std::memory_order_relaxed) : 0ull;
    return AR_HIP_OK;
}

extern "C" const char* ar_hip_last_error(void) { return g_last_error; }

extern "C" const char* ar_hip_version(void) { return "ar-hip 0.1 gfx950"; }

extern "C" int ar_hip_device_count(int* count) {
    AR_CHECK_ARG(count, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        ar_set_error("hipGetDeviceCount: %s", hipGetErrorString(e));
        return AR_HIP_ERR_NO_DEVICE;
    }
    *count = n;
    return AR_HIP_OK;
}

extern "C" int ar_hip_init(int device, ar_hip_ctx** out) {
    AR_CHECK_ARG(out, "out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        ar_set_error("no HIP device available (%s)", e == hipSuccess ? "0 devices" : hipGetErrorString(e));
        return AR_HIP_ERR_NO_DEVICE;
    }
    if (device < 0) {  // the device AR_HIP_DEVICE names (default 0)
        const char* v = getenv("AR_HIP_DEVICE");
        char* end = nullptr;
        const long d = v && *v ? strtol(v, &end, 10) : 0;
        AR_CHECK_ARG(!v || !*v || (*end == '\0' && d >= 0 && d < n), "AR_HIP_DEVICE='%s' is not a device in [0,%d)",
                     v ? v : "", n);
        device = (int)d;
    }
    AR_CHECK_ARG(device >= 0 && device < n, "device %d out of range [0,%d)", device, n);
    AR_HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    AR_HIP_TRY(hipGetDeviceProperties(&prop, device));
    auto* ctx = new ar_hip_ctx();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    ctx->hbm_bytes = prop.totalGlobalMem;
    // Default-priority, non-blocking stream: all work of this context is ordered on it.
    hipError_t se = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (se != hipSuccess) {
        ar_set_error("hipStreamCreateWithFlags: %s", hipGetErrorString(se));
        delete ctx;
        return AR_HIP_ERR_HIP;
    }
    const int rc = ar_ops_init(ctx);
    if (rc != AR_HIP_OK) {
        hipStreamDestroy(ctx->stream);
        delete ctx;
        return rc;
    }
    *out = ctx;
    return AR_HIP_OK;
}

extern "C" int ar_hip_destroy(ar_hip_ctx* ctx) {
    if (!ctx) return AR_HIP_OK;
    ar_ops_release(ctx);
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    gemm_blas_release(ctx);
    for (auto& kv : ctx->device_allocs) hipFree(kv.first);
    for (auto& kv : ctx->host_allocs) hipHostFree(kv.first);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return AR_HIP_OK;
}

extern "C" int ar_hip_synchronize(ar_hip_ctx* ctx) {
    AR_CHECK_ARG(ctx, "ctx is null");
    AR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_device_info(ar_hip_ctx* ctx, int* num_cus, size_t* hbm_bytes, char* name, int name_len) {
    AR_CHECK_ARG(ctx, "ctx is null");
    if (num_cus) *num_cus = ctx->num_cus;
    if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
    if (name && name_len > 0) {
        hipDeviceProp_t prop;
        AR_HIP_TRY(hipGetDeviceProperties(&prop, ctx->device));
        snprintf(name, (size_t)name_len, "%s", prop.gcnArchName);
    }
    return AR_HIP_OK;
}

int ar_device_slot(hipStream_t stream) {
    int dev = -1;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return -1;
    return dev >= 0 && dev < kMaxDevices ? dev : -1;
}

int ar_device_cus(hipStream_t stream) {
    static std::atomic<int> cache[kMaxDevices];
    int dev = -1;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return 256;
    const int slot = dev >= 0 && dev < kMaxDevices ? dev : -1;
    int n = slot >= 0 ? cache[slot].load(std::memory_order_relaxed) : 0;
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    if (slot >= 0) cache[slot].store(n, std::memory_order_relaxed);
    return n;
}

int ar_ctx_alloc(ar_hip_ctx* ctx, size_t bytes, void** out) {
    AR_CHECK_ARG(ctx && out, "null argument");
    AR_CHECK_ARG(bytes > 0, "allocation of 0 bytes");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        ar_set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        return AR_HIP_ERR_HIP;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->device_allocs[p] = bytes;
    ctx->device_bytes += bytes;
    *out = p;
    return AR_HIP_OK;
}

int ar_ctx_free(ar_hip_ctx* ctx, void* p) {
    AR_CHECK_ARG(ctx, "ctx is null");
    if (!p) return AR_HIP_OK;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        auto it = ctx->device_allocs.find(p);
        if (it == ctx->device_allocs.end()) {
            ar_set_error("pointer %p is not owned by this memory provider", p);
            return AR_HIP_ERR_NOT_FOUND;
        }
        ctx->device_bytes -= it->second;
        ctx->device_allocs.erase(it);
    }
    AR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    AR_HIP_TRY(hipFree(p));
    return AR_HIP_OK;
}

namespace {
struct UncachedBlock {
    int device;
    size_t bytes;
    void* p;
    bool used;
};
std::mutex g_uncached_mu;
std::vector<UncachedBlock> g_uncached;  // every uncached block of the process, never freed
}  // namespace

int ar_uncached_get(int device, size_t bytes, void** out) {
    AR_CHECK_ARG(out && bytes > 0, "uncached allocation: bad arguments");
    std::lock_guard<std::mutex> lk(g_uncached_mu);
    UncachedBlock* best = nullptr;
    for (auto& b : g_uncached)
        if (!b.used && b.device == device && b.bytes >= bytes && (!best || b.bytes < best->bytes)) best = &b;
    if (!best) {
        void* p = nullptr;
        hipError_t e = hipExtMallocWithFlags(&p, bytes, hipDeviceMallocUncached);
        if (e != hipSuccess) {
            ar_set_error("uncached allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
            return AR_HIP_ERR_HIP;
        }
        g_uncached.push_back({device, bytes, p, false});
        best = &g_uncached.back();
    }
    best->used = true;
    *out = best->p;
    return AR_HIP_OK;
}

void ar_uncached_put(void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(g_uncached_mu);
    for (auto& b : g_uncached)
        if (b.p == p) b.used = false;
}

extern "C" int ar_hip_alloc(ar_hip_ctx* ctx, size_t bytes, void** device_ptr) {
    return ar_ctx_alloc(ctx, bytes, device_ptr);
}

extern "C" int ar_hip_free(ar_hip_ctx* ctx, void* device_ptr) { return ar_ctx_free(ctx, device_ptr); }

extern "C" int ar_hip_host_alloc(ar_hip_ctx* ctx, size_t bytes, void** pinned_ptr) {
    AR_CHECK_ARG(ctx && pinned_ptr, "null argument");
    AR_CHECK_ARG(bytes > 0, "allocation of 0 bytes");
    void* p = nullptr;
    AR_HIP_TRY(hipHostMalloc(&p, bytes, hipHostMallocDefault));
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->host_allocs[p] = bytes;
    *pinned_ptr = p;
    return AR_HIP_OK;
}

extern "C" int ar_hip_host_free(ar_hip_ctx* ctx, void* pinned_ptr) {
    AR_CHECK_ARG(ctx, "ctx is null");
    if (!pinned_ptr) return AR_HIP_OK;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        auto it = ctx->host_allocs.find(pinned_ptr);
        if (it == ctx->host_allocs.end()) {
            ar_set_error("pinned pointer %p is not owned by this memory provider", pinned_ptr);
            return AR_HIP_ERR_NOT_FOUND;
        }
        ctx->host_allocs.erase(it);
    }
    AR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    AR_HIP_TRY(hipHostFree(pinned_ptr));
    return AR_HIP_OK;
}

extern "C" int ar_hip_memcpy_h2d(ar_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AR_CHECK_ARG(ctx && (bytes == 0 || (dst && src)), "null argument");
    if (!bytes) return AR_HIP_OK;
    AR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_memcpy_d2h(ar_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AR_CHECK_ARG(ctx && (bytes == 0 || (dst && src)), "null argument");
    if (!bytes) return AR_HIP_OK;
    AR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_memcpy_d2d(ar_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AR_CHECK_ARG(ctx && (bytes == 0 || (dst && src)), "null argument");
    if (!bytes) return AR_HIP_OK;
    AR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_memset(ar_hip_ctx* ctx, void* dst, int value, size_t bytes) {
    AR_CHECK_ARG(ctx && (bytes == 0 || dst), "null argument");
    if (!bytes) return AR_HIP_OK;
    AR_HIP_TRY(hipMemsetAsync(dst, value, bytes, ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_allocated_bytes(ar_hip_ctx* ctx, size_t* bytes) {
    AR_CHECK_ARG(ctx && bytes, "null argument");
    std::lock_guard<std::mutex> lk(ctx->mu);
    *bytes = ctx->device_bytes;
    return AR_HIP_OK;
}
