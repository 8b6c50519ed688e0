// Context, error text and stream handling of the C ABI.
#include <cstdlib>

#include "common.hpp"

namespace pfr {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }

void bind(pfr_ctx* ctx) {
    require(ctx != nullptr, "null context");
    int cur = -1;
    PFR_HIP(hipGetDevice(&cur));
    if (cur != ctx->device) PFR_HIP(hipSetDevice(ctx->device));
}

}  // namespace pfr

extern "C" {

const char* pfr_last_error(void) { return pfr::g_last_error.c_str(); }

int pfr_device_count(int* count) {
    return pfr::guarded([&] {
        pfr::require(count != nullptr, "null count");
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        *count = (e == hipSuccess) ? n : 0;
    });
}

int pfr_rocm_init(int device, pfr_ctx** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output handle");
        *out = nullptr;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
            throw pfr::Error(PFR_ERR_NO_DEVICE, "no ROCm device visible");
        pfr::require(device >= 0 && device < n, "device index out of range");
        PFR_HIP(hipSetDevice(device));
        hipDeviceProp_t prop;
        PFR_HIP(hipGetDeviceProperties(&prop, device));
        std::string arch = prop.gcnArchName;
        if (arch.rfind("gfx950", 0) != 0)
            throw pfr::Error(PFR_ERR_UNSUPPORTED, "kernels are built for gfx950, device is " + arch);
        pfr::init_noalloc_workspace(device);
        auto* ctx = new pfr_ctx();
        ctx->device = device;
        ctx->num_cu = prop.multiProcessorCount;
        const char* mp = std::getenv("PFR_CSR_MERGE");
        ctx->merge = !(mp && std::string(mp) == "0");
        hipError_t e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete ctx;
            throw pfr::Error(PFR_ERR_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e));
        }
        ctx->stream = ctx->own_stream;
        *out = ctx;
    });
}

int pfr_rocm_destroy(pfr_ctx* ctx) {
    return pfr::guarded([&] {
        if (!ctx) return;
        pfr::bind(ctx);
        (void)hipStreamSynchronize(ctx->stream);
        for (auto& b : ctx->scratch) b.release();
        if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
    });
}

int pfr_ctx_get_stream(pfr_ctx* ctx, void** stream) {
    return pfr::guarded([&] {
        pfr::require(ctx && stream, "null argument");
        *stream = reinterpret_cast<void*>(ctx->stream);
    });
}

int pfr_ctx_set_stream(pfr_ctx* ctx, void* stream) {
    return pfr::guarded([&] {
        pfr::require(ctx != nullptr, "null context");
        ctx->stream = reinterpret_cast<hipStream_t>(stream);
    });
}

int pfr_synchronize(pfr_ctx* ctx) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int pfr_dev_alloc(pfr_ctx* ctx, int64_t bytes, void** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output pointer");
        *out = nullptr;
        pfr::require(bytes >= 0, "negative size");
        pfr::bind(ctx);
        PFR_HIP(hipMalloc(out, (size_t)(bytes > 0 ? bytes : 4)));
    });
}

int pfr_dev_free(pfr_ctx* ctx, void* p) {
    return pfr::guarded([&] {
        if (!p) return;
        pfr::bind(ctx);
        PFR_HIP(hipStreamSynchronize(ctx->stream));  // no kernel may still use it
        PFR_HIP(hipFree(p));
    });
}

int pfr_copy_to_device(pfr_ctx* ctx, void* dst, const void* src, int64_t bytes) {
    return pfr::guarded([&] {
        pfr::require(bytes >= 0 && (bytes == 0 || (dst && src)), "bad copy");
        pfr::bind(ctx);
        if (bytes) PFR_HIP(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, ctx->stream));
    });
}

int pfr_copy_to_host(pfr_ctx* ctx, void* dst, const void* src, int64_t bytes) {
    return pfr::guarded([&] {
        pfr::require(bytes >= 0 && (bytes == 0 || (dst && src)), "bad copy");
        pfr::bind(ctx);
        if (bytes) PFR_HIP(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

}  // extern "C"
