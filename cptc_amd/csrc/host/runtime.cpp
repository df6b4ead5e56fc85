// Library status, error strings and the per-device scratch cache.
#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "hip_util.hpp"

namespace cptc {

namespace {
thread_local char g_err[1024] = "";

struct ScratchBuf
{
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct ScratchTable
{
    std::mutex mu;
    std::vector<std::vector<ScratchBuf>> per_dev;
    ~ScratchTable()
    {
        // Process exit: the runtime may already be torn down; freeing is
        // best effort and its status is ignored.
        for (auto& d : per_dev)
            for (auto& b : d)
                if (b.ptr) (void)hipFree(b.ptr);
    }
};

ScratchTable& table()
{
    static ScratchTable t;
    return t;
}

std::atomic<uint64_t> g_scratch_gen{0};
}  // namespace

uint64_t scratch_generation() { return g_scratch_gen.load(); }

void set_error(const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int scratch_get(int slot, size_t bytes, void** out)
{
    int dev = 0;
    CPTC_HIP(hipGetDevice(&dev));
    ScratchTable& t = table();
    std::lock_guard<std::mutex> lk(t.mu);
    if (size_t(dev) >= t.per_dev.size()) t.per_dev.resize(size_t(dev) + 1);
    auto& v = t.per_dev[size_t(dev)];
    if (v.size() < SCR_NSLOTS) v.resize(SCR_NSLOTS);
    ScratchBuf& b = v[size_t(slot)];
    if (b.bytes < bytes)
    {
        if (b.ptr)
        {
            // The old buffer may still be read by queued work on any stream.
            CPTC_HIP(hipDeviceSynchronize());
            CPTC_HIP(hipFree(b.ptr));
            b.ptr = nullptr;
            b.bytes = 0;
        }
        size_t want = bytes < 4096 ? 4096 : bytes;
        want = (want + 4095) & ~size_t(4095);
        CPTC_HIP(hipMalloc(&b.ptr, want));
        b.bytes = want;
        ++g_scratch_gen;   // captured graphs that hold the old address are stale
    }
    *out = b.ptr;
    return CPTC_OK;
}

}  // namespace cptc

extern "C" const char* cptc_version(void) { return "cptc-mi355x 0.1 (gfx950)"; }

extern "C" const char* cptc_last_error(void) { return cptc::g_err; }

extern "C" int cptc_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int cptc_dev_malloc(size_t bytes, void** d_ptr)
{
    CPTC_REQUIRE(d_ptr, CPTC_ERR_ARG, "cptc_dev_malloc: null out pointer");
    *d_ptr = nullptr;
    CPTC_HIP(hipMalloc(d_ptr, bytes ? bytes : 1));
    return CPTC_OK;
}

extern "C" int cptc_dev_free(void* d_ptr)
{
    if (d_ptr) CPTC_HIP(hipFree(d_ptr));
    return CPTC_OK;
}

extern "C" int cptc_dev_upload(void* d_dst, const void* src, size_t bytes)
{
    if (bytes == 0) return CPTC_OK;
    CPTC_REQUIRE(d_dst && src, CPTC_ERR_ARG, "cptc_dev_upload: null pointer");
    CPTC_HIP(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice));
    return CPTC_OK;
}

extern "C" int cptc_dev_download(void* dst, const void* d_src, size_t bytes)
{
    if (bytes == 0) return CPTC_OK;
    CPTC_REQUIRE(dst && d_src, CPTC_ERR_ARG, "cptc_dev_download: null pointer");
    CPTC_HIP(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost));
    return CPTC_OK;
}

extern "C" int cptc_dev_memset(void* d_ptr, int value, size_t bytes)
{
    if (bytes == 0) return CPTC_OK;
    CPTC_REQUIRE(d_ptr, CPTC_ERR_ARG, "cptc_dev_memset: null pointer");
    CPTC_HIP(hipMemset(d_ptr, value, bytes));
    return CPTC_OK;
}

extern "C" int cptc_dev_sync(void)
{
    CPTC_HIP(hipDeviceSynchronize());
    CPTC_HIP(hipGetLastError());
    return CPTC_OK;
}
