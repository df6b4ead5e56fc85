// Error plumbing shared by the C ABI: every entry point returns an int status
// and records a message retrievable with cptc_last_error().
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "cptc_hip.h"

namespace cptc {

void set_error(const char* fmt, ...);

// Kernel launches and HIP calls inside entry points.
#define CPTC_HIP(call)                                                                     \
    do                                                                                     \
    {                                                                                      \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
        {                                                                                  \
            ::cptc::set_error("%s:%d %s -> %s", __FILE__, __LINE__, #call,                 \
                              hipGetErrorString(e_));                                      \
            return CPTC_ERR_HIP;                                                           \
        }                                                                                  \
    } while (0)

#define CPTC_LAUNCHED()                                                                    \
    do                                                                                     \
    {                                                                                      \
        hipError_t e_ = hipGetLastError();                                                 \
        if (e_ != hipSuccess)                                                              \
        {                                                                                  \
            ::cptc::set_error("%s:%d launch -> %s", __FILE__, __LINE__,                    \
                              hipGetErrorString(e_));                                      \
            return CPTC_ERR_HIP;                                                           \
        }                                                                                  \
    } while (0)

#define CPTC_REQUIRE(cond, code, ...)                                                      \
    do                                                                                     \
    {                                                                                      \
        if (!(cond))                                                                       \
        {                                                                                  \
            ::cptc::set_error(__VA_ARGS__);                                                \
            return (code);                                                                 \
        }                                                                                  \
    } while (0)

#define CPTC_TRY(expr)                                                                     \
    do                                                                                     \
    {                                                                                      \
        int rc_ = (expr);                                                                  \
        if (rc_ != CPTC_OK) return rc_;                                                    \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned grid_for(size_t n, unsigned block, unsigned cap = 1u << 20)
{
    size_t g = (n + block - 1) / block;
    if (g == 0) g = 1;
    if (g > cap) g = cap;
    return unsigned(g);
}

// Compute units of device `dev`, queried once per device (0..63; others are
// queried every time) and kept in atomics, so concurrent first calls are
// safe; 256 if the query fails.
inline int cu_count(int dev)
{
    static std::atomic<int> cache[64];
    if (dev >= 0 && dev < 64)
        if (const int c = cache[dev].load(std::memory_order_relaxed); c > 0) return c;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Raises the dynamic-LDS limit of kernels once per device (the attribute
// belongs to the device that is current), safe against concurrent first
// calls:  static cptc::DeviceOnce once;
//         CPTC_HIP(once.lds_limit({kernel...}, bytes));
class DeviceOnce
{
public:
    hipError_t lds_limit(std::initializer_list<const void*> kernels, int bytes)
    {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        std::lock_guard<std::mutex> lk(mu_);
        if (size_t(dev) >= done_.size()) done_.resize(size_t(dev) + 1, 0);
        if (done_[size_t(dev)]) return hipSuccess;
        for (const void* k : kernels)
        {
            e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
            if (e != hipSuccess) return e;
        }
        done_[size_t(dev)] = 1;
        return hipSuccess;
    }

private:
    std::mutex mu_;
    std::vector<char> done_;
};

// Library-owned device scratch, one growing buffer per (device, slot),
// freed at process exit.  Slots separate buffers that are live at the same
// time within one entry point.
enum ScratchSlot { SCR_GRAM = 0, SCR_PINV, SCR_FLAGS, SCR_REDUCE, SCR_LAYOUT_A, SCR_LAYOUT_B, SCR_NSLOTS };
int scratch_get(int slot, size_t bytes, void** out);
// Changes whenever a scratch buffer is (re)allocated: a captured HIP graph
// that holds scratch addresses is replayed only while it is unchanged.
uint64_t scratch_generation();

}  // namespace cptc
