// Device allocation and rocPRIM helpers shared by the layout builders
// (included by .hip sources only).
#pragma once

#include <cstring>

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_run_length_encode.hpp>
#include <rocprim/device/device_scan.hpp>

#include "../host/hip_util.hpp"

namespace cptc {
namespace dev {

template <class T>
int dalloc(T** p, size_t n)
{
    *p = nullptr;
    if (n == 0) return CPTC_OK;
    CPTC_HIP(hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)));
    return CPTC_OK;
}

template <class T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

// RAII for temporaries inside one function.
template <class T>
struct Tmp
{
    T* p = nullptr;
    Tmp() = default;
    Tmp(const Tmp&) = delete;
    Tmp& operator=(const Tmp&) = delete;
    ~Tmp() { dfree(p); }
    int alloc(size_t n)
    {
        dfree(p);
        return dalloc(&p, n);
    }
    void reset() { dfree(p); }
};

inline int bit_width(uint64_t v)
{
    int b = 0;
    while (b < 64 && (v >> b) != 0) ++b;
    return b < 1 ? 1 : b;
}

template <class K, class V>
int sort_pairs(const K* kin, K* kout, const V* vin, V* vout, size_t n, int end_bit,
               hipStream_t s)
{
    size_t bytes = 0;
    CPTC_HIP(rocprim::radix_sort_pairs(nullptr, bytes, kin, kout, vin, vout, n, 0,
                                       unsigned(end_bit), s));
    Tmp<char> tmp;
    CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
    CPTC_HIP(rocprim::radix_sort_pairs(tmp.p, bytes, kin, kout, vin, vout, n, 0,
                                       unsigned(end_bit), s));
    return CPTC_OK;
}

template <class In, class Out>
int exclusive_sum(const In* in, Out* out, size_t n, hipStream_t s)
{
    size_t bytes = 0;
    CPTC_HIP(rocprim::exclusive_scan(nullptr, bytes, in, out, Out(0), n, rocprim::plus<Out>(), s));
    Tmp<char> tmp;
    CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
    CPTC_HIP(rocprim::exclusive_scan(tmp.p, bytes, in, out, Out(0), n, rocprim::plus<Out>(), s));
    return CPTC_OK;
}

template <class T>
int inclusive_sum(const T* in, T* out, size_t n, hipStream_t s)
{
    size_t bytes = 0;
    CPTC_HIP(rocprim::inclusive_scan(nullptr, bytes, in, out, n, rocprim::plus<T>(), s));
    Tmp<char> tmp;
    CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
    CPTC_HIP(rocprim::inclusive_scan(tmp.p, bytes, in, out, n, rocprim::plus<T>(), s));
    return CPTC_OK;
}

template <class T>
int d2h_one(T* h, const T* d, hipStream_t s)
{
    CPTC_HIP(hipMemcpyAsync(h, d, sizeof(T), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// Runs of equal keys in a sorted array: unique keys, counts, number of runs.
template <class K>
int run_length(const K* keys, size_t n, K* ukeys, uint32_t* counts, uint32_t* d_nruns,
               hipStream_t s)
{
    size_t bytes = 0;
    CPTC_HIP(rocprim::run_length_encode(nullptr, bytes, keys, n, ukeys, counts, d_nruns, s));
    Tmp<char> tmp;
    CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
    CPTC_HIP(rocprim::run_length_encode(tmp.p, bytes, keys, n, ukeys, counts, d_nruns, s));
    return CPTC_OK;
}

}  // namespace dev
}  // namespace cptc
