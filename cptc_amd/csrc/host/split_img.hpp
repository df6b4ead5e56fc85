// Compacted split tile images for the split-bf16 MFMA kernel, one per target
// slot (its A operand, split into bf16 hi / lo once instead of per launch),
// built from a dense FP32 tile or unit image.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>

#include "cptc_hip.h"
#include "hip_util.hpp"

namespace cptc {

struct SplitImg
{
    uint32_t* cmask = nullptr;    // ntiles x 64 (occupancy words, running counts)
    uint32_t* segoff = nullptr;   // ntiles + 1
    void* seg = nullptr;          // nseg x 16 bytes
    uint64_t nseg = 0;
    bool ready() const { return seg != nullptr; }
};

inline void free_split_img(SplitImg& g)
{
    for (void* p : {static_cast<void*>(g.cmask), static_cast<void*>(g.segoff), g.seg})
        if (p) (void)hipFree(p);
    g = SplitImg{};
}

// Slot `slot`'s image of `nt` tiles; left empty (not ready) when its segments
// exceed the kernel's 32-bit byte offsets, and the caller reads the dense image.
inline int build_split_img(const float* tiles, size_t nt, int slot, SplitImg& g, hipStream_t s)
{
    free_split_img(g);
    if (nt == 0 || !tiles) return CPTC_OK;
    struct Guard
    {
        SplitImg& g;
        bool ok = false;
        ~Guard()
        {
            if (!ok) free_split_img(g);
        }
    } guard{g};
    CPTC_HIP(hipMalloc(&g.cmask, nt * 64 * sizeof(uint32_t)));
    CPTC_HIP(hipMalloc(&g.segoff, (nt + 1) * sizeof(uint32_t)));
    CPTC_TRY(cptc_dense_tiles_compact3_mask(tiles, nt, slot, g.cmask, g.segoff, &g.nseg, s));
    if (g.nseg * 16u >= 0xFFFFFFF0ull) return CPTC_OK;
    CPTC_HIP(hipMalloc(&g.seg, std::max<uint64_t>(g.nseg, 1) * 16));
    CPTC_TRY(cptc_dense_tiles_compact3_fill(tiles, nt, slot, g.cmask, g.segoff, g.seg, s));
    guard.ok = true;
    return CPTC_OK;
}

}  // namespace cptc
