// Shape of the blocked order-3 residual layout, shared by the layout builder's
// caller (als3.cpp) and the kernel (mttkrp_blk.hip), which must agree on the
// block sizes: log2 of the target rows and run-level rows per block pair,
// elements per chunk (one workgroup) and the element count from which a
// block pair's run-level rows are staged in LDS.
#pragma once

#ifndef CPTC_BLK3_LG_TB
#define CPTC_BLK3_LG_TB 5
#endif
#ifndef CPTC_BLK3_LG_KB
#define CPTC_BLK3_LG_KB 4
#endif
#ifndef CPTC_BLK3_CHUNK
#define CPTC_BLK3_CHUNK 1024
#endif
#ifndef CPTC_BLK3_STAGE_MIN
#define CPTC_BLK3_STAGE_MIN 64
#endif
