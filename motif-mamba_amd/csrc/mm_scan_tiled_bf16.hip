// mm_scan_tiled_bf16.hip -- the bfloat16 instances of the dstate-16 forward kernels of
// mm_scan_tiled.hip (compiled once per input type, so that the three sets build in parallel).
#define MM_TILED_TYPE bf16_t
#include "mm_scan_tiled.hip"
