// mm_scan_tiled.hip -- tiled gfx950 forward scan (placeholder: defers to the lane-per-row kernel).
#include "mm_common.h"
#include "mm_internal.h"

namespace mm {

template <typename T>
int try_launch_tiled(const mm_scan_fwd_params &, hipStream_t) {
    return MM_ERR_UNSUPPORTED;
}

template int try_launch_tiled<float>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<f16_t>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<bf16_t>(const mm_scan_fwd_params &, hipStream_t);

}  // namespace mm
