// mm_norm.hip -- gfx950 row RMSNorm, y = x * w / sqrt(mean(x^2) + eps) over the channel dimension
// of a (n0, cols, n2) tensor (the rms_norm_forward of selective_scan_interface.py:217-234 that
// MambaInnerFn applies to B, C and delta).
//
// HBM-bound: each element is read twice (sum of squares, then scale) and written once. A block has
// 64 lanes along n2 (adjacent positions of the scan layout, so each access is one contiguous row
// segment) and kGroups waves that split the channels; the partial sums meet in LDS.
#include <hip/hip_runtime.h>

#include "mm_common.h"
#include "mm_internal.h"
#include "mm_norm.h"

namespace mm {
namespace norm {

constexpr int kLanes = 64;
constexpr int kGroups = 4;

__device__ __forceinline__ float load_w(const void *p, mm_dtype dt, int64_t i) {
    switch (dt) {
        case MM_FLOAT32: return reinterpret_cast<const float *>(p)[i];
        case MM_FLOAT16: return to_f32(reinterpret_cast<const f16_t *>(p)[i]);
        default: return to_f32(reinterpret_cast<const bf16_t *>(p)[i]);
    }
}

template <typename T>
__global__ void __launch_bounds__(kLanes * kGroups)
rms_norm_kernel(const mm_rms_norm_params p) {
    __shared__ float sSum[kGroups][kLanes];
    const int lane = threadIdx.x % kLanes, grp = threadIdx.x / kLanes;
    const int64_t i2 = int64_t(blockIdx.x) * kLanes + lane;
    const int64_t i0 = blockIdx.y;
    const bool live = i2 < p.n2;
    const T *xr = reinterpret_cast<const T *>(p.x) + i0 * p.x_stride0 + (live ? i2 : 0) * p.x_stride2;
    T *orow = reinterpret_cast<T *>(p.out) + i0 * p.out_stride0 + (live ? i2 : 0) * p.out_stride2;
    float ss = 0.f;
    if (live)
        for (int64_t c = grp; c < p.cols; c += kGroups) {
            const float v = to_f32(xr[c * p.x_stride_c]);
            ss = __builtin_fmaf(v, v, ss);
        }
    sSum[grp][lane] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) tot += sSum[g][lane];
    const float rstd = 1.f / sqrtf(tot / float(p.cols) + p.eps);
    if (!live) return;
    for (int64_t c = grp; c < p.cols; c += kGroups) {
        const float v = to_f32(xr[c * p.x_stride_c]);
        orow[c * p.out_stride_c] = from_f32<T>(v * rstd * load_w(p.weight, p.wtype, c * p.weight_stride));
    }
}

template <typename T>
int launch(const mm_rms_norm_params &p, hipStream_t s) {
    dim3 grid(unsigned((p.n2 + kLanes - 1) / kLanes), unsigned(p.n0));
    hipLaunchKernelGGL(rms_norm_kernel<T>, grid, dim3(kLanes * kGroups), 0, s, p);
    return launch_status("rms_norm");
}

}  // namespace norm
}  // namespace mm

extern "C" int mm_rms_norm_fwd(const mm_rms_norm_params *params, void *stream) {
    using namespace mm;
    if (!params) return set_error(MM_ERR_INVALID_ARGUMENT, "mm_rms_norm_fwd: params is NULL");
    const mm_rms_norm_params &p = *params;
    auto ok = [](mm_dtype t) { return t == MM_FLOAT32 || t == MM_FLOAT16 || t == MM_BFLOAT16; };
    if (!ok(p.itype) || !ok(p.wtype)) return set_error(MM_ERR_INVALID_ARGUMENT, "mm_rms_norm_fwd: unknown dtype");
    if (p.n0 < 0 || p.cols < 0 || p.n2 < 0) return set_error(MM_ERR_INVALID_ARGUMENT, "mm_rms_norm_fwd: negative size");
    if (!(p.eps >= 0.f)) return set_error(MM_ERR_INVALID_ARGUMENT, "mm_rms_norm_fwd: eps must be >= 0");
    if (p.n0 > 65535) return set_error(MM_ERR_UNSUPPORTED, "mm_rms_norm_fwd: n0 must be <= 65535");
    if (p.n0 == 0 || p.cols == 0 || p.n2 == 0) return MM_OK;
    if (!p.x || !p.weight || !p.out) return set_error(MM_ERR_INVALID_ARGUMENT, "mm_rms_norm_fwd: x, weight and out are required");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return norm::launch<float>(p, s);
        case MM_FLOAT16: return norm::launch<f16_t>(p, s);
        default: return norm::launch<bf16_t>(p, s);
    }
}
