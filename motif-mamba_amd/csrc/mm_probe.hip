// mm_probe.hip -- instruction-issue probes for the roofline of the scan kernels (libmm_probe.so).
//
// Not part of the scan library: bench.py loads this library to measure, on the box it runs on and
// in the same run, how fast one MI355X SIMD issues the instructions a selective-scan state update
// is made of. Each probe kernel runs `iters` rounds of a fixed, fully unrolled instruction block
// over 8 independent register chains per lane (enough independent work per wave to hide the
// latency of every instruction measured), in workgroups of four waves. With `blocks` = compute
// units x W, every SIMD runs W waves, so the kernel time gives the SIMD's issue rate for that
// block. The instructions are inline asm (volatile, register-tied), so the compiler neither removes
// nor reorders them; every chain ends in one vector store per lane. Lane 0 of each wave also stores
// the shader-clock and constant-clock ticks its loop took, from which the host derives the clock.
//
// Kinds (per round and lane, 8 chains):
//   0  32 x v_fma_f32                                   (VALU, VGPR operands)
//   1  32 x v_exp_f32                                   (transcendental)
//   2  32 x v_mul_f32_dpp row_newbcast                  (VALU with a DPP row broadcast)
//   3   8 x v_exp_f32 + 32 x v_fma_f32, interleaved     (one wave: do they overlap?)
//   4  waves alternate: even waves kind 1, odd waves kind 0 (different waves: do they overlap?)
//   5  32 x v_fmac_f32_dpp row_newbcast
//   6  16 x v_exp_f32 + 16 x v_fma_f32, interleaved
//   7  the dstate-16 forward's scan core, 16 state updates per lane and round as in the kernel:
//      per step and state exp2(dt' A), B dt'u by DPP row broadcast, the state FMA, y += C h by DPP
//   8  kind 7 with plain VGPR operands instead of the DPP broadcasts
//   9  kind 7 without the exp2 (the decay taken as the exp argument itself)
// Every loop is bounded by `iters`; no kernel waits on another wave.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

#define FMA(a) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(a) : "v"(m), "v"(c))
#define EXP(a) asm volatile("v_exp_f32 %0, %0" : "+v"(a))
#define MULDPP(a) asm volatile("v_mul_f32_dpp %0, %1, %0 row_newbcast:3 row_mask:0xf bank_mask:0xf" : "+v"(a) : "v"(src))
#define FMACDPP(a) asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:5 row_mask:0xf bank_mask:0xf" : "+v"(a) : "v"(src), "v"(m))

template <int LANE>
__device__ __forceinline__ float row_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + LANE, 0xf, 0xf, false));
}
template <int LANE>
__device__ __forceinline__ void fmac_row_bcast(float &acc, float src, float x) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(src), "v"(x), "i"(LANE));
}

// One round of kind 7/8/9: 4 steps x 2 states. dts/dus are the step's dt' and dt'u (as the scan
// reads them from LDS), bv/cv hold B and C values that the DPP forms broadcast along the row.
template <int KIND, int R, int J>
__device__ __forceinline__ void scan_prep(const float (&At)[2], const float (&dts)[4], const float (&dus)[4],
                                          const float (&bv)[4], float (&av)[4][2], float (&bbv)[4][2]) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float arg = dts[J] * At[k];
        av[J][k] = KIND == 9 ? arg : __builtin_amdgcn_exp2f(arg);
    }
    if constexpr (KIND == 8) {
        bbv[J][0] = bv[J] * dus[J];
        bbv[J][1] = bv[(J + 1) & 3] * dus[J];
    } else {
        bbv[J][0] = row_bcast<(R * 4 + J) & 7>(bv[J]) * dus[J];
        bbv[J][1] = row_bcast<8 + ((R * 4 + J) & 7)>(bv[J]) * dus[J];
    }
}

template <int KIND, int R, int J>
__device__ __forceinline__ void scan_step(float (&h)[2], const float (&cv)[4], const float (&av)[4][2],
                                          const float (&bbv)[4][2], float (&pv)[4]) {
    h[0] = __builtin_fmaf(av[J][0], h[0], bbv[J][0]);
    h[1] = __builtin_fmaf(av[J][1], h[1], bbv[J][1]);
    float acc;
    if constexpr (KIND == 8) {
        acc = cv[J] * h[0];
        acc = __builtin_fmaf(cv[(J + 1) & 3], h[1], acc);
    } else {
        acc = row_bcast<(R * 4 + J) & 7>(cv[J]) * h[0];
        fmac_row_bcast<8 + ((R * 4 + J) & 7)>(acc, cv[J], h[1]);
    }
    pv[J] = acc;
}

template <int KIND, int R>
__device__ __forceinline__ void scan_round(float (&h)[2], const float (&At)[2], const float (&dts)[4], const float (&dus)[4],
                                           const float (&bv)[4], const float (&cv)[4], float &ysum) {
    float av[4][2], bbv[4][2], pv[4];
    scan_prep<KIND, R, 0>(At, dts, dus, bv, av, bbv);
    scan_prep<KIND, R, 1>(At, dts, dus, bv, av, bbv);
    scan_prep<KIND, R, 2>(At, dts, dus, bv, av, bbv);
    scan_prep<KIND, R, 3>(At, dts, dus, bv, av, bbv);
    scan_step<KIND, R, 0>(h, cv, av, bbv, pv);
    scan_step<KIND, R, 1>(h, cv, av, bbv, pv);
    scan_step<KIND, R, 2>(h, cv, av, bbv, pv);
    scan_step<KIND, R, 3>(h, cv, av, bbv, pv);
    // the y partials leave the round (the kernel stores them to LDS with one 16-byte write)
    asm volatile("" ::"v"(pv[0]), "v"(pv[1]), "v"(pv[2]), "v"(pv[3]));
    ysum = pv[3];
}

template <int KIND>
__global__ void __launch_bounds__(256) scan_core_probe(int iters, float *out, uint64_t *ticks) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int wave = tid >> 6;
    const float f = threadIdx.x * 1e-6f;
    float h[2] = {0.f, 0.f};
    const float At[2] = {-1.4427f - f, -2.885f + f};
    float dts[4] = {0.01f + f, 0.02f, 0.03f, 0.04f - f}, dus[4] = {0.1f, 0.2f + f, 0.3f, 0.4f};
    float bv[4] = {1.f + f, 0.5f, -0.5f, 0.25f}, cv[4] = {0.3f, -0.2f + f, 0.1f, 0.7f};
    float ysum = 0.f;
    // Two wait states between the last VALU writes of the DPP sources and their first DPP read.
#pragma unroll
    for (int k = 0; k < 4; ++k) asm volatile("s_nop 1" : "+v"(bv[k]), "+v"(cv[k]));
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t w0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        // the step values change every round, as the LDS reads of the kernel make them
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(dts[j]), "+v"(dus[j]));
        scan_round<KIND, 0>(h, At, dts, dus, bv, cv, ysum);
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(dts[j]), "+v"(dus[j]));
        scan_round<KIND, 1>(h, At, dts, dus, bv, cv, ysum);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t w1 = __builtin_amdgcn_s_memrealtime();
    out[tid] = h[0] + h[1] + ysum;
    if ((threadIdx.x & 63) == 0) {
        ticks[2 * wave] = t1 - t0;
        ticks[2 * wave + 1] = w1 - w0;
    }
}

template <int KIND>
__global__ void __launch_bounds__(256) issue_probe(int iters, float *out, uint64_t *ticks) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int wave = tid >> 6;
    float x0 = 0.999f + threadIdx.x * 1e-7f, x1 = x0 + 1e-6f, x2 = x0 + 2e-6f, x3 = x0 + 3e-6f;
    float x4 = x0 + 4e-6f, x5 = x0 + 5e-6f, x6 = x0 + 6e-6f, x7 = x0 + 7e-6f;
    float e0 = -1.f - threadIdx.x * 1e-6f, e1 = e0 - 0.01f, e2 = e0 - 0.02f, e3 = e0 - 0.03f;
    float e4 = e0 - 0.04f, e5 = e0 - 0.05f, e6 = e0 - 0.06f, e7 = e0 - 0.07f;
    float m = 0.9999f, c = 1e-4f;
    float src = 1.0000001f;
    // src, m and c are read by DPP / VALU instructions: two wait states after their last VALU write.
    asm volatile("s_nop 4" : "+v"(src), "+v"(m), "+v"(c));
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t w0 = __builtin_amdgcn_s_memrealtime();
    const int kind = KIND == 4 ? (wave & 1 ? 0 : 1) : KIND;
    for (int it = 0; it < iters; ++it) {
        if (kind == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                FMA(x0); FMA(x1); FMA(x2); FMA(x3); FMA(x4); FMA(x5); FMA(x6); FMA(x7);
            }
        } else if (kind == 1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                EXP(e0); EXP(e1); EXP(e2); EXP(e3); EXP(e4); EXP(e5); EXP(e6); EXP(e7);
            }
        } else if (kind == 2) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                MULDPP(x0); MULDPP(x1); MULDPP(x2); MULDPP(x3); MULDPP(x4); MULDPP(x5); MULDPP(x6); MULDPP(x7);
            }
        } else if (kind == 3) {
            EXP(e0); FMA(x0); FMA(x1); FMA(x2); FMA(x3);
            EXP(e1); FMA(x4); FMA(x5); FMA(x6); FMA(x7);
            EXP(e2); FMA(x0); FMA(x1); FMA(x2); FMA(x3);
            EXP(e3); FMA(x4); FMA(x5); FMA(x6); FMA(x7);
            EXP(e4); FMA(x0); FMA(x1); FMA(x2); FMA(x3);
            EXP(e5); FMA(x4); FMA(x5); FMA(x6); FMA(x7);
            EXP(e6); FMA(x0); FMA(x1); FMA(x2); FMA(x3);
            EXP(e7); FMA(x4); FMA(x5); FMA(x6); FMA(x7);
        } else if (kind == 5) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                FMACDPP(x0); FMACDPP(x1); FMACDPP(x2); FMACDPP(x3); FMACDPP(x4); FMACDPP(x5); FMACDPP(x6); FMACDPP(x7);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                EXP(e0); FMA(x0); EXP(e1); FMA(x1); EXP(e2); FMA(x2); EXP(e3); FMA(x3);
                EXP(e4); FMA(x4); EXP(e5); FMA(x5); EXP(e6); FMA(x6); EXP(e7); FMA(x7);
            }
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t w1 = __builtin_amdgcn_s_memrealtime();
    out[tid] = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7 + e0 + e1 + e2 + e3 + e4 + e5 + e6 + e7;
    if ((threadIdx.x & 63) == 0) {
        ticks[2 * wave] = t1 - t0;
        ticks[2 * wave + 1] = w1 - w0;
    }
}

#undef FMA
#undef EXP
#undef MULDPP
#undef FMACDPP

}  // namespace

extern "C" {

// Launches probe `kind` (0-9) as `blocks` workgroups of 256 lanes for `iters` rounds on `stream`.
// `out` holds blocks * 256 floats; `ticks` holds 2 x 64-bit counters per wave (blocks * 8 values):
// shader-clock ticks, then constant-clock ticks, of the wave's loop. Returns 0 or a hipError_t.
int mm_probe_launch(int kind, int blocks, int iters, float *out, uint64_t *ticks, void *stream) {
    if (blocks <= 0 || blocks > 65536 || iters <= 0 || !out || !ticks) return int(hipErrorInvalidValue);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (kind) {
        case 0: hipLaunchKernelGGL(issue_probe<0>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 1: hipLaunchKernelGGL(issue_probe<1>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 2: hipLaunchKernelGGL(issue_probe<2>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 3: hipLaunchKernelGGL(issue_probe<3>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 4: hipLaunchKernelGGL(issue_probe<4>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 5: hipLaunchKernelGGL(issue_probe<5>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 6: hipLaunchKernelGGL(issue_probe<6>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 7: hipLaunchKernelGGL(scan_core_probe<7>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 8: hipLaunchKernelGGL(scan_core_probe<8>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        case 9: hipLaunchKernelGGL(scan_core_probe<9>, dim3(blocks), dim3(256), 0, s, iters, out, ticks); break;
        default: return int(hipErrorInvalidValue);
    }
    return int(hipGetLastError());
}

// Compute units of the current device, and the constant (wall) clock rate in kHz.
int mm_probe_device(int *cus, int *wall_khz) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(wall_khz, hipDeviceAttributeWallClockRate, dev);
    return int(e);
}

}  // extern "C"
