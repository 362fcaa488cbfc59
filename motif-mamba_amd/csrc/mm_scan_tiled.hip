// mm_scan_tiled.hip -- the gfx950 forward selective scan for dstate = 16 (the Mamba shape).
//
// Reference behaviour: selective_scan_fwd_kernel (csrc/selective_scan/selective_scan_fwd_kernel.cuh:
// 301-544) / selective_scan_ref (mamba_ssm/ops/selective_scan_interface.py:353-451). The design is
// this file's own: instead of one 128-thread block per (batch, channel) row with a block-wide scan
// per state, one wave64 owns 16 channels x 16 states and walks the sequence serially:
//
//   lane = 16 * q + c      q = state group (states 4q .. 4q+3, held in registers), c = channel
//
// so every state update is a dependent FMA in one lane's registers (no scan operator, no partial
// products). The operands each row of 16 lanes shares -- B[n, t] and C[n, t] of its four states --
// are loaded once per 32-step tile, one 8-step vector per lane, and broadcast to the row with
// DPP row_newbcast fused into the instruction that consumes them. The per-element terms shared by
// the four rows -- delta' = softplus(delta + bias) and delta' * u -- are computed once per element
// (each lane owns 8 consecutive steps of one channel per tile) and exchanged through LDS; the four
// per-row partial sums of y = sum_n h_n C_n go back through LDS and are added by the lane that owns
// the element, which also applies D * u, the silu(z) gate and the output conversion. Global loads
// for tile i+1 are issued before the scan of tile i.
//
// Per state update the VALU executes: delta' * A (v_mul), exp2 (v_exp_f32), B * delta'u (v_mul with
// DPP), h = a h + b (v_fma), y += C h (v_fmac with DPP).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace tiled {

constexpr int kTile = 32;   // sequence steps per tile
constexpr int kCh = 16;     // channels per wave
constexpr int kPad = 36;    // LDS row stride (floats) of the [channel][step] tiles: 16-B aligned, spreads banks

template <int LANE>
__device__ __forceinline__ float row_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + LANE, 0xf, 0xf, false));
}

// acc += bcast_row(src, LANE) * x  as a single v_fmac_f32_dpp (the compiler does not fuse DPP into
// the tied-operand v_fmac). The DPP source register must not be written by a VALU instruction in
// the two preceding wait states; see the s_nop guard where the sources are produced.
template <int LANE>
__device__ __forceinline__ void fmac_row_bcast(float &acc, float src, float x) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(src), "v"(x), "i"(LANE));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

template <typename T>
__device__ __forceinline__ Vec8<T> load_vec(const T *p) { return *reinterpret_cast<const Vec8<T> *>(p); }

template <typename T>
__device__ __forceinline__ Vec8<T> zero_vec() {
    Vec8<T> v;
    __builtin_memset(&v, 0, sizeof(v));
    return v;
}

template <typename T, bool SOFTPLUS, bool CHUNKS>
__global__ void __launch_bounds__(64)
scan_fwd_tiled16(const mm_scan_fwd_params p, const int64_t ratio) {
    __shared__ __align__(16) float sDt[kCh * kPad];
    __shared__ __align__(16) float sDu[kCh * kPad];
    __shared__ __align__(16) float sY[4 * kCh * kPad];

    const int lane = threadIdx.x;
    const int q = lane >> 4;   // state group of the scan; 8-step slot of the prologue/epilogue
    const int c = lane & 15;   // channel within the wave
    const int64_t b = blockIdx.y;
    const int64_t d0 = int64_t(blockIdx.x) * kCh;
    const int64_t d = d0 + c;
    const int64_t g = d0 / ratio;  // all 16 channels share one group (checked on the host)
    const int64_t L = p.seqlen;

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    T *op = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    T *ozp = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    // The B/C slice this lane loads for its row: state 4q + c/4, steps 8 (c % 4) .. +7 of each tile.
    const int sb = 8 * (c & 3);
    const int64_t nrow = 4 * q + (c >> 2);
    const T *Bp = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride + nrow * p.B_dstate_stride + sb;
    const T *Cp = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride + nrow * p.C_dstate_stride + sb;

    float At[4], h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        At[k] = p.A[d * p.A_d_stride + (4 * q + k) * p.A_dstate_stride] * kLog2e;
        h[k] = 0.f;
    }
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const int es = 8 * q;  // first step (within a tile) of this lane's 8 prologue/epilogue elements
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    float cum_dt = 0.f;

    // Loads past the end of a row are redirected to the row's last 8 elements (always in bounds,
    // L >= 8 and L % 8 == 0); the prologue zeroes delta' and delta' u of those steps, so they leave
    // the state unchanged and their outputs are not stored.
    const int64_t last8 = L - 8;
    auto clampi = [&](int64_t i) { return i < last8 ? i : last8; };
    Vec8<T> ru = load_vec(up + clampi(es));
    Vec8<T> rd = load_vec(dp + clampi(es));
    Vec8<T> rz = zp ? load_vec(zp + clampi(es)) : zero_vec<T>();
    Vec8<T> rb = load_vec(Bp - sb + clampi(sb));
    Vec8<T> rc = load_vec(Cp - sb + clampi(sb));

    for (int64_t t0 = 0; t0 < L; t0 += kTile) {
        const bool ev = t0 + es < L;  // this lane's 8 elements exist (L is a multiple of 8)
        float uu[8], dd[8], zz[8], bv[8], cv[8];
        unpack8(ru, uu);
        unpack8(rd, dd);
        unpack8(rz, zz);
        unpack8(rb, bv);
        unpack8(rc, cv);
        // Prefetch the next tile while this one is processed.
        const int64_t t1 = t0 + kTile;
        if (t1 < L) {
            ru = load_vec(up + clampi(t1 + es));
            rd = load_vec(dp + clampi(t1 + es));
            if (zp) rz = load_vec(zp + clampi(t1 + es));
            rb = load_vec(Bp - sb + clampi(t1 + sb));
            rc = load_vec(Cp - sb + clampi(t1 + sb));
        }
        // Prologue: delta' and delta' u for (channel c, steps es .. es+7); zero past the end so the
        // padded steps leave the state unchanged (a = 1, b = 0).
        float dtp[8], dup[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = dd[i] + bias;
            dtp[i] = SOFTPLUS ? softplus_fast(x) : x;
        }
        if (t1 > L && !ev) {  // padded steps of the last, partial tile
#pragma unroll
            for (int i = 0; i < 8; ++i) dtp[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) dup[i] = dtp[i] * uu[i];
        *reinterpret_cast<float4 *>(&sDt[c * kPad + es]) = make_float4(dtp[0], dtp[1], dtp[2], dtp[3]);
        *reinterpret_cast<float4 *>(&sDt[c * kPad + es + 4]) = make_float4(dtp[4], dtp[5], dtp[6], dtp[7]);
        *reinterpret_cast<float4 *>(&sDu[c * kPad + es]) = make_float4(dup[0], dup[1], dup[2], dup[3]);
        *reinterpret_cast<float4 *>(&sDu[c * kPad + es + 4]) = make_float4(dup[4], dup[5], dup[6], dup[7]);
        // Two wait states between the VALU writes of the DPP sources and their first DPP read.
        asm volatile("s_nop 1"
                     : "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]), "+v"(bv[4]), "+v"(bv[5]), "+v"(bv[6]), "+v"(bv[7]),
                       "+v"(cv[0]), "+v"(cv[1]), "+v"(cv[2]), "+v"(cv[3]), "+v"(cv[4]), "+v"(cv[5]), "+v"(cv[6]), "+v"(cv[7]));
        __syncthreads();

        // Scan: 32 steps, 4 per LDS read.
        static_for<0, kTile / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            const float4 dtq = *reinterpret_cast<const float4 *>(&sDt[c * kPad + 4 * s4]);
            const float4 duq = *reinterpret_cast<const float4 *>(&sDu[c * kPad + 4 * s4]);
            const float dts[4] = {dtq.x, dtq.y, dtq.z, dtq.w};
            const float dus[4] = {duq.x, duq.y, duq.z, duq.w};
            float pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int t = 4 * s4 + j;
                if (CHUNKS) cum_dt += dts[j];
                float acc;
                static_for<0, 4>([&](auto K) {
                    constexpr int k = decltype(K)::value;
                    // B and C of state 4q + k at step t sit in lane 4k + t/8 of this row, register t % 8.
                    constexpr int src = 4 * k + t / 8;
                    const float a = __builtin_amdgcn_exp2f(dts[j] * At[k]);
                    const float bb = row_bcast<src>(bv[t % 8]) * dus[j];
                    h[k] = __builtin_fmaf(a, h[k], bb);
                    if constexpr (k == 0)
                        acc = row_bcast<src>(cv[t % 8]) * h[k];
                    else
                        fmac_row_bcast<src>(acc, cv[t % 8], h[k]);
                });
                pv[j] = acc;
            });
            *reinterpret_cast<float4 *>(&sY[(q * kCh + c) * kPad + 4 * s4]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        });
        __syncthreads();

        // Epilogue: y for (channel c, steps es .. es+7) = sum of the four row partials.
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
            float4 acc = *reinterpret_cast<const float4 *>(&sY[(0 * kCh + c) * kPad + es + i]);
#pragma unroll
            for (int r = 1; r < 4; ++r) {
                const float4 v = *reinterpret_cast<const float4 *>(&sY[(r * kCh + c) * kPad + es + i]);
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
            y[i] = acc.x; y[i + 1] = acc.y; y[i + 2] = acc.z; y[i + 3] = acc.w;
        }
        if (ev) {
            float o[8], oz[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                o[i] = p.D ? __builtin_fmaf(Dv, uu[i], y[i]) : y[i];
                oz[i] = zp ? o[i] * silu_fast(zz[i]) : o[i];
            }
            if (op) store8(op + t0 + es, o);
            if (ozp) store8(ozp + t0 + es, oz);
        }
        if (CHUNKS && p.chunk_states) {
            const int64_t tend = t1 < L ? t1 : L;
            if (tend % MM_SCAN_CHUNK == 0 || tend == L) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *cs = p.chunk_states + ((b * p.dim + d) * n_chunks + ci) * 32 + 8 * q;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    cs[2 * k] = __builtin_amdgcn_exp2f(At[k] * cum_dt);
                    cs[2 * k + 1] = h[k];
                }
            }
        }
    }
    if (p.last_state) {
        *reinterpret_cast<float4 *>(p.last_state + (b * p.dim + d) * 16 + 4 * q) = make_float4(h[0], h[1], h[2], h[3]);
    }
}

}  // namespace tiled

template <typename T>
int try_launch_tiled(const mm_scan_fwd_params &p, hipStream_t stream) {
    if (p.dstate != 16 || !p.is_variable_B || !p.is_variable_C) return MM_ERR_UNSUPPORTED;
    if (p.dim % tiled::kCh != 0 || (p.dim / p.n_groups) % tiled::kCh != 0) return MM_ERR_UNSUPPORTED;
    if (p.seqlen < 1 || !fwd_vector_ok(&p)) return MM_ERR_UNSUPPORTED;
    if (p.batch > 65535) return MM_ERR_UNSUPPORTED;
    if (p.last_state && (reinterpret_cast<uintptr_t>(p.last_state) & 15u)) return MM_ERR_UNSUPPORTED;
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / tiled::kCh), unsigned(p.batch));
    auto *kern = p.delta_softplus ? (p.chunk_states ? tiled::scan_fwd_tiled16<T, true, true> : tiled::scan_fwd_tiled16<T, true, false>)
                                  : (p.chunk_states ? tiled::scan_fwd_tiled16<T, false, true> : tiled::scan_fwd_tiled16<T, false, false>);
    hipLaunchKernelGGL(kern, grid, dim3(64), 0, stream, p, ratio);
    return launch_status("scan_fwd_tiled16");
}

template int try_launch_tiled<float>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<f16_t>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<bf16_t>(const mm_scan_fwd_params &, hipStream_t);

}  // namespace mm
