// mm_scan_tiled.hip -- the gfx950 forward selective scan for dstate = 16 (the Mamba shape).
//
// Reference behaviour: selective_scan_fwd_kernel (csrc/selective_scan/selective_scan_fwd_kernel.cuh:
// 301-544) / selective_scan_ref (mamba_ssm/ops/selective_scan_interface.py:353-451). The design is
// this file's own. Instead of one thread block per (batch, channel) row running a block-wide scan
// per state, a workgroup of NW wave64s owns 16 channels x 16 states of one batch row and walks the
// sequence serially, every state update being one dependent FMA in a lane's registers:
//
//   wave w, lane = 16 q + c:  channel c of the group, states (4 w + q) K .. +K-1,  K = 4 / NW
//
// so each row of 16 lanes shares its K states, and each column shares a channel.
//  * B[n, t] and C[n, t] of the row's K states are loaded once per 32-step tile, one small vector
//    per lane, and broadcast along the row by DPP row_newbcast fused into the instruction that
//    consumes them (v_mul_f32_dpp for B * delta'u, v_fmac_f32_dpp for y += C h).
//  * delta' = softplus(delta + bias) and delta' u are computed once per (channel, step) -- each lane
//    owns 8/NW consecutive steps of one channel per tile -- and exchanged through LDS.
//  * The 4 NW per-row partial sums of y = sum_n C_n h_n go back through LDS; the lane that owns the
//    element adds them in a fixed order, applies D u and the silu(z) gate and stores the output.
//  * Global loads for tile i+1 are issued before the scan of tile i.
// NW trades per-update overhead (smaller K shares the per-step work among fewer updates) for more
// concurrent waves per SIMD, which gfx950 needs to reach its VALU/transcendental issue rate.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace tiled {

constexpr int kTile = 32;   // sequence steps per tile
constexpr int kCh = 16;     // channels per workgroup
constexpr int kPad = 36;    // LDS row stride (floats) of the [channel][step] tiles: 16-B aligned, spreads banks

template <int LANE>
__device__ __forceinline__ float row_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + LANE, 0xf, 0xf, false));
}

// acc += bcast_row(src, LANE) * x as one v_fmac_f32_dpp (the compiler does not fuse DPP into the
// tied-operand v_fmac). The DPP source register must not be written by a VALU instruction in the
// two preceding wait states; the s_nop guard where the sources are produced provides that.
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

// N consecutive elements moved as one vector (N * sizeof(T) bytes: 4, 8, 16 or 32).
template <typename T, int N> struct RawVec { uint32_t w[(N * sizeof(T) + 3) / 4]; };

template <typename T, int N>
__device__ __forceinline__ RawVec<T, N> load_raw(const T *p) {
    RawVec<T, N> r;
    constexpr int W = sizeof(r.w) / 4;
    if constexpr (W == 8) {
        const uint4 *q = reinterpret_cast<const uint4 *>(p);
        const uint4 a = q[0], b = q[1];
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w; r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    } else if constexpr (W == 4) {
        const uint4 a = *reinterpret_cast<const uint4 *>(p);
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    } else if constexpr (W == 2) {
        const uint2 a = *reinterpret_cast<const uint2 *>(p);
        r.w[0] = a.x; r.w[1] = a.y;
    } else {
        r.w[0] = *reinterpret_cast<const uint32_t *>(p);
    }
    return r;
}

template <typename T, int N>
__device__ __forceinline__ void unpack_raw(const RawVec<T, N> &r, float *o) {
    if constexpr (std::is_same_v<T, float>) {
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = __uint_as_float(r.w[i]);
    } else if constexpr (std::is_same_v<T, bf16_t>) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) unpack_bf16x2(r.w[i], o[2 * i], o[2 * i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) unpack_f16x2(r.w[i], o[2 * i], o[2 * i + 1]);
    }
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T *p, const float *x) {
    if constexpr (std::is_same_v<T, float>) {
        if constexpr (N == 8) {
            uint4 *q = reinterpret_cast<uint4 *>(p);
            q[0] = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
            q[1] = make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7]));
        } else if constexpr (N == 4) {
            *reinterpret_cast<uint4 *>(p) = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
        } else {
            *reinterpret_cast<uint2 *>(p) = make_uint2(__float_as_uint(x[0]), __float_as_uint(x[1]));
        }
    } else {
        uint32_t w[N / 2];
#pragma unroll
        for (int i = 0; i < N / 2; ++i)
            w[i] = std::is_same_v<T, bf16_t> ? pack_bf16x2(x[2 * i], x[2 * i + 1]) : pack_f16x2(x[2 * i], x[2 * i + 1]);
        if constexpr (N == 8) *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        else if constexpr (N == 4) *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
        else *reinterpret_cast<uint32_t *>(p) = w[0];
    }
}

template <typename T, int NW, bool SOFTPLUS, bool CHUNKS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 4)))
scan_fwd_tiled16(const mm_scan_fwd_params p, const int64_t ratio) {
    constexpr int K = 4 / NW;            // states per lane
    constexpr int E = 8 / NW;            // prologue/epilogue steps per lane per tile
    constexpr int LPS = 16 / K;          // lanes of a row holding one state's B/C
    constexpr int SPL = kTile / LPS;     // B/C steps per lane per tile (= 2K)
    constexpr int NR = 4 * NW;           // rows (state groups) in the workgroup
    __shared__ __align__(16) float sDt[kCh * kPad];
    __shared__ __align__(16) float sDu[kCh * kPad];
    __shared__ __align__(16) float sY[NR * kCh * kPad];

    const int w = threadIdx.x >> 6;        // wave
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4;               // row within the wave
    const int r = 4 * w + q;               // row within the workgroup: state group, and prologue slot
    const int c = lane & 15;               // channel within the group
    const int64_t b = blockIdx.y;
    const int64_t d0 = int64_t(blockIdx.x) * kCh;
    const int64_t d = d0 + c;
    const int64_t g = d0 / ratio;          // all 16 channels share one group (checked on the host)
    const int64_t L = p.seqlen;

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    T *op = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    T *ozp = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    // The B/C slice this lane loads for its row: state r K + c / LPS, steps SPL (c % LPS) .. +SPL-1.
    const int sb = SPL * (c % LPS);
    const int64_t nrow = int64_t(r) * K + c / LPS;
    const T *Bp = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride + nrow * p.B_dstate_stride;
    const T *Cp = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride + nrow * p.C_dstate_stride;

    float At[K], h[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        At[k] = p.A[d * p.A_d_stride + (r * K + k) * p.A_dstate_stride] * kLog2e;
        h[k] = 0.f;
    }
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const int es = E * r;                  // first step (within a tile) of this lane's elements
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    float cum_dt = 0.f;

    // Loads at or past the end of a row are redirected into the row's last elements (always in
    // bounds: L >= 8, L % 8 == 0). The prologue zeroes delta' and delta' u of padded steps, so
    // they leave the state unchanged; their outputs are not stored.
    const int64_t lastE = L - E, lastS = L - SPL;
    auto ce = [&](int64_t i) { return i < lastE ? i : lastE; };
    auto cs = [&](int64_t i) { return i < lastS ? i : lastS; };
    RawVec<T, E> ru = load_raw<T, E>(up + ce(es));
    RawVec<T, E> rd = load_raw<T, E>(dp + ce(es));
    RawVec<T, E> rz = {};
    if (zp) rz = load_raw<T, E>(zp + ce(es));
    RawVec<T, SPL> rb = load_raw<T, SPL>(Bp + cs(sb));
    RawVec<T, SPL> rc = load_raw<T, SPL>(Cp + cs(sb));

    for (int64_t t0 = 0; t0 < L; t0 += kTile) {
        const bool ev = t0 + es < L;  // this lane's E elements exist (L is a multiple of 8)
        float uu[E], dd[E], zz[E], bv[SPL], cv[SPL];
        unpack_raw<T, E>(ru, uu);
        unpack_raw<T, E>(rd, dd);
        unpack_raw<T, E>(rz, zz);
        unpack_raw<T, SPL>(rb, bv);
        unpack_raw<T, SPL>(rc, cv);
        // Prefetch the next tile (clamped addresses: always issued, never out of bounds).
        const int64_t t1 = t0 + kTile;
        ru = load_raw<T, E>(up + ce(t1 + es));
        rd = load_raw<T, E>(dp + ce(t1 + es));
        if (zp) rz = load_raw<T, E>(zp + ce(t1 + es));
        rb = load_raw<T, SPL>(Bp + cs(t1 + sb));
        rc = load_raw<T, SPL>(Cp + cs(t1 + sb));

        // Prologue: delta' and delta' u for (channel c, steps es .. es+E-1).
        float dtp[E], dup[E];
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float x = dd[i] + bias;
            dtp[i] = SOFTPLUS ? softplus_fast(x) : x;
        }
        if (t1 > L && !ev) {  // padded steps of a last, partial tile
#pragma unroll
            for (int i = 0; i < E; ++i) dtp[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < E; ++i) dup[i] = dtp[i] * uu[i];
#pragma unroll
        for (int i = 0; i < E; i += 2) {
            *reinterpret_cast<float2 *>(&sDt[c * kPad + es + i]) = make_float2(dtp[i], dtp[i + 1]);
            *reinterpret_cast<float2 *>(&sDu[c * kPad + es + i]) = make_float2(dup[i], dup[i + 1]);
        }
        // Two wait states between the VALU writes of the DPP sources and their first DPP read.
#pragma unroll
        for (int i = 0; i < SPL; ++i) asm volatile("s_nop 1" : "+v"(bv[i]), "+v"(cv[i]));
        __syncthreads();

        // Scan: 32 steps, 4 per LDS read; y partial (sum over this lane's K states) per step.
        static_for<0, kTile / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            const float4 dtq = *reinterpret_cast<const float4 *>(&sDt[c * kPad + 4 * s4]);
            const float4 duq = *reinterpret_cast<const float4 *>(&sDu[c * kPad + 4 * s4]);
            const float dts[4] = {dtq.x, dtq.y, dtq.z, dtq.w};
            const float dus[4] = {duq.x, duq.y, duq.z, duq.w};
            // The decay factors and input terms of the 4 steps do not depend on the state: compute
            // them all first (16 independent exp2 per lane for K = 4), then run the recurrences.
            // B and C of state r K + k at step t sit in lane k LPS + t / SPL of this row, register
            // t % SPL.
            float av[4][K], bbv[4][K];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int t = 4 * s4 + j;
                if (CHUNKS) cum_dt += dts[j];
                static_for<0, K>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    constexpr int src = k * LPS + t / SPL;
                    av[j][k] = __builtin_amdgcn_exp2f(dts[j] * At[k]);
                    bbv[j][k] = row_bcast<src>(bv[t % SPL]) * dus[j];
                });
            });
            float pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int t = 4 * s4 + j;
                float acc;
                static_for<0, K>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    constexpr int src = k * LPS + t / SPL;
                    h[k] = __builtin_fmaf(av[j][k], h[k], bbv[j][k]);
                    if constexpr (k == 0)
                        acc = row_bcast<src>(cv[t % SPL]) * h[k];
                    else
                        fmac_row_bcast<src>(acc, cv[t % SPL], h[k]);
                });
                pv[j] = acc;
            });
            *reinterpret_cast<float4 *>(&sY[(r * kCh + c) * kPad + 4 * s4]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        });
        __syncthreads();

        // Epilogue: y for (channel c, steps es .. es+E-1) = the NR row partials, added in row order.
        float y[E];
#pragma unroll
        for (int i = 0; i < E; i += 2) {
            float2 acc = *reinterpret_cast<const float2 *>(&sY[(0 * kCh + c) * kPad + es + i]);
#pragma unroll
            for (int rr = 1; rr < NR; ++rr) {
                const float2 v = *reinterpret_cast<const float2 *>(&sY[(rr * kCh + c) * kPad + es + i]);
                acc.x += v.x;
                acc.y += v.y;
            }
            y[i] = acc.x;
            y[i + 1] = acc.y;
        }
        if (ev) {
            float o[E];
#pragma unroll
            for (int i = 0; i < E; ++i) o[i] = __builtin_fmaf(Dv, uu[i], y[i]);
            if (op) store_vec<T, E>(op + t0 + es, o);
            if (zp) {
#pragma unroll
                for (int i = 0; i < E; ++i) o[i] *= silu_fast(zz[i]);
                store_vec<T, E>(ozp + t0 + es, o);
            }
        }
        if (CHUNKS && p.chunk_states) {
            const int64_t tend = t1 < L ? t1 : L;
            if (tend % MM_SCAN_CHUNK == 0 || tend == L) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *csp = p.chunk_states + ((b * p.dim + d) * n_chunks + ci) * 32 + 2 * K * r;
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    csp[2 * k] = __builtin_amdgcn_exp2f(At[k] * cum_dt);
                    csp[2 * k + 1] = h[k];
                }
            }
        }
    }
    if (p.last_state) {
        float *ls = p.last_state + (b * p.dim + d) * 16 + K * r;
#pragma unroll
        for (int k = 0; k < K; ++k) ls[k] = h[k];
    }
}

template <typename T, int NW>
int launch_nw(const mm_scan_fwd_params &p, hipStream_t stream) {
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / kCh), unsigned(p.batch));
    auto *kern = p.delta_softplus
                     ? (p.chunk_states ? scan_fwd_tiled16<T, NW, true, true> : scan_fwd_tiled16<T, NW, true, false>)
                     : (p.chunk_states ? scan_fwd_tiled16<T, NW, false, true> : scan_fwd_tiled16<T, NW, false, false>);
    hipLaunchKernelGGL(kern, grid, dim3(64 * NW), 0, stream, p, ratio);
    return launch_status("scan_fwd_tiled16");
}

}  // namespace tiled

// Waves per 16-channel workgroup; MM_SCAN_NW in the environment overrides the default (1, 2, 4).
static int tiled_waves() {
    static int nw = [] {
        const char *e = getenv("MM_SCAN_NW");
        const int v = e ? atoi(e) : 2;
        return (v == 1 || v == 2 || v == 4) ? v : 2;
    }();
    return nw;
}

template <typename T>
int try_launch_tiled(const mm_scan_fwd_params &p, hipStream_t stream) {
    if (p.dstate != 16 || !p.is_variable_B || !p.is_variable_C) return MM_ERR_UNSUPPORTED;
    if (p.dim % tiled::kCh != 0 || (p.dim / p.n_groups) % tiled::kCh != 0) return MM_ERR_UNSUPPORTED;
    if (p.seqlen < 8 || !fwd_vector_ok(&p)) return MM_ERR_UNSUPPORTED;
    if (p.batch > 65535) return MM_ERR_UNSUPPORTED;
    switch (tiled_waves()) {
        case 1: return tiled::launch_nw<T, 1>(p, stream);
        case 4: return tiled::launch_nw<T, 4>(p, stream);
        default: return tiled::launch_nw<T, 2>(p, stream);
    }
}

template int try_launch_tiled<float>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<f16_t>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<bf16_t>(const mm_scan_fwd_params &, hipStream_t);

}  // namespace mm
