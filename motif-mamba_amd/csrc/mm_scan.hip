// mm_scan.hip -- gfx950 (CDNA4) selective-scan kernels and the C ABI of libmm_scan.so.
//
// Entry points (declared in include/mm_scan.h):
//   mm_scan_fwd      -- replaces selective_scan_cuda.fwd (reference csrc/selective_scan/
//                       selective_scan.cpp:270-413) for real A; requests with P/Q go to
//                       mm_scan_pq.hip.
//   mm_scan_bwd      -- replaces selective_scan_cuda.bwd (selective_scan.cpp:415-612); kernels in
//                       mm_scan_bwd.hip.
//   mm_state_update  -- replaces the upstream selective_state_update called at
//                       mamba_ssm/modules/mamba_simplemotif.py:397-399.
//
// Kernels in this file:
//   scan_fwd_rowlane<T, NS, VEC>  one lane owns one (batch, channel) row and all of its NS states
//                                 in registers and walks the sequence serially, 8 steps per
//                                 iteration. Used for every shape the tiled kernel does not take.
//   state_update<T, SPL>          one decode step; LPR lanes share a row, SPL states per lane.
//   state_update_vec16<T, U>      one decode step for dstate 16 with aligned unit-stride rows: four
//                                 lanes per row, four states each as one 16-byte vector, U batch rows
//                                 per workgroup sharing A, D and dt_bias.
// The tiled forward kernel lives in mm_scan_tiled.hip.
#include <hip/hip_runtime.h>

#include <atomic>

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "mm_common.h"
#include "mm_internal.h"
#include "mm_scan.h"

namespace mm {

// ================================================================================================
// Forward scan, lane-per-row kernel.
// ================================================================================================
constexpr int kRowBlock = 64;

template <typename T, int NS, bool VEC>
__global__ void __launch_bounds__(kRowBlock)
scan_fwd_rowlane(const mm_scan_fwd_params p, const int64_t ratio, const int32_t uniform_g) {
    const int64_t d_raw = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t b = blockIdx.y;
    const bool active = d_raw < p.dim;
    const int64_t d = active ? d_raw : p.dim - 1;  // clamped for loads; stores are predicated
    int64_t g = d / ratio;
    if (uniform_g) g = __builtin_amdgcn_readfirstlane(int(g));
    const int64_t L = p.seqlen;
    const int N = int(p.dstate);

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    T *op = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    T *ozp = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    const T *Bv = p.is_variable_B ? reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride : nullptr;
    const T *Cv = p.is_variable_C ? reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride : nullptr;

    float At[NS], h[NS], Bc[NS], Cc[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        const bool on = n < N;
        At[n] = on ? p.A[d * p.A_d_stride + n * p.A_dstate_stride] * kLog2e : 0.f;
        h[n] = 0.f;
        Bc[n] = (on && !p.is_variable_B) ? reinterpret_cast<const float *>(p.B)[d * p.B_d_stride + n * p.B_dstate_stride] : 0.f;
        Cc[n] = (on && !p.is_variable_C) ? reinterpret_cast<const float *>(p.C)[d * p.C_d_stride + n * p.C_dstate_stride] : 0.f;
    }
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    float cum_dt = 0.f;  // running sum of delta' (chunk-state prod a = exp2(A log2e * cum_dt))

    for (int64_t l0 = 0; l0 < L; l0 += 8) {
        const int nt = int(L - l0 < 8 ? L - l0 : 8);
        float uu[8], dd[8], zz[8];
        if (VEC && nt == 8) {
            load8(up + l0, uu);
            load8(dp + l0, dd);
            if (zp) load8(zp + l0, zz);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uu[t] = t < nt ? to_f32(up[l0 + t]) : 0.f;
                dd[t] = t < nt ? to_f32(dp[l0 + t]) : 0.f;
                zz[t] = (zp && t < nt) ? to_f32(zp[l0 + t]) : 0.f;
            }
        }
        float dtp[8], du[8], y[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float x = dd[t] + bias;
            dtp[t] = p.delta_softplus ? softplus_f32(x) : x;
            du[t] = dtp[t] * uu[t];
            y[t] = 0.f;
            if (t < nt) cum_dt += dtp[t];
        }
#pragma unroll(NS <= 64 ? NS : 8)
        for (int n = 0; n < NS; ++n) {
            if (n >= N) break;  // states past dstate: no B/C rows exist there
            float bb[8], cc[8];
            if (Bv) {
                if (VEC && nt == 8) {
                    load8(Bv + n * p.B_dstate_stride + l0, bb);
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) bb[t] = t < nt ? to_f32(Bv[n * p.B_dstate_stride + l0 + t]) : 0.f;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) bb[t] = Bc[n];
            }
            if (Cv) {
                if (VEC && nt == 8) {
                    load8(Cv + n * p.C_dstate_stride + l0, cc);
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = t < nt ? to_f32(Cv[n * p.C_dstate_stride + l0 + t]) : 0.f;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) cc[t] = Cc[n];
            }
            float hn = h[n];
            const float an = At[n];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (VEC || t < nt) {
                    const float a = decay_exp2(dtp[t], an);
                    hn = __builtin_fmaf(a, hn, du[t] * bb[t]);
                    y[t] = __builtin_fmaf(hn, cc[t], y[t]);
                }
            }
            h[n] = hn;
        }
        float o[8], oz[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            o[t] = p.D ? __builtin_fmaf(Dv, uu[t], y[t]) : y[t];
            oz[t] = zp ? o[t] * silu_f32(zz[t]) : o[t];
        }
        if (active) {
            if (VEC && nt == 8) {
                if (op) store8(op + l0, o);
                if (ozp) store8(ozp + l0, oz);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (t < nt) {
                        if (op) op[l0 + t] = from_f32<T>(o[t]);
                        if (ozp) ozp[l0 + t] = from_f32<T>(oz[t]);
                    }
                }
            }
            const int64_t lend = l0 + nt;
            if (p.chunk_states && (lend % MM_SCAN_CHUNK == 0 || lend == L)) {
                const int64_t c = (lend - 1) / MM_SCAN_CHUNK;
                float *cs = p.chunk_states + ((b * p.dim + d) * n_chunks + c) * 2 * N;
#pragma unroll
                for (int n = 0; n < NS; ++n) {
                    if (n < N) {
                        cs[2 * n] = fast_exp2(At[n] * cum_dt);
                        cs[2 * n + 1] = h[n];
                    }
                }
            }
        }
    }
    if (active && p.last_state) {
        float *ls = p.last_state + (b * p.dim + d) * N;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) ls[n] = h[n];
    }
}

// ================================================================================================
// Decode step: LPR lanes per (batch, channel) row, SPL states per lane.
// ================================================================================================
constexpr int kDecBlock = 256;

// A per-channel decode parameter (D, dt_bias) of any float element type, widened to float32.
__device__ __forceinline__ float load_param(const void *base, mm_dtype t, int64_t i) {
    if (t == MM_FLOAT16) return to_f32(reinterpret_cast<const f16_t *>(base)[i]);
    if (t == MM_BFLOAT16) return to_f32(reinterpret_cast<const bf16_t *>(base)[i]);
    return reinterpret_cast<const float *>(base)[i];
}

template <typename T, typename S, int SPL, int LPR>
__global__ void __launch_bounds__(kDecBlock)
state_update_kernel(const mm_state_update_params p, const int64_t ratio) {
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t row = tid / LPR;
    const int part = int(tid % LPR);
    const int64_t nrows = p.batch * p.dim;
    const bool active = row < nrows;
    const int64_t rr = active ? row : nrows - 1;
    const int64_t b = rr / p.dim;
    const int64_t d = rr % p.dim;
    const int64_t g = d / ratio;
    const int N = int(p.dstate);

    float dt = to_f32(reinterpret_cast<const T *>(p.dt)[b * p.dt_batch_stride + d * p.dt_d_stride]);
    if (p.dt_bias) dt += load_param(p.dt_bias, p.dt_bias_type, d);
    if (p.dt_softplus) dt = softplus_f32(dt);
    const float x = to_f32(reinterpret_cast<const T *>(p.x)[b * p.x_batch_stride + d * p.x_d_stride]);
    const float dtx = dt * x;
    const T *Bp = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cp = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;
    S *sp = reinterpret_cast<S *>(p.state) + b * p.state_batch_stride + d * p.state_d_stride;

    float y = 0.f;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
        const int n = part * SPL + k;
        if (n < N) {
            const float a = decay_exp2(dt, p.A[d * p.A_d_stride + n * p.A_dstate_stride] * kLog2e);
            float s = to_f32(sp[n * p.state_dstate_stride]);
            s = __builtin_fmaf(s, a, dtx * to_f32(Bp[n * p.B_dstate_stride]));
            if (active) sp[n * p.state_dstate_stride] = from_f32<S>(s);
            y = __builtin_fmaf(s, to_f32(Cp[n * p.C_dstate_stride]), y);   // the float32 state
        }
    }
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) y += __shfl_xor(y, off, LPR);
    if (active && part == 0) {
        if (p.D) y = __builtin_fmaf(load_param(p.D, p.D_type, d), x, y);
        if (p.z) y *= silu_f32(to_f32(reinterpret_cast<const T *>(p.z)[b * p.z_batch_stride + d * p.z_d_stride]));
        reinterpret_cast<T *>(p.out)[b * p.out_batch_stride + d * p.out_d_stride] = from_f32<T>(y);
    }
}

// Four consecutive elements of T as fp32 (8-byte load for 16-bit types, 16-byte for fp32).
template <typename T>
__device__ __forceinline__ float4 load4(const T *p) {
    if constexpr (std::is_same_v<T, float>) {
        return *reinterpret_cast<const float4 *>(p);
    } else {
        const uint2 w = *reinterpret_cast<const uint2 *>(p);
        float4 r;
        if constexpr (std::is_same_v<T, bf16_t>) {
            unpack_bf16x2(w.x, r.x, r.y);
            unpack_bf16x2(w.y, r.z, r.w);
        } else {
            unpack_f16x2(w.x, r.x, r.y);
            unpack_f16x2(w.y, r.z, r.w);
        }
        return r;
    }
}

// Loads of one (batch, channel) row's quarter for the dstate-16 decode step, issued before any
// arithmetic so that a lane has U rows' worth of memory requests in flight.
template <typename T>
struct DecRow {
    float4 s;           // four states (float32 state)
    uint2 sw;           // four states as raw words (16-bit state)
    uint2 bw, cw;       // four B / C values as raw words (16-bit types; fp32 uses bf/cf)
    float4 bf, cf;
    T dt, x, z;
};

// Four consecutive 16-bit values (two packed words) as float32, and back with round to nearest even.
template <typename S>
__device__ __forceinline__ float4 unpack4(uint2 w) {
    float4 r;
    if constexpr (std::is_same_v<S, bf16_t>) {
        unpack_bf16x2(w.x, r.x, r.y);
        unpack_bf16x2(w.y, r.z, r.w);
    } else {
        unpack_f16x2(w.x, r.x, r.y);
        unpack_f16x2(w.y, r.z, r.w);
    }
    return r;
}
template <typename S>
__device__ __forceinline__ uint2 pack4(float4 v) {
    if constexpr (std::is_same_v<S, bf16_t>) return make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    else return make_uint2(pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w));
}

// dstate 16 with every row of state, A, B and C contiguous and 4-element aligned (checked on the
// host). Four lanes per (batch, channel) row, each moving four consecutive states as one 16-byte
// vector; a 256-lane workgroup covers 64 channels of U consecutive batch rows. A, D and dt_bias of
// the lane's channel are loaded once and reused for the U rows, and every load of the U rows is
// issued before the first state is updated (one 16-byte state load in flight per lane leaves too
// few bytes in flight to cover HBM latency). The grid is one-dimensional, blockIdx.x = batch block
// * n_dblk + channel block, so no 64-bit division runs per lane; channels past `dim` and rows past
// `batch` reload the last one and store nothing.
template <typename T, typename S, int U>
__global__ void __launch_bounds__(kDecBlock)
state_update_vec16(const mm_state_update_params p, const uint32_t ratio, const uint32_t n_dblk) {
    const uint32_t bb = blockIdx.x / n_dblk;
    const uint32_t jd = blockIdx.x - bb * n_dblk;
    const int part = int(threadIdx.x & 3);
    const uint32_t dim = uint32_t(p.dim);
    const uint32_t dr = jd * 64u + (threadIdx.x >> 2);
    const uint32_t d = dr < dim ? dr : dim - 1;
    const uint32_t g = d / ratio;
    const float4 a4 = *reinterpret_cast<const float4 *>(p.A + int64_t(d) * p.A_d_stride + 4 * part);
    const float Dv = p.D ? load_param(p.D, p.D_type, d) : 0.f;
    const float bias = p.dt_bias ? load_param(p.dt_bias, p.dt_bias_type, d) : 0.f;
    S *const state = reinterpret_cast<S *>(p.state);
    DecRow<T> r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t b0 = bb * U + u;
        const uint32_t b = b0 < uint32_t(p.batch) ? b0 : uint32_t(p.batch) - 1;
        const S *sp = state + int64_t(b) * p.state_batch_stride + int64_t(d) * p.state_d_stride + 4 * part;
        if constexpr (std::is_same_v<S, float>) r[u].s = *reinterpret_cast<const float4 *>(sp);
        else r[u].sw = *reinterpret_cast<const uint2 *>(sp);
        const T *Bb = reinterpret_cast<const T *>(p.B) + int64_t(b) * p.B_batch_stride + int64_t(g) * p.B_group_stride + 4 * part;
        const T *Cb = reinterpret_cast<const T *>(p.C) + int64_t(b) * p.C_batch_stride + int64_t(g) * p.C_group_stride + 4 * part;
        if constexpr (std::is_same_v<T, float>) {
            r[u].bf = *reinterpret_cast<const float4 *>(Bb);
            r[u].cf = *reinterpret_cast<const float4 *>(Cb);
        } else {
            r[u].bw = *reinterpret_cast<const uint2 *>(Bb);
            r[u].cw = *reinterpret_cast<const uint2 *>(Cb);
        }
        r[u].dt = reinterpret_cast<const T *>(p.dt)[int64_t(b) * p.dt_batch_stride + int64_t(d) * p.dt_d_stride];
        r[u].x = reinterpret_cast<const T *>(p.x)[int64_t(b) * p.x_batch_stride + int64_t(d) * p.x_d_stride];
        if (p.z) r[u].z = reinterpret_cast<const T *>(p.z)[int64_t(b) * p.z_batch_stride + int64_t(d) * p.z_d_stride];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t b = bb * U + u;
        float4 b4, c4;
        if constexpr (std::is_same_v<T, float>) {
            b4 = r[u].bf;
            c4 = r[u].cf;
        } else if constexpr (std::is_same_v<T, bf16_t>) {
            unpack_bf16x2(r[u].bw.x, b4.x, b4.y);
            unpack_bf16x2(r[u].bw.y, b4.z, b4.w);
            unpack_bf16x2(r[u].cw.x, c4.x, c4.y);
            unpack_bf16x2(r[u].cw.y, c4.z, c4.w);
        } else {
            unpack_f16x2(r[u].bw.x, b4.x, b4.y);
            unpack_f16x2(r[u].bw.y, b4.z, b4.w);
            unpack_f16x2(r[u].cw.x, c4.x, c4.y);
            unpack_f16x2(r[u].cw.y, c4.z, c4.w);
        }
        float dt = to_f32(r[u].dt) + bias;
        if (p.dt_softplus) dt = softplus_fast(dt);
        const float x = to_f32(r[u].x);
        const float dtx = dt * x;
        const float dl = dt * kLog2e;
        float4 s;
        if constexpr (std::is_same_v<S, float>) s = r[u].s;
        else s = unpack4<S>(r[u].sw);
        s.x = __builtin_fmaf(s.x, decay_exp2(dl, a4.x), dtx * b4.x);
        s.y = __builtin_fmaf(s.y, decay_exp2(dl, a4.y), dtx * b4.y);
        s.z = __builtin_fmaf(s.z, decay_exp2(dl, a4.z), dtx * b4.z);
        s.w = __builtin_fmaf(s.w, decay_exp2(dl, a4.w), dtx * b4.w);
        const bool live = dr < dim && b < uint32_t(p.batch);
        if (live) {
            S *sp = state + int64_t(b) * p.state_batch_stride + int64_t(dr) * p.state_d_stride + 4 * part;
            if constexpr (std::is_same_v<S, float>) *reinterpret_cast<float4 *>(sp) = s;
            else *reinterpret_cast<uint2 *>(sp) = pack4<S>(s);
        }
        // y from the float32 state, before a 16-bit state is rounded.
        float y = __builtin_fmaf(s.x, c4.x, __builtin_fmaf(s.y, c4.y, __builtin_fmaf(s.z, c4.z, s.w * c4.w)));
        y += __shfl_xor(y, 1, 4);
        y += __shfl_xor(y, 2, 4);
        if (live && part == 0) {
            y = __builtin_fmaf(Dv, x, y);
            if (p.z) y *= silu_fast(to_f32(r[u].z));
            reinterpret_cast<T *>(p.out)[int64_t(b) * p.out_batch_stride + int64_t(dr) * p.out_d_stride] = from_f32<T>(y);
        }
    }
}

// The raw bits of a 16- or 32-bit value of lane (quad base + Q) of every quad (v_mov_b32_dpp
// quad_perm [Q,Q,Q,Q]).
template <int Q>
__device__ __forceinline__ int quad_bcast(int v) {
    return __builtin_amdgcn_update_dpp(0, v, Q * 0x55, 0xf, 0xf, false);
}
template <typename T>
__device__ __forceinline__ int raw_bits(T v) {
    if constexpr (std::is_same_v<T, float>) return __float_as_int(v);
    else return int(__builtin_bit_cast(uint16_t, v));
}
template <typename T>
__device__ __forceinline__ T from_bits(int v) {
    if constexpr (std::is_same_v<T, float>) return __int_as_float(v);
    else return __builtin_bit_cast(T, uint16_t(v));
}

// state_update_vec16 for four batch rows per workgroup whose 64 channels lie in one group, with
// the per-row loads shared: the four lanes of a channel row load x, dt and z of four different batch
// rows (lane part p: row bb * 4 + p) and pass them round the quad with DPP, one load per lane per
// tensor instead of one per lane per row; B and C of the four rows (2 x 4 x 16 values) come in
// with one element per lane into LDS; each lane stores the output of batch row p. Per lane that is
// about half the memory instructions of state_update_vec16<T, S, 4>, whose operations and order it
// keeps (the results are bit-identical).
template <typename T, typename S>
__global__ void __launch_bounds__(kDecBlock)
state_update_vec16x(const mm_state_update_params p, const uint32_t ratio, const uint32_t n_dblk) {
    constexpr int U = 4;
    __shared__ __align__(16) float sBC[U * 2 * 16];   // [row u][B | C][state]
    const uint32_t bb = blockIdx.x / n_dblk;
    const uint32_t jd = blockIdx.x - bb * n_dblk;
    const int tid = int(threadIdx.x);
    const int part = tid & 3;
    const uint32_t dim = uint32_t(p.dim), batch = uint32_t(p.batch);
    const uint32_t dr = jd * 64u + uint32_t(tid >> 2);
    const uint32_t d = dr < dim ? dr : dim - 1;
    const uint32_t g = (jd * 64u < dim ? jd * 64u : dim - 1) / ratio;   // one group per workgroup
    if (tid < U * 2 * 16) {
        const uint32_t u = uint32_t(tid) >> 5, n = uint32_t(tid) & 15;
        const uint32_t b = bb * U + u < batch ? bb * U + u : batch - 1;
        const T *src = (tid & 16) ? reinterpret_cast<const T *>(p.C) + int64_t(b) * p.C_batch_stride + int64_t(g) * p.C_group_stride
                                  : reinterpret_cast<const T *>(p.B) + int64_t(b) * p.B_batch_stride + int64_t(g) * p.B_group_stride;
        sBC[tid] = to_f32(src[n]);
    }
    const float4 a4 = *reinterpret_cast<const float4 *>(p.A + int64_t(d) * p.A_d_stride + 4 * part);
    const float Dv = p.D ? load_param(p.D, p.D_type, d) : 0.f;
    const float bias = p.dt_bias ? load_param(p.dt_bias, p.dt_bias_type, d) : 0.f;
    S *const state = reinterpret_cast<S *>(p.state);
    // This lane's batch row for x, dt, z and the output: bb * 4 + part.
    const uint32_t bp0 = bb * U + uint32_t(part);
    const uint32_t bp = bp0 < batch ? bp0 : batch - 1;
    const T xp = reinterpret_cast<const T *>(p.x)[int64_t(bp) * p.x_batch_stride + int64_t(d) * p.x_d_stride];
    const T dtp = reinterpret_cast<const T *>(p.dt)[int64_t(bp) * p.dt_batch_stride + int64_t(d) * p.dt_d_stride];
    T zp{};
    if (p.z) zp = reinterpret_cast<const T *>(p.z)[int64_t(bp) * p.z_batch_stride + int64_t(d) * p.z_d_stride];
    float4 sv[U];
    uint2 sw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t b0 = bb * U + u;
        const uint32_t b = b0 < batch ? b0 : batch - 1;
        const S *sp = state + int64_t(b) * p.state_batch_stride + int64_t(d) * p.state_d_stride + 4 * part;
        if constexpr (std::is_same_v<S, float>) sv[u] = *reinterpret_cast<const float4 *>(sp);
        else sw[u] = *reinterpret_cast<const uint2 *>(sp);
    }
    __syncthreads();   // sBC written
    float y_mine = 0.f;
    static_for<0, U>([&](auto Uc) {
        constexpr int u = decltype(Uc)::value;
        const uint32_t b = bb * U + u;
        const float4 b4 = *reinterpret_cast<const float4 *>(&sBC[(u * 2 + 0) * 16 + 4 * part]);
        const float4 c4 = *reinterpret_cast<const float4 *>(&sBC[(u * 2 + 1) * 16 + 4 * part]);
        float dt = to_f32(from_bits<T>(quad_bcast<u>(raw_bits(dtp)))) + bias;
        if (p.dt_softplus) dt = softplus_fast(dt);
        const float x = to_f32(from_bits<T>(quad_bcast<u>(raw_bits(xp))));
        const float dtx = dt * x;
        const float dl = dt * kLog2e;
        float4 st;
        if constexpr (std::is_same_v<S, float>) st = sv[u];
        else st = unpack4<S>(sw[u]);
        st.x = __builtin_fmaf(st.x, decay_exp2(dl, a4.x), dtx * b4.x);
        st.y = __builtin_fmaf(st.y, decay_exp2(dl, a4.y), dtx * b4.y);
        st.z = __builtin_fmaf(st.z, decay_exp2(dl, a4.z), dtx * b4.z);
        st.w = __builtin_fmaf(st.w, decay_exp2(dl, a4.w), dtx * b4.w);
        if (dr < dim && b < batch) {
            S *sp = state + int64_t(b) * p.state_batch_stride + int64_t(dr) * p.state_d_stride + 4 * part;
            if constexpr (std::is_same_v<S, float>) *reinterpret_cast<float4 *>(sp) = st;
            else *reinterpret_cast<uint2 *>(sp) = pack4<S>(st);
        }
        // y from the float32 state, before a 16-bit state is rounded.
        float y = __builtin_fmaf(st.x, c4.x, __builtin_fmaf(st.y, c4.y, __builtin_fmaf(st.z, c4.z, st.w * c4.w)));
        y += __shfl_xor(y, 1, 4);
        y += __shfl_xor(y, 2, 4);
        if (part == u) y_mine = y;
    });
    if (dr < dim && bp0 < batch) {
        float y = __builtin_fmaf(Dv, to_f32(xp), y_mine);
        if (p.z) y *= silu_fast(to_f32(zp));
        reinterpret_cast<T *>(p.out)[int64_t(bp0) * p.out_batch_stride + int64_t(dr) * p.out_d_stride] = from_f32<T>(y);
    }
}

}  // namespace mm

// ================================================================================================
// Host side: validation, dispatch, error reporting.
// ================================================================================================
// Scratch of mm_scan_fwd_noalloc: the sequence-segment carries of the dstate-16 forward. One copy
// per GPU (a device variable of the code object), held until the process ends. Host code never
// passes `scratch` itself to a kernel or copy: it is a host-side stand-in whose device address
// differs per GPU; noalloc_scratch() looks that address up once per device.
static __device__ __align__(256) float scratch[MM_SCAN_FWD_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int elem_bytes(mm_dtype t) { return t == MM_FLOAT32 ? 4 : 2; }

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

namespace mm {

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(int(e), "%s: launch failed: %s", what, hipGetErrorString(e));
    g_err[0] = '\0';
    return MM_OK;
}

int set_error(int code, const char *msg) { return fail(code, "%s", msg); }

// 16-byte vector I/O is legal when every row start is 16-byte aligned and L is a multiple of 8.
bool fwd_vector_ok(const mm_scan_fwd_params *p) {
    const int64_t eb = elem_bytes(p->itype);
    auto row_ok = [&](const void *base, int64_t s0, int64_t s1) {
        return base == nullptr || (aligned16(base) && (s0 * eb) % 16 == 0 && (s1 * eb) % 16 == 0);
    };
    if (p->seqlen % 8 != 0) return false;
    bool ok = row_ok(p->u, p->u_batch_stride, p->u_d_stride) && row_ok(p->delta, p->delta_batch_stride, p->delta_d_stride) &&
              row_ok(p->z, p->z_batch_stride, p->z_d_stride) && row_ok(p->out, p->out_batch_stride, p->out_d_stride) &&
              row_ok(p->out_z, p->out_z_batch_stride, p->out_z_d_stride);
    if (p->is_variable_B)
        ok = ok && aligned16(p->B) && (p->B_batch_stride * eb) % 16 == 0 && (p->B_group_stride * eb) % 16 == 0 &&
             (p->B_dstate_stride * eb) % 16 == 0;
    if (p->is_variable_C)
        ok = ok && aligned16(p->C) && (p->C_batch_stride * eb) % 16 == 0 && (p->C_group_stride * eb) % 16 == 0 &&
             (p->C_dstate_stride * eb) % 16 == 0;
    return ok;
}


}  // namespace mm

namespace {

int validate_fwd(const mm_scan_fwd_params *p) {
    if (!p) return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: params is NULL");
    if (p->itype != MM_FLOAT32 && p->itype != MM_FLOAT16 && p->itype != MM_BFLOAT16)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: unknown itype %d", int(p->itype));
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: negative size");
    if (p->dstate < 1 || p->dstate > MM_SCAN_MAX_DSTATE)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: selective_scan only supports state dimension <= %d (got %lld)",
                    MM_SCAN_MAX_DSTATE, (long long)p->dstate);
    if (p->n_groups < 1 || (p->dim > 0 && p->dim % p->n_groups != 0))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: dim (%lld) must be a multiple of n_groups (%lld)",
                    (long long)p->dim, (long long)p->n_groups);
    if (p->batch == 0 || p->dim == 0) return MM_OK;
    if (!p->u || !p->delta || !p->A || !p->B || !p->C)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: u, delta, A, B and C are required");
    if (p->z && !p->out_z)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: out_z is required when z is given");
    if (!p->z && p->out_z)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: out_z given without z");
    if (!p->out && !p->out_z && !p->last_state && !p->chunk_states && !p->tile_states)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: no output requested");
    // Low-rank coupling (selective_scan.cpp:342-359): P and Q together, rank <= 8.
    if ((p->P == nullptr) != (p->Q == nullptr))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: P and Q must be given together");
    if (p->P && (p->pq_rank < 0 || p->pq_rank > 8))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: pq_rank must be in [0, 8] (got %lld)",
                    (long long)p->pq_rank);
    if (p->tile_states && p->dstate > 16)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: tile_states need dstate <= 16");
    if (p->tile_states && !p->P && !p->chunk_states)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_fwd: without P/Q, tile_states are written with chunk_states "
                                             "(the training forward)");
    if (p->tile_states && !p->P && !mm::tile_states_ok(*p) && !mm::diag_via_pq_fwd(*p))
        return fail(MM_ERR_UNSUPPORTED, "mm_scan_fwd: without P/Q, tile_states are written by the dstate-16 kernels "
                                        "and, below dstate 16, by the P/Q kernels with a zero coupling (variable "
                                        "B/C, dim and dim / n_groups multiples of 16, L a multiple of 8, aligned "
                                        "rows); mm_scan_fwd_tile_states_size tells");
    return MM_OK;
}

template <typename T, int NS>
int launch_rowlane_ns(const mm_scan_fwd_params &p, hipStream_t s, bool vec) {
    const int64_t ratio = p.dim / p.n_groups;
    // The B/C row of a 64-lane block is uniform when no block straddles a group boundary.
    const int32_t uniform_g = (p.n_groups == 1 || ratio % mm::kRowBlock == 0) ? 1 : 0;
    dim3 grid(unsigned((p.dim + mm::kRowBlock - 1) / mm::kRowBlock), unsigned(p.batch));
    if (vec)
        hipLaunchKernelGGL((mm::scan_fwd_rowlane<T, NS, true>), grid, dim3(mm::kRowBlock), 0, s, p, ratio, uniform_g);
    else
        hipLaunchKernelGGL((mm::scan_fwd_rowlane<T, NS, false>), grid, dim3(mm::kRowBlock), 0, s, p, ratio, uniform_g);
    return mm::launch_status("scan_fwd_rowlane");
}

template <typename T>
int launch_rowlane(const mm_scan_fwd_params &p, hipStream_t s) {
    const bool vec = mm::fwd_vector_ok(&p);
    if (p.dstate <= 16) return launch_rowlane_ns<T, 16>(p, s, vec);
    if (p.dstate <= 32) return launch_rowlane_ns<T, 32>(p, s, vec);
    if (p.dstate <= 64) return launch_rowlane_ns<T, 64>(p, s, vec);
    return launch_rowlane_ns<T, MM_SCAN_MAX_DSTATE>(p, s, vec);
}

template <typename T>
int dispatch_fwd(const mm_scan_fwd_params &p, hipStream_t s) {
    if (p.P) return mm::launch_pq<T>(p, s);
    if (mm::diag_via_pq_fwd(p)) {
        mm_scan_fwd_params q = p;
        if (mm::attach_zero_pair(q) == MM_OK) return mm::launch_pq<T>(q, s, true);
    }
    int rc = mm::try_launch_tiled<T>(p, s);
    if (rc != MM_ERR_UNSUPPORTED || p.tile_states) return rc;   // the general kernel writes no tile states
    return launch_rowlane<T>(p, s);
}

// ------------------------------------------------------------------------------------------------
int validate_bwd(const mm_scan_bwd_params *p) {
    if (!p) return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: params is NULL");
    if (p->itype != MM_FLOAT32 && p->itype != MM_FLOAT16 && p->itype != MM_BFLOAT16)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: unknown itype %d", int(p->itype));
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: negative size");
    if (p->dstate < 1 || p->dstate > MM_SCAN_MAX_DSTATE)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: selective_scan only supports state dimension <= %d (got %lld)",
                    MM_SCAN_MAX_DSTATE, (long long)p->dstate);
    if (p->n_groups < 1 || (p->dim > 0 && p->dim % p->n_groups != 0))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: dim (%lld) must be a multiple of n_groups (%lld)",
                    (long long)p->dim, (long long)p->n_groups);
    if (p->batch == 0 || p->dim == 0) return MM_OK;
    if (!p->u || !p->delta || !p->A || !p->B || !p->C || !p->dout)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: u, delta, A, B, C and dout are required");
    if (!p->du || !p->ddelta || !p->dA || !p->dB || !p->dC)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: du, ddelta, dA, dB and dC are required");
    if (p->z && (!p->out || !p->dz))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: out and dz are required when z is given");
    if ((p->D == nullptr) != (p->dD == nullptr))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: dD is required exactly when D is given");
    if ((p->delta_bias == nullptr) != (p->ddelta_bias == nullptr))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: ddelta_bias is required exactly when delta_bias is given");
    if ((p->P == nullptr) != (p->Q == nullptr))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: P and Q must both be given or both be NULL");
    if (p->P && (!p->dP || !p->dQ))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: dP and dQ are required when P and Q are given");
    if (p->P && (p->pq_rank < 1 || p->pq_rank > 8))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: pq_rank must be in [1, 8] (got %lld)", (long long)p->pq_rank);

    const int64_t need = mm::bwd_workspace_min_bytes(*p);
    if (p->seqlen > 0 && (!p->workspace || p->workspace_bytes < need || reinterpret_cast<uintptr_t>(p->workspace) % 16))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_scan_bwd: needs a 16-byte aligned workspace of %lld bytes (got %lld)",
                    (long long)need, (long long)p->workspace_bytes);
    return MM_OK;
}

// ------------------------------------------------------------------------------------------------
int validate_su(const mm_state_update_params *p) {
    if (!p) return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: params is NULL");
    auto known = [](mm_dtype t) { return t == MM_FLOAT32 || t == MM_FLOAT16 || t == MM_BFLOAT16; };
    if (!known(p->itype))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: unknown itype %d", int(p->itype));
    if (!known(p->state_type) || !known(p->D_type) || !known(p->dt_bias_type))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: unknown state_type, D_type or dt_bias_type");
    if (p->batch < 0 || p->dim < 0)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: negative size");
    if (p->dstate < 1 || p->dstate > MM_SCAN_MAX_DSTATE)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: dstate must be in [1, %d]", MM_SCAN_MAX_DSTATE);
    if (p->n_groups < 1 || (p->dim > 0 && p->dim % p->n_groups != 0))
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: dim must be a multiple of n_groups");
    if (p->batch == 0 || p->dim == 0) return MM_OK;
    if (!p->state || !p->x || !p->dt || !p->A || !p->B || !p->C || !p->out)
        return fail(MM_ERR_INVALID_ARGUMENT, "mm_state_update: state, x, dt, A, B, C and out are required");
    return MM_OK;
}

template <typename T, typename S, int SPL, int LPR>
int launch_su(const mm_state_update_params &p, hipStream_t s) {
    const int64_t threads = p.batch * p.dim * LPR;
    // gridDim.x * blockDim.x must stay below 2^32.
    if ((threads + mm::kDecBlock - 1) / mm::kDecBlock >= (int64_t(1) << 24))
        return fail(MM_ERR_UNSUPPORTED, "mm_state_update: batch * dim too large for one launch");
    dim3 grid(unsigned((threads + mm::kDecBlock - 1) / mm::kDecBlock));
    hipLaunchKernelGGL((mm::state_update_kernel<T, S, SPL, LPR>), grid, dim3(mm::kDecBlock), 0, s, p, p.dim / p.n_groups);
    return mm::launch_status("state_update");
}

// The vectorised dstate-16 kernel's layout requirements: unit state strides and 4-element aligned
// rows of state, A, B and C.
bool su_vec16_ok(const mm_state_update_params &p) {
    const int64_t eb = elem_bytes(p.itype);
    auto al = [](const void *ptr, int64_t bytes) { return (reinterpret_cast<uintptr_t>(ptr) % uintptr_t(bytes)) == 0; };
    return p.dstate == 16 && p.state_dstate_stride == 1 && p.A_dstate_stride == 1 && p.B_dstate_stride == 1 &&
           p.C_dstate_stride == 1 && al(p.state, 4 * elem_bytes(p.state_type)) && p.state_batch_stride % 4 == 0 &&
           p.state_d_stride % 4 == 0 &&
           al(p.A, 16) && p.A_d_stride % 4 == 0 && al(p.B, 4 * eb) && al(p.C, 4 * eb) && p.B_batch_stride % 4 == 0 &&
           p.B_group_stride % 4 == 0 && p.C_batch_stride % 4 == 0 && p.C_group_stride % 4 == 0;
}

template <typename T, typename S, int U>
int launch_vec16(const mm_state_update_params &p, hipStream_t s) {
    const int64_t n_dblk = (p.dim + 63) / 64;
    const int64_t n_bblk = (p.batch + U - 1) / U;
    hipLaunchKernelGGL((mm::state_update_vec16<T, S, U>), dim3(unsigned(n_bblk * n_dblk)), dim3(mm::kDecBlock), 0, s, p,
                       uint32_t(p.dim / p.n_groups), uint32_t(n_dblk));
    return mm::launch_status("state_update");
}

template <typename T, typename S>
int launch_vec16x(const mm_state_update_params &p, hipStream_t s) {
    const int64_t n_dblk = (p.dim + 63) / 64;
    const int64_t n_bblk = (p.batch + 3) / 4;
    hipLaunchKernelGGL((mm::state_update_vec16x<T, S>), dim3(unsigned(n_bblk * n_dblk)), dim3(mm::kDecBlock), 0, s, p,
                       uint32_t(p.dim / p.n_groups), uint32_t(n_dblk));
    return mm::launch_status("state_update");
}

template <typename T, typename S>
int dispatch_su_state(const mm_state_update_params &p, hipStream_t s) {
    // A 1-D grid of fewer than 2^24 workgroups of 256 lanes keeps gridDim.x * blockDim.x < 2^32.
    const int64_t U = p.batch >= 4 ? 4 : 1;
    if (su_vec16_ok(p) && p.dim < (int64_t(1) << 31) && p.batch < (int64_t(1) << 31) &&
        ((p.batch + U - 1) / U) * ((p.dim + 63) / 64) < (int64_t(1) << 24)) {
        // Four batch rows per workgroup share the loads of A, D and dt_bias (batch 256: 41 -> 37 us),
        // and, when the workgroup's 64 channels lie in one group, those of x, dt, z, B and C
        // (MM_SU_KERNEL=vec16 keeps the per-row loads, for comparison).
        static const bool per_row = [] {
            const char *e = getenv("MM_SU_KERNEL");
            return e && !strcmp(e, "vec16");
        }();
        const int64_t ratio = p.dim / p.n_groups;
        if (p.batch >= 4 && !per_row && (p.n_groups == 1 || ratio % 64 == 0)) return launch_vec16x<T, S>(p, s);
        if (p.batch >= 4) return launch_vec16<T, S, 4>(p, s);
        return launch_vec16<T, S, 1>(p, s);
    }
    if (p.dstate <= 16) return launch_su<T, S, 4, 4>(p, s);
    if (p.dstate <= 64) return launch_su<T, S, 4, 16>(p, s);
    return launch_su<T, S, 16, 16>(p, s);
}

template <typename T>
int dispatch_su(const mm_state_update_params &p, hipStream_t s) {
    switch (p.state_type) {
        case MM_FLOAT16: return dispatch_su_state<T, mm::f16_t>(p, s);
        case MM_BFLOAT16: return dispatch_su_state<T, mm::bf16_t>(p, s);
        default: return dispatch_su_state<T, float>(p, s);
    }
}

// The device address of `scratch` on the current GPU, looked up with hipGetSymbolAddress on the
// first call on each device (with that device current) and kept per device; later calls on the
// device reuse it. Concurrent first calls may both look it up; they store the same address.
constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];

int noalloc_scratch(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(int(e), "mm_scan_fwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(MM_ERR_UNSUPPORTED, "mm_scan_fwd_noalloc: device index %d out of range", dev);
    void *ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (ptr == nullptr) {
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return fail(e != hipSuccess ? int(e) : MM_ERR_UNSUPPORTED,
                        "mm_scan_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
    *out = ptr;
    return MM_OK;
}

}  // namespace

extern "C" {

int mm_scan_fwd(const mm_scan_fwd_params *params, void *stream) {
    int rc = validate_fwd(params);
    if (rc != MM_OK) return rc;
    const mm_scan_fwd_params &p = *params;
    if (p.batch == 0 || p.dim == 0) return MM_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return dispatch_fwd<float>(p, s);
        case MM_FLOAT16: return dispatch_fwd<mm::f16_t>(p, s);
        default: return dispatch_fwd<mm::bf16_t>(p, s);
    }
}

int mm_state_update(const mm_state_update_params *params, void *stream) {
    int rc = validate_su(params);
    if (rc != MM_OK) return rc;
    const mm_state_update_params &p = *params;
    if (p.batch == 0 || p.dim == 0) return MM_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return dispatch_su<float>(p, s);
        case MM_FLOAT16: return dispatch_su<mm::f16_t>(p, s);
        default: return dispatch_su<mm::bf16_t>(p, s);
    }
}

int mm_scan_bwd(const mm_scan_bwd_params *params, void *stream) {
    int rc = validate_bwd(params);
    if (rc != MM_OK) return rc;
    const mm_scan_bwd_params &p = *params;
    if (p.batch == 0 || p.dim == 0) return MM_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return mm::launch_bwd<float>(p, s);
        case MM_FLOAT16: return mm::launch_bwd<mm::f16_t>(p, s);
        default: return mm::launch_bwd<mm::bf16_t>(p, s);
    }
}

int64_t mm_scan_bwd_workspace_size(const mm_scan_bwd_params *params) {
    if (!params || params->batch < 0 || params->dim < 0 || params->seqlen < 0 || params->dstate < 1 ||
        params->dstate > MM_SCAN_MAX_DSTATE || params->n_groups < 1 ||
        (params->dim > 0 && params->dim % params->n_groups != 0))
        return 0;
    return mm::bwd_workspace_bytes(*params);
}

int64_t mm_scan_fwd_tile_states_size(const mm_scan_fwd_params *params) {
    if (!params || params->batch < 0 || params->dim < 0 || params->seqlen < 0 || params->dstate < 1 ||
        params->dstate > 16 || params->n_groups < 1 || (params->dim > 0 && params->dim % params->n_groups))
        return 0;
    const mm_scan_fwd_params &p = *params;
    if (!p.P && (!p.chunk_states || !(mm::tile_states_ok(p) || mm::diag_via_pq_fwd(p)))) return 0;
    return ((p.seqlen + 15) / 16) * p.batch * p.dim * 16 * int64_t(sizeof(float));
}

int64_t mm_scan_fwd_workspace_size(const mm_scan_fwd_params *params) {
    if (validate_fwd(params) != MM_OK) return 0;
    if (params->batch == 0 || params->dim == 0 || params->P) return 0;
    return mm::segment_workspace_bytes(*params, mm::segment_count(*params));
}

int mm_scan_fwd_noalloc(const mm_scan_fwd_params *params, void *stream) {
    int rc = validate_fwd(params);
    if (rc != MM_OK) return rc;
    if (params->batch == 0 || params->dim == 0) return MM_OK;
    mm_scan_fwd_params p = *params;
    p.workspace = nullptr;
    p.workspace_bytes = 0;
    // A segment plan larger than the static buffer: the single-pass kernels (workspace left NULL).
    const int64_t need = mm_scan_fwd_workspace_size(params);
    if (need > 0 && need <= int64_t(MM_SCAN_FWD_NOALLOC_SCRATCH_BYTES)) {
        rc = noalloc_scratch(&p.workspace);
        if (rc != MM_OK) return rc;
        p.workspace_bytes = MM_SCAN_FWD_NOALLOC_SCRATCH_BYTES;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return dispatch_fwd<float>(p, s);
        case MM_FLOAT16: return dispatch_fwd<mm::f16_t>(p, s);
        default: return dispatch_fwd<mm::bf16_t>(p, s);
    }
}

const char *mm_last_error(void) { return g_err; }

int mm_abi_version(void) { return MM_SCAN_ABI_VERSION; }

}  // extern "C"
