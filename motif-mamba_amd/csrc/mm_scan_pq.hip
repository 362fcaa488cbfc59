// mm_scan_pq.hip -- gfx950 forward selective scan with the MotifMamba low-rank P/Q coupling.
//
// Reference behaviour: selective_scan_full_matrix_cuda (mamba_ssm/ops/selective_scan_interface.py:
// 262-350), the path selective_scan_fn takes for P/Q (selective_scan_interface.py:237-259), and the
// dense CUDA forward selective_scan_fwd_dense_pq_kernel (csrc/selective_scan/
// selective_scan_fwd_kernel.cuh:159-251, one thread per (batch, channel) row). The recurrence
//
//     h_t = exp(dt'_t A[d,:]) * h_{t-1} + dt'_t P_d (Q_d h_{t-1}) + dt'_t u_t B_t
//
// couples every state of a row to every other one through the rank-R product, so a row is not a
// set of independent per-state scans: each state needs Q h_{t-1} before it can take step t. The
// design of this file is its own:
//
//   scan_fwd_pq_tiled<T, S, LPR, R>   a wave64 owns 64/LPR channels of one (batch, group); the LPR
//       consecutive lanes of a channel hold S states each (S * LPR >= dstate, padded with states
//       whose A, P, Q, B and C are zero, which stay zero). Per step each lane forms its partial
//       Q h over its S states, a DPP butterfly inside the LPR lanes sums the partials (every lane
//       ends with the same bits; where the rank is at most LPR one transposed butterfly serves all
//       R sums, lane_sums in mm_common.h), and the lane updates its S states with
//       P (dt' q) + dt' u B.
//       The lane's rows of P and Q live in registers for the whole sequence. (16-bit inputs with
//       16 lanes of one state and rank <= 2 carry the butterfly's total from step to step and form
//       the next partial as Q (a h + dt' u B) + (Q P) q, which shortens the dependent chain.)
//       * B and C of the (batch, group) are staged per 32-step tile in LDS as float32, [step][state],
//         and each step reads the lane's S states as one vector.
//       * dt' = softplus(delta + bias) and dt' u are computed once per (channel, step): each lane
//         owns 32/LPR consecutive steps of its channel per tile and shares them through LDS.
//       * Per-lane partial sums of y = sum_n C_n h_n go back through LDS; the owner of the step adds
//         the LPR partials in lane order, applies D u and the silu(z) gate and stores.
//       * Global loads for tile i+1 are issued before the scan of tile i.
//   scan_fwd_pq_rowlane<T>   one lane per row, the row's states in LDS, P/Q read through the cache
//       every step: any dstate <= 256, constant B/C, any strides and lengths.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <algorithm>
#include <atomic>

#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace pq {

constexpr int kT = 32;      // sequence steps per tile
constexpr int kPad = 36;    // LDS row stride (floats) of per-channel step rows: 16-B aligned, spreads banks
constexpr int kMaxRank = 8; // selective_scan.cpp:359

// S consecutive floats of LDS (16-B, 8-B or 4-B aligned by construction).
template <int S>
__device__ __forceinline__ void lds_read_vec(const float *src, float *o) {
    if constexpr (S == 4) {
        const float4 v = *reinterpret_cast<const float4 *>(src);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else if constexpr (S == 2) {
        const float2 v = *reinterpret_cast<const float2 *>(src);
        o[0] = v.x; o[1] = v.y;
    } else {
        o[0] = *src;
    }
}

// DX: the chunk states in the diagonal scan's form, (prod of the decays since step 0, h), for the
// diagonal requests run with a zero P/Q pair; otherwise (1, h), the P/Q form.
template <typename T, int S, int LPR, int R, bool DX = false>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
scan_fwd_pq_tiled(const mm_scan_fwd_params p, const int64_t ratio, const int32_t blocks_per_group) {
    constexpr int NP = S * LPR;            // padded states per channel
    constexpr int CPW = 64 / LPR;          // channels per wave
    constexpr int E = kT / LPR;            // prologue / epilogue steps per lane per tile
    // sBC row stride (floats): NP B values, then NP C values. The staging writes, for one element
    // position, lanes (state n = lane / 4, step block q = lane % 4) at q 8 BCS + n: with BCS = 2 NP + 2
    // (S <= 2; the scan reads S-vectors of 8 bytes) 8 BCS = 16 mod 64, so the 64 lanes cover 64
    // consecutive banks; S = 4 needs 16-byte aligned rows (2 NP + 4).
    constexpr int BCS = S <= 2 ? 2 * NP + 2 : 2 * NP + 4;
    constexpr int HR = NP / 16;            // B/C half-rows (16 steps of one state) staged per lane
    static_assert(HR >= 1 && E >= 2 && E % 2 == 0 && 2 * CPW <= 64, "tile shape");
    __shared__ __align__(16) float sBC[kT * BCS];
    // During the scan: dt' rows then dt'u rows of the wave's channels; after it: the y partials.
    __shared__ __align__(16) float sX[64 * kPad];
    float *sDt = sX;
    float *sDu = sX + CPW * kPad;
    float *sY = sX;

    const int lane = threadIdx.x;
    const int cw = lane / LPR;             // channel slot in the wave
    const int k = lane % LPR;              // state slice: states k S .. k S + S - 1
    const int64_t b = blockIdx.y;
    const int64_t g = blockIdx.x / blocks_per_group;
    const int64_t cl = int64_t(blockIdx.x % blocks_per_group) * CPW + cw;  // channel within the group
    const bool active = cl < ratio;
    const int64_t d = g * ratio + (active ? cl : ratio - 1);  // inactive slots mirror a real channel
    const int64_t L = p.seqlen;
    const int N = int(p.dstate);
    const int rank = int(p.pq_rank);

    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    const T *Bg = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cg = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;

    // XK: the carried form described below. TS: the coupling's R sums over the channel's lanes are one transposed
    // reduction (lane_sums, R <= LPR), which wants the lane's rows of Q and columns of P in its
    // order: position t holds rank t ^ ro.
    constexpr bool XK = LPR == 16 && S == 1 && R <= 2 && !std::is_same<T, float>::value;
    constexpr bool TS = R <= LPR && !XK;
    int ro = 0;
    if constexpr (TS) ro = lane_rank_offset<LPR, R>(k);
    float A2[S], h[S], Pr[S][R], Qr[R][S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int n = k * S + s;
        const bool on = n < N;
        A2[s] = on ? p.A[d * p.A_d_stride + n * p.A_dstate_stride] * kLog2e : 0.f;
        h[s] = 0.f;
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const int j = t ^ ro;
            const bool use = on && j < rank;
            Pr[s][t] = use ? p.P[d * p.P_d_stride + n * p.P_dstate_stride + j * p.P_r_stride] : 0.f;
            Qr[t][s] = use ? p.Q[d * p.Q_d_stride + j * p.Q_r_stride + n * p.Q_dstate_stride] : 0.f;
        }
    }
    // With 16 lanes of one state per channel (dstate <= 16, chosen when their waves fit one per
    // SIMD, where each step's dependent chain sets the time) and rank <= 2, the coupling carries
    // gq = Q h_{t-1} over all states of the channel from step to step (h = 0 before the first
    // step) and forms the next one as Q hb + K q with K = Q P over the lane's states (R x R): the
    // chain from gq to the next gq is then q, R fmas and the butterfly instead of q, the P fmas,
    // the S-term dot product and the butterfly, for R^2 + R S more VALU per step. Measured at one
    // wave per SIMD: -8 % at one state per lane, +4 % at two (the extra VALU outweigh the shorter
    // chain); +10 % at two waves per SIMD with 8 lanes, where issue sets the time. 16-bit inputs
    // only: float32 callers keep the direct Q h, whose rounding the long-sequence float32 checks
    // pin; 16-bit outputs round far above the float32 rounding difference of the two forms.
    float Kr[R][R], gq[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        gq[r] = 0.f;
#pragma unroll
        for (int r2 = 0; r2 < R; ++r2) {
            float acc = Qr[r][0] * Pr[0][r2];
#pragma unroll
            for (int s = 1; s < S; ++s) acc = __builtin_fmaf(Qr[r][s], Pr[s][r2], acc);
            Kr[r][r2] = acc;
        }
    }
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const bool softplus = p.delta_softplus != 0;
    const int es = E * k;                  // first step (within a tile) of this lane's elements
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    float cum_dt = 0.f;                    // DX: running sum of dt' (prod a = exp2(A log2e cum_dt))
    // Checkpoints for the backward: the S states of this lane before every 16-step tile.
    const int64_t ck_tile = p.batch * p.dim * 16;
    float *const ckp = (p.tile_states && active) ? p.tile_states + (b * p.dim + d) * 16 + k * S : nullptr;
    auto put_ck = [&](int64_t j) {
#pragma unroll
        for (int s = 0; s < S; ++s) ckp[j * ck_tile + s] = h[s];
    };

    // The loads of u, delta and z go through buffer resources: the rows of the wave's channels from
    // its first channel dw, with 32-bit byte offsets per lane (the host checks that every offset of
    // these rows fits). A whole tile adds its start as a scalar offset; only the last, partial
    // tile clamps per lane. (B and C, a tensor per lane, keep per-lane pointers: a resource
    // descriptor must be uniform.)
    constexpr uint32_t SZ = sizeof(T);
    const int64_t dw = g * ratio + int64_t(blockIdx.x % blocks_per_group) * CPW;
    const int64_t dl = d - dw;             // 0 .. CPW - 1 (inactive slots mirror the group's last channel)
    const __amdgpu_buffer_rsrc_t rs_u = buffer_rsrc(reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + dw * p.u_d_stride);
    const __amdgpu_buffer_rsrc_t rs_d =
        buffer_rsrc(reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + dw * p.delta_d_stride);
    const __amdgpu_buffer_rsrc_t rs_z =    // (p.z, not zp: the condition must be uniform)
        buffer_rsrc(p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + dw * p.z_d_stride : nullptr);
    const uint32_t fo_u = uint32_t(dl * p.u_d_stride) * SZ, fo_d = uint32_t(dl * p.delta_d_stride) * SZ;
    const uint32_t fo_z = uint32_t(dl * p.z_d_stride) * SZ;
    // The outputs likewise (stores only from lanes of real channels, at existing steps).
    const __amdgpu_buffer_rsrc_t rs_o =
        buffer_rsrc(p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + dw * p.out_d_stride : nullptr);
    const __amdgpu_buffer_rsrc_t rs_oz =
        buffer_rsrc(p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + dw * p.out_z_d_stride : nullptr);
    const uint32_t fo_o = uint32_t(dl * p.out_d_stride + es) * SZ, fo_oz = uint32_t(dl * p.out_z_d_stride + es) * SZ;

    // B and C of the (batch, group) through buffer resources too. Per 32-step tile every lane stages
    // NU = NP / 16 units of each tensor: unit u = lane + 64 i is the 8 steps 8 (u % 4) .. + 7 of
    // state u / 4, one 8-element load from B and one from C (a 32-bit offset per lane, the tile
    // start as a scalar offset). Units of padded states (u / 4 >= dstate) and, in a last partial
    // tile, units past L (L is a multiple of 8: a unit is all in or all out) are zeroed once when
    // loaded, so the staging below writes every unit unconditionally.
    constexpr int NU = NP / 16;
    const __amdgpu_buffer_rsrc_t rs_B = buffer_rsrc(Bg), rs_C = buffer_rsrc(Cg);
    uint32_t fo_B[NU], fo_C[NU];
    int u_lds[NU], u_q[NU];
    bool u_on[NU];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const int u = lane + 64 * i;
        const int n = u / 4;
        u_q[i] = u % 4;
        u_on[i] = n < N;
        const int64_t nn = n < N ? n : 0;
        fo_B[i] = uint32_t(nn * p.B_dstate_stride) * SZ;
        fo_C[i] = uint32_t(nn * p.C_dstate_stride) * SZ;
        u_lds[i] = 8 * u_q[i] * BCS + n;
    }
    const bool padded = N < NP;            // uniform

    // Loads at or past the end of a row are redirected into the row's last elements (always in
    // bounds: L is a multiple of 8); the steps they feed are padding with dt' = 0.
    const int64_t lastE = L - E;
    // Loads run D tiles ahead: rings of D entries (elements, B/C) whose registers stay fixed (the
    // tile loop is unrolled by D below; copying an entry whose loads are in flight would wait for
    // them). D = 2 where the second entry fits in registers (S <= 2); at S = 4 it would spill.
    constexpr int D = S <= 2 ? 2 : 1;
    struct Elems {
        RawVec<T, E> u, d, z;
    };
    auto load_elems = [&](int64_t t, Elems &e) {
        uint32_t eo, so;
        if (t + kT <= L) {                 // uniform: a whole tile
            eo = uint32_t(es) * SZ;
            so = uint32_t(t) * SZ;
        } else {
            eo = uint32_t(t + es < lastE ? t + es : lastE) * SZ;
            so = 0;
        }
        e.u = buffer_load_rawn<T, E>(rs_u, fo_u + eo, so);
        e.d = buffer_load_rawn<T, E>(rs_d, fo_d + eo, so);
        if (zp) e.z = buffer_load_rawn<T, E>(rs_z, fo_z + eo, so);
        else e.z = {};
    };
    struct BCs {
        RawVec<T, 8> b[NU], c[NU];
    };
    auto load_bc = [&](int64_t t0, BCs &r) {
        if (t0 + kT <= L) {                // uniform: a whole tile
            const uint32_t so = uint32_t(t0) * SZ;
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                r.b[i] = buffer_load_rawn<T, 8>(rs_B, fo_B[i] + uint32_t(8 * u_q[i]) * SZ, so);
                r.c[i] = buffer_load_rawn<T, 8>(rs_C, fo_C[i] + uint32_t(8 * u_q[i]) * SZ, so);
            }
        } else {                           // the last, partial tile
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const int64_t st = t0 + 8 * u_q[i];
                const uint32_t o = uint32_t(st < L ? st : L - 8) * SZ;
                r.b[i] = buffer_load_rawn<T, 8>(rs_B, fo_B[i] + o, 0);
                r.c[i] = buffer_load_rawn<T, 8>(rs_C, fo_C[i] + o, 0);
                if (st >= L) r.b[i] = r.c[i] = {};
            }
        }
        if (padded) {
#pragma unroll
            for (int i = 0; i < NU; ++i)
                if (!u_on[i]) r.b[i] = r.c[i] = {};
        }
    };
    // Tile rows [step][B states | C states] as float32 (zeros for padded states and past L).
    auto stage_bc = [&](const BCs &r) {
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            float vb[8], vc[8];
            unpack_raw<T, 8>(r.b[i], vb);
            unpack_raw<T, 8>(r.c[i], vc);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sBC[u_lds[i] + e * BCS] = vb[e];
                sBC[u_lds[i] + e * BCS + NP] = vc[e];
            }
        }
    };
    Elems e0, e1;
    BCs b0, b1;
    load_elems(0, e0);
    if (D == 2) load_elems(kT, e1);
    load_bc(0, b0);
    stage_bc(b0);
    if (D == 2) load_bc(kT, b1);

    // Tile t0: its elements in ec, its B/C (already staged) in bc, the next tile's B/C in bn (the
    // same entry as bc when D = 1: loaded at the top of the tile, staged at its end).
    auto tile = [&](const int64_t t0, Elems &ec, BCs &bc, const BCs &bn) __attribute__((always_inline)) {
        const int64_t t1 = t0 + kT;
        const bool ev = t0 + es < L;       // this lane's E elements exist (L is a multiple of E)
        float uu[E], dd[E], zz[E];
        unpack_raw<T, E>(ec.u, uu);
        unpack_raw<T, E>(ec.d, dd);
        unpack_raw<T, E>(ec.z, zz);
        // Prefetch D tiles ahead into the entries just consumed (clamped addresses: in bounds).
        load_elems(t0 + D * kT, ec);
        load_bc(t0 + D * kT, bc);

        // Prologue: dt' and dt' u of (channel, steps es .. es + E - 1).
        float dtp[E], dup[E];
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float x = dd[i] + bias;
            dtp[i] = softplus ? softplus_fast(x) : x;
            if (!ev) dtp[i] = 0.f;         // padded steps of a last, partial tile
            dup[i] = dtp[i] * uu[i];
        }
#pragma unroll
        for (int i = 0; i < E; i += 2) {
            *reinterpret_cast<float2 *>(&sDt[cw * kPad + es + i]) = make_float2(dtp[i], dtp[i + 1]);
            *reinterpret_cast<float2 *>(&sDu[cw * kPad + es + i]) = make_float2(dup[i], dup[i + 1]);
        }
        __syncthreads();
        if (ckp) put_ck(t0 / 16);

        // Scan: 32 steps in groups of 4. The decay factors and the input terms of a group do not
        // depend on the state and are formed first; then the coupled updates run in order.
        float yp[kT];
        static_for<0, kT / 4>([&](auto G4) {
            constexpr int s4 = decltype(G4)::value;
            if constexpr (s4 == 4) {
                if (ckp && t0 + 16 < L) put_ck(t0 / 16 + 1);
            }
            const float4 dt4 = *reinterpret_cast<const float4 *>(&sDt[cw * kPad + 4 * s4]);
            const float4 du4 = *reinterpret_cast<const float4 *>(&sDu[cw * kPad + 4 * s4]);
            const float dts[4] = {dt4.x, dt4.y, dt4.z, dt4.w};
            const float dus[4] = {du4.x, du4.y, du4.z, du4.w};
            float av[4][S], bu[4][S], cv[4][S];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 4 * s4 + j;
                float bv[S];
                lds_read_vec<S>(&sBC[t * BCS + k * S], bv);
                lds_read_vec<S>(&sBC[t * BCS + NP + k * S], cv[j]);
                if constexpr (DX) cum_dt += dts[j];   // steps past L have dt' = 0
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    av[j][s] = decay_exp2(dts[j], A2[s]);
                    bu[j][s] = dus[j] * bv[s];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float q[R], y = 0.f;
                if constexpr (XK) {
                    // h_t = hb + P q with hb = a h_{t-1} + dt' u B and q = dt' gq; the next step's
                    // lane partial of Q h_t as X + K q, where X = Q hb needs only h_{t-1} (off the
                    // serial chain) and K = Q P over the lane's states.
                    float hb[S], X[R];
#pragma unroll
                    for (int s = 0; s < S; ++s) hb[s] = __builtin_fmaf(av[j][s], h[s], bu[j][s]);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        X[r] = Qr[r][0] * hb[0];
#pragma unroll
                        for (int s = 1; s < S; ++s) X[r] = __builtin_fmaf(Qr[r][s], hb[s], X[r]);
                        q[r] = gq[r] * dts[j];
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float acc = X[r];
#pragma unroll
                        for (int r2 = 0; r2 < R; ++r2) acc = __builtin_fmaf(Kr[r][r2], q[r2], acc);
                        gq[r] = group_sum<LPR>(acc);
                    }
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        float w = hb[s];
#pragma unroll
                        for (int r = 0; r < R; ++r) w = __builtin_fmaf(Pr[s][r], q[r], w);
                        h[s] = w;
                        y = s == 0 ? cv[j][0] * h[0] : __builtin_fmaf(cv[j][s], h[s], y);
                    }
                } else if constexpr (TS) {
#pragma unroll
                    for (int t = 0; t < R; ++t) {
                        q[t] = Qr[t][0] * h[0];
#pragma unroll
                        for (int s = 1; s < S; ++s) q[t] = __builtin_fmaf(Qr[t][s], h[s], q[t]);
                    }
                    lane_sums<LPR, R>(q);
#pragma unroll
                    for (int t = 0; t < R; ++t) q[t] *= dts[j];
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        float w = bu[j][s];
#pragma unroll
                        for (int t = 0; t < R; ++t) w = __builtin_fmaf(Pr[s][t], q[t], w);
                        h[s] = __builtin_fmaf(av[j][s], h[s], w);
                        y = s == 0 ? cv[j][0] * h[0] : __builtin_fmaf(cv[j][s], h[s], y);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float acc = Qr[r][0] * h[0];
#pragma unroll
                        for (int s = 1; s < S; ++s) acc = __builtin_fmaf(Qr[r][s], h[s], acc);
                        q[r] = group_sum<LPR>(acc) * dts[j];
                    }
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        float w = bu[j][s];
#pragma unroll
                        for (int r = 0; r < R; ++r) w = __builtin_fmaf(Pr[s][r], q[r], w);
                        h[s] = __builtin_fmaf(av[j][s], h[s], w);
                        y = s == 0 ? cv[j][0] * h[0] : __builtin_fmaf(cv[j][s], h[s], y);
                    }
                }
                yp[4 * s4 + j] = y;
            }
        });
        __syncthreads();                   // sDt / sDu / sBC reads done: sY and sBC are rewritten

#pragma unroll
        for (int t = 0; t < kT; t += 4)
            *reinterpret_cast<float4 *>(&sY[(cw * LPR + k) * kPad + t]) = make_float4(yp[t], yp[t + 1], yp[t + 2], yp[t + 3]);
        if (t1 < L) stage_bc(bn);
        __syncthreads();

        // Epilogue: y of (channel, steps es .. es + E - 1) = the LPR partials, added in lane order.
        float y[E];
#pragma unroll
        for (int i = 0; i < E; i += 2) {
            float2 acc = *reinterpret_cast<const float2 *>(&sY[(cw * LPR) * kPad + es + i]);
#pragma unroll
            for (int kk = 1; kk < LPR; ++kk) {
                const float2 v = *reinterpret_cast<const float2 *>(&sY[(cw * LPR + kk) * kPad + es + i]);
                acc.x += v.x;
                acc.y += v.y;
            }
            y[i] = acc.x;
            y[i + 1] = acc.y;
        }
        if (active && ev) {
            float o[E];
#pragma unroll
            for (int i = 0; i < E; ++i) o[i] = p.D ? __builtin_fmaf(Dv, uu[i], y[i]) : y[i];
            if (p.out) buffer_store_vecn<T, E>(rs_o, fo_o, uint32_t(t0) * SZ, o);
            if (zp) {
#pragma unroll
                for (int i = 0; i < E; ++i) o[i] *= silu_fast(zz[i]);
                buffer_store_vecn<T, E>(rs_oz, fo_oz, uint32_t(t0) * SZ, o);
            }
        }
        if (active && p.chunk_states) {
            const int64_t tend = t1 < L ? t1 : L;
            if (tend % MM_SCAN_CHUNK == 0 || tend == L) {
                const int64_t c = (tend - 1) / MM_SCAN_CHUNK;
                float *cs = p.chunk_states + ((b * p.dim + d) * n_chunks + c) * 2 * N;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const int n = k * S + s;
                    if (n < N) {
                        cs[2 * n] = DX ? __builtin_amdgcn_exp2f(A2[s] * cum_dt) : 1.f;
                        cs[2 * n + 1] = h[s];
                    }
                }
            }
        }
        __syncthreads();                   // sY reads done before the next prologue overwrites sX
    };
    if constexpr (D == 2) {
        for (int64_t t0 = 0; t0 < L; t0 += 2 * kT) {
            tile(t0, e0, b0, b1);
            if (t0 + kT < L) tile(t0 + kT, e1, b1, b0);
        }
    } else {
        for (int64_t t0 = 0; t0 < L; t0 += kT) tile(t0, e0, b0, b0);
    }
    if (active && p.last_state) {
        float *ls = p.last_state + (b * p.dim + d) * N;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int n = k * S + s;
            if (n < N) ls[n] = h[s];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// General kernel: one lane per (batch, channel) row; the row's states in LDS (dstate x 64 floats per
// block, lane-minor so every access is conflict-free), P and Q read through the cache.
// ------------------------------------------------------------------------------------------------
constexpr int kRowBlock = 64;

template <typename T>
__global__ void __launch_bounds__(kRowBlock)
scan_fwd_pq_rowlane(const mm_scan_fwd_params p, const int64_t ratio) {
    extern __shared__ float sH[];          // [dstate][64]
    const int lane = threadIdx.x;
    const int64_t d_raw = int64_t(blockIdx.x) * blockDim.x + lane;
    const int64_t b = blockIdx.y;
    const bool active = d_raw < p.dim;
    const int64_t d = active ? d_raw : p.dim - 1;  // clamped for loads; stores are predicated
    const int64_t g = d / ratio;
    const int64_t L = p.seqlen;
    const int N = int(p.dstate);
    const int rank = int(p.pq_rank);

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    T *op = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    T *ozp = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    const T *Bv = p.is_variable_B ? reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride : nullptr;
    const T *Cv = p.is_variable_C ? reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride : nullptr;
    const float *Bc = reinterpret_cast<const float *>(p.B) + d * p.B_d_stride;
    const float *Cc = reinterpret_cast<const float *>(p.C) + d * p.C_d_stride;
    const float *Ad = p.A + d * p.A_d_stride;
    const float *Pd = p.P + d * p.P_d_stride;
    const float *Qd = p.Q + d * p.Q_d_stride;

    for (int n = 0; n < N; ++n) sH[n * kRowBlock + lane] = 0.f;
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;

    for (int64_t t = 0; t < L; ++t) {
        if (p.tile_states && active && t % 16 == 0) {
            // The state before this 16-step tile, for the backward (states past dstate are 0).
            float *ck = p.tile_states + ((t / 16) * p.batch * p.dim + b * p.dim + d) * 16;
            for (int n = 0; n < 16; ++n) ck[n] = n < N ? sH[n * kRowBlock + lane] : 0.f;
        }
        float dt = to_f32(dp[t]) + bias;
        if (p.delta_softplus) dt = softplus_fast(dt);
        const float uu = to_f32(up[t]);
        const float du = dt * uu;
        // q = dt' (Q h_{t-1}), from the state before this step.
        float q[kMaxRank];
#pragma unroll
        for (int j = 0; j < kMaxRank; ++j) q[j] = 0.f;
        for (int n = 0; n < N; ++n) {
            const float hn = sH[n * kRowBlock + lane];
#pragma unroll
            for (int j = 0; j < kMaxRank; ++j)
                if (j < rank) q[j] = __builtin_fmaf(Qd[j * p.Q_r_stride + n * p.Q_dstate_stride], hn, q[j]);
        }
#pragma unroll
        for (int j = 0; j < kMaxRank; ++j) q[j] *= dt;
        float y = 0.f;
        for (int n = 0; n < N; ++n) {
            const float bn = Bv ? to_f32(Bv[n * p.B_dstate_stride + t]) : Bc[n * p.B_dstate_stride];
            const float cn = Cv ? to_f32(Cv[n * p.C_dstate_stride + t]) : Cc[n * p.C_dstate_stride];
            float w = du * bn;
#pragma unroll
            for (int j = 0; j < kMaxRank; ++j)
                if (j < rank) w = __builtin_fmaf(Pd[n * p.P_dstate_stride + j * p.P_r_stride], q[j], w);
            const float a = decay_exp2(dt, Ad[n * p.A_dstate_stride] * kLog2e);
            const float hn = __builtin_fmaf(a, sH[n * kRowBlock + lane], w);
            sH[n * kRowBlock + lane] = hn;
            y = __builtin_fmaf(hn, cn, y);
        }
        if (active) {
            const float o = p.D ? __builtin_fmaf(Dv, uu, y) : y;
            if (op) op[t] = from_f32<T>(o);
            if (ozp) ozp[t] = from_f32<T>(o * silu_fast(to_f32(zp[t])));
            if (p.chunk_states && ((t + 1) % MM_SCAN_CHUNK == 0 || t == L - 1)) {
                float *cs = p.chunk_states + ((b * p.dim + d) * n_chunks + t / MM_SCAN_CHUNK) * 2 * N;
                for (int n = 0; n < N; ++n) {
                    cs[2 * n] = 1.f;
                    cs[2 * n + 1] = sH[n * kRowBlock + lane];
                }
            }
        }
    }
    if (active && p.last_state) {
        float *ls = p.last_state + (b * p.dim + d) * N;
        for (int n = 0; n < N; ++n) ls[n] = sH[n * kRowBlock + lane];
    }
}

// ------------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------------
struct TiledShape { int S, LPR; };

// The tiled kernel addresses u, delta, z, out and out_z with 32-bit byte offsets from the first of a
// wave's channel rows (up to 16), and B / C from the (batch, group) base: every offset must fit.
static bool offsets_ok(const mm_scan_fwd_params &p) {
    const int64_t eb = p.itype == MM_FLOAT32 ? 4 : 2;
    const int64_t ch = 15 * std::max({p.u_d_stride, p.delta_d_stride, p.z ? p.z_d_stride : int64_t(0),
                                      p.out ? p.out_d_stride : int64_t(0), p.out_z ? p.out_z_d_stride : int64_t(0)});
    const int64_t bc = (p.dstate - 1) * std::max(p.B_dstate_stride, p.C_dstate_stride);
    return (std::max(ch, bc) + p.seqlen) * eb < (int64_t(1) << 32);
}

// The (S, LPR) of the tiled kernel for this request, or {0, 0} when the request needs the general
// kernel: variable B and C, dstate <= 64, seqlen >= 8, rows movable as 16-byte vectors, offsets
// that fit in 32 bits.
TiledShape tiled_shape(const mm_scan_fwd_params &p) {
    if (!p.is_variable_B || !p.is_variable_C || p.dstate > 64 || p.seqlen < 8 || !fwd_vector_ok(&p) ||
        !offsets_ok(p))
        return {0, 0};
    const int64_t ratio = p.dim / p.n_groups;
    auto waves = [&](int lpr) { return p.batch * p.n_groups * ((ratio + 64 / lpr - 1) / (64 / lpr)); };
    const char *forced = getenv("MM_PQ_LPR");
    const int want = forced ? atoi(forced) : 0;
    TiledShape cands[3];
    int nc = 0;
    if (p.dstate <= 16) { cands[nc++] = {4, 4}; cands[nc++] = {2, 8}; cands[nc++] = {1, 16}; }
    else if (p.dstate <= 32) { cands[nc++] = {4, 8}; cands[nc++] = {2, 16}; }
    else { cands[nc++] = {4, 16}; }
    for (int i = 0; i < nc; ++i)
        if (cands[i].LPR == want) return cands[i];
    // Measured (fp16, rank 2, L 2048, 2,048-5,120 channels, batch 1-8, on 1,024 SIMDs). 16 lanes per
    // channel add a butterfly stage to every reduction: they win only while their waves fit one per
    // SIMD (dstate 16: 0.191 against 0.214 ms with 8 lanes; dstate 32: 0.244 against 0.31 ms with
    // 8 lanes of 4 states), and lose beyond (dstate 16: 0.58 against 0.30 ms at two waves of 8 lanes
    // per SIMD; dstate 32: 0.60 against 0.47 ms at 1.5). At dstate 16, 8 lanes of 2 states stay the
    // fastest up to 2.5 of their waves per SIMD (0.30 ms at two, 0.40 ms at 2.5 against 0.45 ms with
    // 4 lanes); past that the 4-lane layout's half as many waves win (0.45 against 0.55 ms at 3).
    const int64_t simds = device_simds();
    if (nc == 1) return cands[0];
    if (waves(16) <= simds) return cands[nc - 1];
    if (nc == 2) return cands[0];
    return 2 * waves(8) <= 5 * simds ? cands[1] : cands[0];
}

template <typename T, int S, int LPR, int R, bool DX = false>
int launch_tiled_sr(const mm_scan_fwd_params &p, hipStream_t s) {
    constexpr int CPW = 64 / LPR;
    const int64_t ratio = p.dim / p.n_groups;
    const int64_t bpg = (ratio + CPW - 1) / CPW;
    dim3 grid(unsigned(bpg * p.n_groups), unsigned(p.batch));
    hipLaunchKernelGGL((scan_fwd_pq_tiled<T, S, LPR, R, DX>), grid, dim3(64), 0, s, p, ratio, int32_t(bpg));
    return launch_status("scan_fwd_pq_tiled");
}

// diag_x: the zero-pair diagonal route, which has rank 1 and wants the diagonal chunk states.
template <typename T, int S, int LPR>
int launch_tiled_s(const mm_scan_fwd_params &p, hipStream_t s, bool diag_x) {
    if (diag_x) return launch_tiled_sr<T, S, LPR, 2, true>(p, s);
    if (p.pq_rank <= 2) return launch_tiled_sr<T, S, LPR, 2>(p, s);
    if (p.pq_rank <= 4) return launch_tiled_sr<T, S, LPR, 4>(p, s);
    return launch_tiled_sr<T, S, LPR, 8>(p, s);
}

template <typename T>
int launch_rowlane(const mm_scan_fwd_params &p, hipStream_t s) {
    dim3 grid(unsigned((p.dim + kRowBlock - 1) / kRowBlock), unsigned(p.batch));
    const size_t lds = size_t(p.dstate) * kRowBlock * sizeof(float);  // <= 64 KB at dstate 256
    hipLaunchKernelGGL((scan_fwd_pq_rowlane<T>), grid, dim3(kRowBlock), lds, s, p, p.dim / p.n_groups);
    return launch_status("scan_fwd_pq_rowlane");
}

}  // namespace pq

template <typename T>
int launch_pq(const mm_scan_fwd_params &p, hipStream_t s, bool diag_x) {
    const pq::TiledShape sh = pq::tiled_shape(p);
    if (sh.LPR == 4) return pq::launch_tiled_s<T, 4, 4>(p, s, diag_x);
    if (sh.LPR == 8)
        return sh.S == 4 ? pq::launch_tiled_s<T, 4, 8>(p, s, diag_x) : pq::launch_tiled_s<T, 2, 8>(p, s, diag_x);
    if (sh.LPR == 16) {
        if (sh.S == 4) return pq::launch_tiled_s<T, 4, 16>(p, s, diag_x);
        if (sh.S == 2) return pq::launch_tiled_s<T, 2, 16>(p, s, diag_x);
        return pq::launch_tiled_s<T, 1, 16>(p, s, diag_x);
    }
    return pq::launch_rowlane<T>(p, s);   // not reached with diag_x (diag_via_pq_fwd requires a tiled shape)
}

template int launch_pq<float>(const mm_scan_fwd_params &, hipStream_t, bool);
template int launch_pq<f16_t>(const mm_scan_fwd_params &, hipStream_t, bool);
template int launch_pq<bf16_t>(const mm_scan_fwd_params &, hipStream_t, bool);

// ------------------------------------------------------------------------------------------------
// The diagonal scan through the P/Q kernels. A zero rank-1 pair shared by every channel (P = Q = 0)
// leaves the coupled recurrence exactly the diagonal one: q = Q h = 0 and every coupling term is
// fma(0, q, w) = w. Diagonal requests the dstate-16 kernels do not take (dstate below 16, or 17 to
// 64, variable B and C) run several times faster this way than on the general kernels. The pair and
// the sink for its dP / dQ (written by the backward's atomics, never read) are static device arrays;
// their addresses are looked up once per device.
namespace {
__device__ __align__(16) float pq_zero_pair[64];   // zero-initialised, never written
__device__ __align__(16) float pq_grad_sink[64];   // receives the zero pair's gradients

constexpr int kMaxDev = 64;
std::atomic<float *> g_zero_ptr[kMaxDev], g_sink_ptr[kMaxDev];

int zero_pair_pointers(float **zero, float **sink) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return MM_ERR_UNSUPPORTED;
    float *z = g_zero_ptr[dev].load(std::memory_order_acquire);
    float *k = g_sink_ptr[dev].load(std::memory_order_acquire);
    if (z == nullptr || k == nullptr) {
        void *a = nullptr, *b = nullptr;
        if (hipGetSymbolAddress(&a, HIP_SYMBOL(pq_zero_pair)) != hipSuccess || a == nullptr) return MM_ERR_UNSUPPORTED;
        if (hipGetSymbolAddress(&b, HIP_SYMBOL(pq_grad_sink)) != hipSuccess || b == nullptr) return MM_ERR_UNSUPPORTED;
        z = static_cast<float *>(a);
        k = static_cast<float *>(b);
        g_zero_ptr[dev].store(z, std::memory_order_release);
        g_sink_ptr[dev].store(k, std::memory_order_release);
    }
    *zero = z;
    *sink = k;
    return MM_OK;
}

// MM_DIAG_VIA_PQ=0 keeps such requests on the general kernels (read per call, for the tests).
bool diag_pq_enabled() {
    const char *e = getenv("MM_DIAG_VIA_PQ");
    return !(e && e[0] == '0');
}
}  // namespace

bool diag_via_pq_fwd(const mm_scan_fwd_params &p) {
    // The tiled P/Q kernel then writes the chunk states in the diagonal form (DX), and the tile
    // states below dstate 16 (states past dstate stay 0), which the zero-pair backward reads.
    if (p.P || p.dstate == 16 || p.dstate > 64 || (p.tile_states && p.dstate > 16) || !diag_pq_enabled())
        return false;
    return pq::tiled_shape(p).LPR != 0;
}

int attach_zero_pair(mm_scan_fwd_params &q) {
    float *zero = nullptr, *sink = nullptr;
    const int rc = zero_pair_pointers(&zero, &sink);
    if (rc != MM_OK) return rc;
    q.P = zero;
    q.Q = zero;
    q.gamma = nullptr;
    q.pq_rank = 1;
    q.P_d_stride = 0; q.P_dstate_stride = 1; q.P_r_stride = 0;
    q.Q_d_stride = 0; q.Q_r_stride = 0; q.Q_dstate_stride = 1;
    return MM_OK;
}

bool diag_via_pq_bwd(const mm_scan_bwd_params &p) {
    if (p.P || p.dstate >= 16 || !diag_pq_enabled()) return false;
    mm_scan_bwd_params q = p;
    q.pq_rank = 1;
    return pq_bwd_ok(q);
}

int attach_zero_pair(mm_scan_bwd_params &q) {
    float *zero = nullptr, *sink = nullptr;
    const int rc = zero_pair_pointers(&zero, &sink);
    if (rc != MM_OK) return rc;
    q.P = zero;
    q.Q = zero;
    q.pq_rank = 1;
    q.P_d_stride = 0; q.P_dstate_stride = 1; q.P_r_stride = 0;
    q.Q_d_stride = 0; q.Q_r_stride = 0; q.Q_dstate_stride = 1;
    q.dP = sink;
    q.dQ = sink;
    q.dP_d_stride = 0; q.dP_dstate_stride = 1; q.dP_r_stride = 0;
    q.dQ_d_stride = 0; q.dQ_r_stride = 0; q.dQ_dstate_stride = 1;
    return MM_OK;
}

}  // namespace mm
