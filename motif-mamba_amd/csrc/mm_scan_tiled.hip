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
//
// The file is compiled three times, in parallel: on its own for fp32 inputs, where it also defines
// the shape queries (segment_count, segment_workspace_bytes, tile_states_ok), and through
// mm_scan_tiled_f16.hip / mm_scan_tiled_bf16.hip, which set MM_TILED_TYPE, for the 16-bit instances.
#ifndef MM_TILED_TYPE
#define MM_TILED_TYPE float
#define MM_TILED_COMMON
#endif
#include <hip/hip_runtime.h>

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
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

// bcast_row(src, LANE) * x as one v_mul_f32_dpp, fixed in the instruction stream (the compiler may
// otherwise split the broadcast into a v_mov_b32_dpp and fold the product elsewhere). Same source
// hazard rule as fmac_row_bcast.
template <int LANE>
__device__ __forceinline__ float mul_row_bcast(float src, float x) {
    float r;
    asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(src), "v"(x), "i"(LANE));
    return r;
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
                    av[j][k] = decay_exp2(dts[j], At[k]);
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

// ---------------------------------------------------------------------------------------------
// scan_fwd_pipe<K>: K states per lane, NW = 4 / K waves = 16 channels x 16 states per workgroup.
//
//   lane l of wave w:  row r = 4 w + l / 16 holding states r K .. r K + K-1,  channel c = l % 16
//
// The sequence is walked in 16-step tiles with two barriers per tile:
//
//   [A]  scan tile j: h_k = exp2(dt' A_k) h_k + B_k dt'u;  sum_k C_k h_k -> sY[r][c][t]
//   [B]  role group j % 2 (waves [g NW/2, (g+1) NW/2)) finishes tile j: y = sum of the 16/K row
//        partials, D u, silu(z) gate, store; the other group prepares tile j+1:
//        dt' = softplus(dt + bias), dt' u -> sDt/sDu[(j+1) % 2]
//
// so the per-element work of one tile overlaps the scan bookkeeping of the next and no wave idles
// between the barriers. Each group owns the elements of every other tile: its 32 NW lanes x E = 2K
// consecutive steps x 16 channels. B and C of a row's K states are held E steps per lane (LPS lanes
// per state) and broadcast along the row with DPP. Global loads (B/C for 32 steps, each lane's
// u/delta/z slice) run PF tile pairs ahead of use.
//
// K = 1 gives 5 waves on every SIMD for config 2 (1280 workgroups of 256 threads: 5 per CU), but
// 2 LDS floats read and 1 written per state update; K = 2 halves that traffic, which on gfx950 (LDS
// writes ~74 B/clk/CU) decides the rate, at the price of 2-3 waves per SIMD.
// ---------------------------------------------------------------------------------------------
constexpr int kT1 = 16;   // steps per tile

// LDS rows of 16 floats, one per channel (the delta' and delta' u of a tile) or per (state row,
// channel) (the row partials of y), are stored as four 4-float blocks, block q of channel c at
// position q ^ swz16(c). The scan accesses them with one lane per channel (c = lane % 16) in
// 128-bit loads and stores, which the LDS serves 8 lanes per cycle over 32 banks: among the lanes
// c = 8m .. 8m + 7, c % 2 selects the half of the banks and swz16 takes all four values for either
// parity, so the 8 lanes hit every bank once. On a 64-bank LDS (16 lanes per cycle) the same holds
// with c % 4 selecting the quarter and swz16 a bijection of c / 4. The per-element lanes read and
// write whole rows of adjacent channels, which the permutation inside a row does not change.
__device__ __forceinline__ int swz16(int c) { return (((c >> 1) ^ (c >> 3)) & 1) | ((c >> 1) & 2); }

template <typename T, int K>
struct PairData {                  // one lane's global data for one 32-step tile pair
    RawVec<T, 2 * K> b, c;         // B, C of one of the row's states, 2K steps
    RawVec<T, 2 * K> u, dl, z;     // u, delta, z of the lane's element slice in its group's tile
};

// Sequence segments of one launch (blockIdx.z = segment): MODE 0 scans whole rows; MODE 1 scans
// segments 0 .. n_seg-2 from a zero state and writes only their end state (h) and the sum of
// delta' (sumdt); MODE 2 scans every segment from the carried state h[segment] with the delta'
// prefix cum[segment] and writes all outputs (last_state from the last segment). MODE 3 scans
// whole rows for the states alone and writes only p.tile_states (the backward's checkpoints).
struct SegArgs {
    int64_t pairs;   // 32-step tile pairs per segment
    int32_t n_seg;
    float *h;        // (batch * dim, n_seg, 16)
    float *sumdt;    // (batch * dim, n_seg)
    float *cum;      // (batch * dim, n_seg)
};

template <typename T, int K, int PF, bool SOFTPLUS, bool CHUNKS, int MODE>
__global__ void __launch_bounds__(256 / K) __attribute__((amdgpu_waves_per_eu(5 - 2 * (K - 1), 8)))
scan_fwd_pipe(const mm_scan_fwd_params p, const int64_t ratio, const SegArgs sg) {
    constexpr int NW = 4 / K;              // waves per workgroup
    constexpr int NR = 16 / K;             // rows per workgroup
    constexpr int E = 2 * K;               // element steps per lane per tile (and B/C steps per lane per pair)
    constexpr int LPS = 16 / K;            // lanes of a row holding one state's B/C
    constexpr int GL = 32 * NW;            // lanes per role group
    __shared__ __align__(16) float sDt[2][kCh * kT1];
    __shared__ __align__(16) float sDu[2][kCh * kT1];
    // Row partials of y [row][channel][16 steps], 4-float blocks permuted by swz16(channel).
    __shared__ __align__(16) float sY[NR * kCh * kT1];

    const int lane = threadIdx.x & 63;
    const int r = threadIdx.x >> 4;        // row of this lane in the scan
    const int c = lane & 15;               // channel of this lane in the scan
    const int grp = int(threadIdx.x) / GL; // role group (wave-uniform)
    const int gl = int(threadIdx.x) % GL;
    const int ce = gl / (16 / E);          // channel of this lane's element slice
    const int es = E * (gl % (16 / E));    // first step (within a tile) of the slice
    const int swc = swz16(c), swe = swz16(ce);   // LDS block permutations of the two channels
    const int64_t b = blockIdx.y;
    const int64_t d0 = int64_t(blockIdx.x) * kCh;
    const int64_t g = d0 / ratio;
    const int64_t L = p.seqlen;
    const int64_t n_pairs = (L + 2 * kT1 - 1) / (2 * kT1);
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    constexpr bool WHOLE = MODE == 0 || MODE == 3;   // whole rows, no segments
    constexpr bool YP = MODE == 0 || MODE == 2;      // y partials and outputs
    const int seg = WHOLE ? 0 : int(blockIdx.z);
    const int64_t pb = WHOLE ? 0 : seg * sg.pairs;                                          // first pair
    const int64_t pe = WHOLE ? n_pairs : (pb + sg.pairs < n_pairs ? pb + sg.pairs : n_pairs);  // end
    const int64_t srow = (b * p.dim + d0 + c) * int64_t(sg.n_seg) + seg;                   // segment slot

    const int64_t de = d0 + ce;
    // Uniform row-group bases (scalar registers) plus 32-bit per-lane element offsets; the host
    // checks that every offset of the group fits in 31 bits.
    const T *ub = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d0 * p.u_d_stride;
    const T *db = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d0 * p.delta_d_stride;
    const T *zb = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d0 * p.z_d_stride : nullptr;
    T *ob = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d0 * p.out_d_stride : nullptr;
    T *ozb = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d0 * p.out_z_d_stride : nullptr;
    const T *Bb = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cb = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;
    const uint32_t u_row = uint32_t(ce * p.u_d_stride), d_row = uint32_t(ce * p.delta_d_stride);
    const uint32_t z_row = uint32_t(ce * p.z_d_stride), o_row = uint32_t(ce * p.out_d_stride);
    const uint32_t oz_row = uint32_t(ce * p.out_z_d_stride);
    const int nl = r * K + c / LPS;        // the state whose B/C this lane loads
    const uint32_t B_row = uint32_t(nl * p.B_dstate_stride), C_row = uint32_t(nl * p.C_dstate_stride);
    const int sb = E * (c % LPS);          // first step (within a pair) of this lane's B/C slice

    float At[K], h[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        At[k] = p.A[(d0 + c) * p.A_d_stride + int64_t(r * K + k) * p.A_dstate_stride] * kLog2e;
        h[k] = MODE == 2 ? sg.h[srow * 16 + r * K + k] : 0.f;
    }
    const float Dv = p.D ? p.D[de] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[de] : 0.f;
    float cum_dt = (MODE == 2 && CHUNKS) ? sg.cum[srow] : 0.f;

    // Global loads of tile pair i; positions at or past the end of a row are clamped into the
    // row's last E elements (L >= 8, L % 8 == 0), the prologue zeroes delta' of such steps.
    const uint32_t lastE = uint32_t(L - E);
    auto clampE = [&](int64_t t) { return t < int64_t(lastE) ? uint32_t(t) : lastE; };
    auto load_pair = [&](int64_t i, PairData<T, K> &dst) {
        const int64_t t0 = i * (2 * kT1);
        const uint32_t tb = clampE(t0 + sb);
        dst.b = load_raw<T, E>(Bb + (B_row + tb));
        const uint32_t te = clampE(t0 + kT1 * grp + es);
        dst.u = load_raw<T, E>(ub + (u_row + te));
        dst.dl = load_raw<T, E>(db + (d_row + te));
        dst.c = {};
        dst.z = {};
        if constexpr (YP) {                // C and z feed only the outputs
            dst.c = load_raw<T, E>(Cb + (C_row + tb));
            if (zb) dst.z = load_raw<T, E>(zb + (z_row + te));
        }
    };

    // Prologue of the tile starting at t0 (this lane's slice): delta', delta' u -> LDS buffer buf.
    float uu[E], zz[E];
    auto prologue = [&](const PairData<T, K> &src, int64_t t0, int buf) {
        float dd[E], dtp[E], dup[E];
        unpack_raw<T, E>(src.u, uu);
        unpack_raw<T, E>(src.dl, dd);
        if constexpr (YP) unpack_raw<T, E>(src.z, zz);
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float x = dd[k] + bias;
            dtp[k] = SOFTPLUS ? softplus_fast(x) : x;
        }
        if (t0 + es >= L) {  // padded steps of a last, partial tile (L % 8 == 0: all E or none)
#pragma unroll
            for (int k = 0; k < E; ++k) dtp[k] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < E; ++k) dup[k] = dtp[k] * uu[k];
#pragma unroll
        for (int k = 0; k < E; k += 2) {
            const int col = ((((es + k) >> 2) ^ swe) << 2) + ((es + k) & 3);
            *reinterpret_cast<float2 *>(&sDt[buf][ce * kT1 + col]) = make_float2(dtp[k], dtp[k + 1]);
            *reinterpret_cast<float2 *>(&sDu[buf][ce * kT1 + col]) = make_float2(dup[k], dup[k + 1]);
        }
    };

    // Epilogue of the tile starting at t0 (this lane's slice): rows added in a fixed order.
    auto epilogue = [&](int64_t t0) {
        if constexpr (!YP) return;  // state-only scans produce no outputs
        const int ecol = (((es >> 2) ^ swe) << 2) + (es & 3);
        float y[E];
        if constexpr (E == 4) {
            float4 a = *reinterpret_cast<const float4 *>(&sY[ce * kT1 + ecol]);
#pragma unroll
            for (int rr = 1; rr < NR; ++rr) {
                const float4 v = *reinterpret_cast<const float4 *>(&sY[(rr * kCh + ce) * kT1 + ecol]);
                a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
            }
            y[0] = a.x; y[1] = a.y; y[2] = a.z; y[3] = a.w;
        } else {
            float2 a = *reinterpret_cast<const float2 *>(&sY[ce * kT1 + ecol]);
#pragma unroll
            for (int rr = 1; rr < NR; ++rr) {
                const float2 v = *reinterpret_cast<const float2 *>(&sY[(rr * kCh + ce) * kT1 + ecol]);
                a.x += v.x; a.y += v.y;
            }
            y[0] = a.x; y[1] = a.y;
        }
        if (t0 + es < L) {
            float o[E];
#pragma unroll
            for (int k = 0; k < E; ++k) o[k] = __builtin_fmaf(Dv, uu[k], y[k]);
            const uint32_t t = uint32_t(t0 + es);
            if (ob) store_vec<T, E>(ob + (o_row + t), o);
            if (zb) {
#pragma unroll
                for (int k = 0; k < E; ++k) o[k] *= silu_fast(zz[k]);
                store_vec<T, E>(ozb + (oz_row + t), o);
            }
        }
    };

    // Scan of one 16-step tile from LDS buffer buf. B/C of state r K + k at step t of the pair
    // half H sit in lane k LPS + (16 H + t) / E of this row, register (16 H + t) % E.
    float bv[E], cv[E];
    auto scan_tile = [&](auto Hc, int64_t t0, int buf) {
        constexpr int H = decltype(Hc)::value;
        // The tile's dt' and dt'u: with outputs all read before the scan starts (the y-partial
        // stores between the 4-step groups would otherwise hold each group's reads back until it
        // is needed); without them, where registers are short, one group at a time.
        float4 dtg[kT1 / 4], dug[kT1 / 4];
        auto read_group = [&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            dtg[s4] = *reinterpret_cast<const float4 *>(&sDt[buf][c * kT1 + ((s4 ^ swc) << 2)]);
            dug[s4] = *reinterpret_cast<const float4 *>(&sDu[buf][c * kT1 + ((s4 ^ swc) << 2)]);
        };
        if constexpr (YP) static_for<0, kT1 / 4>(read_group);
        static_for<0, kT1 / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            if constexpr (!YP) read_group(S4);
            const float dts[4] = {dtg[s4].x, dtg[s4].y, dtg[s4].z, dtg[s4].w};
            const float dus[4] = {dug[s4].x, dug[s4].y, dug[s4].z, dug[s4].w};
            float av[4][K], bbv[4][K], pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                if (CHUNKS || MODE == 1) cum_dt += dts[j];
                static_for<0, K>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    constexpr int src = k * LPS + s / E;
                    av[j][k] = decay_exp2(dts[j], At[k]);
                    bbv[j][k] = mul_row_bcast<src>(bv[s % E], dus[j]);
                });
            });
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                float acc;
                static_for<0, K>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    constexpr int src = k * LPS + s / E;
                    h[k] = __builtin_fmaf(av[j][k], h[k], bbv[j][k]);
                    if constexpr (YP) {
                        if constexpr (k == 0)
                            acc = row_bcast<src>(cv[s % E]) * h[k];
                        else
                            fmac_row_bcast<src>(acc, cv[s % E], h[k]);
                    }
                });
                if constexpr (YP) pv[j] = acc;
            });
            if constexpr (YP)
                *reinterpret_cast<float4 *>(&sY[(r * kCh + c) * kT1 + ((s4 ^ swc) << 2)]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
            // Without the y-partial chain the scheduler would hoist the exponentials of a whole tile
            // and run out of registers: keep the state-only scan in 4-step groups.
            if constexpr (!YP) __builtin_amdgcn_sched_barrier(0);
        });
        if (YP && CHUNKS && p.chunk_states) {
            const int64_t tend = t0 + kT1 < L ? t0 + kT1 : L;
            if (t0 < L && (tend % MM_SCAN_CHUNK == 0 || tend == L)) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *csp = p.chunk_states + ((b * p.dim + d0 + c) * n_chunks + ci) * 32 + 2 * K * r;
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    csp[2 * k] = __builtin_amdgcn_exp2f(At[k] * cum_dt);
                    csp[2 * k + 1] = h[k];
                }
            }
        }
        // The state after this tile = the checkpoint before the next one, for the backward (training
        // forwards only: those write chunk states; the inference variants carry no such code).
        if (((MODE == 0 && CHUNKS) || MODE == 3) && p.tile_states && t0 + kT1 < L) {
            float *ck = p.tile_states + ((t0 / kT1 + 1) * p.batch * p.dim + b * p.dim + d0 + c) * 16 + r * K;
#pragma unroll
            for (int k = 0; k < K; ++k) ck[k] = h[k];
        }
    };

    if (((MODE == 0 && CHUNKS) || MODE == 3) && p.tile_states) {   // the checkpoint before the first tile: zero
#pragma unroll
        for (int k = 0; k < K; ++k) p.tile_states[(b * p.dim + d0 + c) * 16 + r * K + k] = 0.f;
    }
    PairData<T, K> ring[PF];
#pragma unroll
    for (int s = 0; s < PF; ++s) load_pair(pb + s, ring[s]);
    if (grp == 0) prologue(ring[0], pb * (2 * kT1), 0);

    for (int64_t i0 = pb; i0 < pe; i0 += PF) {
        static_for<0, PF>([&](auto Sc) {
            constexpr int S = decltype(Sc)::value;
            const int64_t i = i0 + S;
            if (i < pe) {
                const int64_t t0 = i * (2 * kT1);
                unpack_raw<T, E>(ring[S].b, bv);
                // Two wait states between the VALU writes of the DPP sources and their first DPP
                // read by the fmac inline asm (the compiler covers its own DPP instructions).
                if constexpr (YP) {
                    unpack_raw<T, E>(ring[S].c, cv);
#pragma unroll
                    for (int k = 0; k < E; ++k) asm volatile("s_nop 1" : "+v"(bv[k]), "+v"(cv[k]));
                } else {
#pragma unroll
                    for (int k = 0; k < E; ++k) asm volatile("s_nop 1" : "+v"(bv[k]));
                }
                PairData<T, K> mine = ring[S];  // group 1's slice of this pair (used below)
                load_pair(i + PF, ring[S]);
                // Tile 2i: group 0 finishes it, group 1 prepares tile 2i+1.
                __syncthreads();
                scan_tile(std::integral_constant<int, 0>{}, t0, 0);
                __syncthreads();
                if (grp == 0) epilogue(t0);
                else prologue(mine, t0 + kT1, 1);
                // Tile 2i+1: group 1 finishes it, group 0 prepares tile 2i+2.
                __syncthreads();
                scan_tile(std::integral_constant<int, 1>{}, t0 + kT1, 1);
                __syncthreads();
                if (grp == 1) epilogue(t0 + kT1);
                else prologue(ring[(S + 1) % PF], t0 + 2 * kT1, 0);
            }
        });
    }
    if constexpr (MODE == 1) {
#pragma unroll
        for (int k = 0; k < K; ++k) sg.h[srow * 16 + r * K + k] = h[k];
        if (r == 0) sg.sumdt[srow] = cum_dt;
    } else if constexpr (MODE != 3) {
        if (p.last_state && (MODE == 0 || seg == sg.n_seg - 1)) {
#pragma unroll
            for (int k = 0; k < K; ++k) p.last_state[(b * p.dim + d0 + c) * 16 + r * K + k] = h[k];
        }
    }
}

// Carries between segments, one thread per (batch, channel, state): the start state of segment s+1
// is exp2(A log2e sum(delta' of s)) * start(s) + end_from_zero(s); written in place over h, with
// the delta' prefix of every segment in cum.
// (static: each of the file's three translation units holds its own copy.)
static __global__ void __launch_bounds__(256)
seg_carry_kernel(const float *A, int64_t A_d_stride, int64_t A_dstate_stride, int64_t rows, int64_t dim,
                 const SegArgs sg) {
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (tid >= rows * 16) return;
    const int64_t row = tid >> 4;
    const int n = int(tid & 15);
    const int64_t d = row % dim;
    const float A2 = A[d * A_d_stride + n * A_dstate_stride] * kLog2e;
    float H = 0.f, cd = 0.f;
    for (int s = 0; s < sg.n_seg; ++s) {
        float *hp = sg.h + (row * sg.n_seg + s) * 16 + n;
        const bool last = s == sg.n_seg - 1;
        const float he = last ? 0.f : *hp;
        const float sd = last ? 0.f : sg.sumdt[row * sg.n_seg + s];
        *hp = H;
        if (n == 0) sg.cum[row * sg.n_seg + s] = cd;
        H = __builtin_fmaf(__builtin_amdgcn_exp2f(A2 * sd), H, he);
        cd += sd;
    }
}

template <typename T, int K, int PF, int MODE>
int launch_pipe_mode(const mm_scan_fwd_params &p, hipStream_t stream, const SegArgs &sg, unsigned nz) {
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / kCh), unsigned(p.batch), nz);
    auto *kern = p.delta_softplus
                     ? (p.chunk_states ? scan_fwd_pipe<T, K, PF, true, true, MODE> : scan_fwd_pipe<T, K, PF, true, false, MODE>)
                     : (p.chunk_states ? scan_fwd_pipe<T, K, PF, false, true, MODE> : scan_fwd_pipe<T, K, PF, false, false, MODE>);
    hipLaunchKernelGGL(kern, grid, dim3(256 / K), 0, stream, p, ratio, sg);
    return launch_status("scan_fwd_pipe");
}

template <typename T, int K, int PF>
int launch_pipe(const mm_scan_fwd_params &p, hipStream_t stream) {
    return launch_pipe_mode<T, K, PF, 0>(p, stream, SegArgs{0, 1, nullptr, nullptr, nullptr}, 1);
}

// The backward's checkpoints alone (MODE 3): the state before every 16-step tile into
// p.tile_states, nothing else written.
template <typename T>
int launch_fwd_states(const mm_scan_fwd_params &p, hipStream_t stream) {
    return launch_pipe_mode<T, 2, 2, 3>(p, stream, SegArgs{0, 1, nullptr, nullptr, nullptr}, 1);
}

// Segmented scan: state-only pass over segments 0 .. n_seg-2, carry chain, full pass.
template <typename T>
int launch_pipe_segmented(const mm_scan_fwd_params &p, hipStream_t stream, const SegArgs &sg) {
    int rc = launch_pipe_mode<T, 2, 2, 1>(p, stream, sg, unsigned(sg.n_seg - 1));
    if (rc != MM_OK) return rc;
    const int64_t rows = p.batch * p.dim;
    hipLaunchKernelGGL(seg_carry_kernel, dim3(unsigned((rows * 16 + 255) / 256)), dim3(256), 0, stream, p.A,
                       p.A_d_stride, p.A_dstate_stride, rows, p.dim, sg);
    rc = launch_status("seg_carry");
    if (rc != MM_OK) return rc;
    return launch_pipe_mode<T, 2, 2, 2>(p, stream, sg, unsigned(sg.n_seg));
}

// ---------------------------------------------------------------------------------------------
// scan_fwd_k2i: two states per lane, two waves = 16 channels x 16 states per workgroup, and one
// barrier per 16-step tile, the per-element work interleaved with the scan:
//
//   interval j:  both waves scan tile j           (dt', dt'u from sDt/sDu[j % 4] -> row partials sY[j % 2])
//                wave j % 2 prepares tile j + 2   (softplus(dt + bias), dt' u -> sDt/sDu[(j + 2) % 4])
//                wave (j+1) % 2 finishes tile j-1 (sum of the 8 row partials in sY[(j - 1) % 2], D u,
//                                                  silu(z) gate, store)
//                barrier
//
// Tile t belongs to wave t % 2: each of its 64 lanes owns 4 consecutive steps of one channel, loads
// them, prepares them two intervals before the scan and finishes them one interval after it, keeping
// u and z in registers in between. Both waves do the same work in every interval, and the
// prologue/epilogue instructions sit in the same basic block as the scan, so they fill its latency
// gaps instead of forming a latency-bound phase of their own.
//
// FULL (L a multiple of 32, every tile pair whole): the only clamp left is of the pair index, which
// is uniform, so every load and store is a buffer instruction whose address is a per-tensor
// resource (scalar), a byte offset fixed per lane (VGPR) and the pair's byte offset (SGPR) -- no
// per-lane address arithmetic, compares or selects in the loop (they were about a sixth of its
// VALU instructions).
// ---------------------------------------------------------------------------------------------
template <typename T>
struct K2Data {                 // one lane's global data for pair iteration i
    RawVec<T, 4> b, c;          // B, C of one of the lane's row states: 4 steps of tile pair i
    RawVec<T, 4> u, dl, z;      // u, delta, z: 4 steps of this wave's tile of pair i + 1
};

template <typename T, int PF, bool SOFTPLUS, bool CHUNKS, bool FULL>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(3, 8)))
scan_fwd_k2i(const mm_scan_fwd_params p, const int64_t ratio) {
    static_assert(PF % 2 == 0, "the pair loop is unrolled by PF and needs a static parity");
    constexpr int E = 4, LPS = 8, NR = 8;
    __shared__ __align__(16) float sDt0[kCh * kT1], sDt1[kCh * kT1], sDt2[kCh * kT1], sDt3[kCh * kT1];
    __shared__ __align__(16) float sDu0[kCh * kT1], sDu1[kCh * kT1], sDu2[kCh * kT1], sDu3[kCh * kT1];
    // Row partials of y [row][channel][16 steps], 4-float blocks permuted by swz16(channel).
    __shared__ __align__(16) float sY0[NR * kCh * kT1], sY1[NR * kCh * kT1];
    auto DT = [&](auto I) -> float * {
        constexpr int i = decltype(I)::value & 3;
        if constexpr (i == 0) return sDt0; else if constexpr (i == 1) return sDt1;
        else if constexpr (i == 2) return sDt2; else return sDt3;
    };
    auto DU = [&](auto I) -> float * {
        constexpr int i = decltype(I)::value & 3;
        if constexpr (i == 0) return sDu0; else if constexpr (i == 1) return sDu1;
        else if constexpr (i == 2) return sDu2; else return sDu3;
    };
    auto YB = [&](auto I) -> float * {
        if constexpr ((decltype(I)::value & 1) == 0) return sY0; else return sY1;
    };

    const int w = threadIdx.x >> 6;        // wave: owns tiles t with t % 2 == w
    const int lane = threadIdx.x & 63;
    const int r = threadIdx.x >> 4;        // row (states 2r, 2r+1) of this lane in the scan
    const int c = lane & 15;               // channel of this lane in the scan
    const int ce = lane >> 2;              // channel of this lane's element slice
    const int es = E * (lane & 3);         // first step (within a tile) of the slice
    const int swc = swz16(c), swe = swz16(ce);   // LDS block permutations of the two channels
    const int64_t b = blockIdx.y;
    const int64_t d0 = int64_t(blockIdx.x) * kCh;
    const int64_t g = d0 / ratio;
    const int64_t L = p.seqlen;
    const int64_t n_pairs = (L + 2 * kT1 - 1) / (2 * kT1);
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;

    const int64_t de = d0 + ce;
    // Uniform row-group bases (scalar registers) plus 32-bit per-lane element offsets; the host
    // checks that every offset of the group fits in 31 bits.
    const T *ub = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d0 * p.u_d_stride;
    const T *db = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d0 * p.delta_d_stride;
    const T *zb = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d0 * p.z_d_stride : nullptr;
    T *ob = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d0 * p.out_d_stride : nullptr;
    T *ozb = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d0 * p.out_z_d_stride : nullptr;
    const T *Bb = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cb = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;
    const uint32_t u_row = uint32_t(ce * p.u_d_stride), d_row = uint32_t(ce * p.delta_d_stride);
    const uint32_t z_row = uint32_t(ce * p.z_d_stride), o_row = uint32_t(ce * p.out_d_stride);
    const uint32_t oz_row = uint32_t(ce * p.out_z_d_stride);
    const int nl = 2 * r + c / LPS;        // the state whose B/C this lane loads
    const uint32_t B_row = uint32_t(nl * p.B_dstate_stride), C_row = uint32_t(nl * p.C_dstate_stride);
    const int sb = E * (c % LPS);          // first step (within a pair) of this lane's B/C slice

    float At[2], h[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        At[k] = p.A[(d0 + c) * p.A_d_stride + int64_t(2 * r + k) * p.A_dstate_stride] * kLog2e;
        h[k] = 0.f;
    }
    const float Dv = p.D ? p.D[de] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[de] : 0.f;
    float cum_dt = 0.f;

    // Positions at or past the end of a row are clamped into the row's last 4 elements (L >= 8,
    // L % 8 == 0); the prologue zeroes delta' of such steps, so they leave the state unchanged.
    const uint32_t last4 = uint32_t(L - E);
    auto clamp4 = [&](int64_t t) { return t < int64_t(last4) ? uint32_t(t) : last4; };
    // FULL: buffer resources of the group's rows (the host checks that every byte offset of the
    // group is below 2^32) and this lane's byte offsets from them.
    constexpr uint32_t SZ = sizeof(T);
    const uint32_t fo_u = (u_row + kT1 * w + es) * SZ, fo_d = (d_row + kT1 * w + es) * SZ;
    const uint32_t fo_z = (z_row + kT1 * w + es) * SZ;
    const uint32_t fo_b = (B_row + sb) * SZ, fo_c = (C_row + sb) * SZ;
    const uint32_t fo_o = (o_row + es) * SZ, fo_oz = (oz_row + es) * SZ;
    const __amdgpu_buffer_rsrc_t rs_u = buffer_rsrc(ub), rs_d = buffer_rsrc(db), rs_z = buffer_rsrc(zb);
    const __amdgpu_buffer_rsrc_t rs_b = buffer_rsrc(Bb), rs_c = buffer_rsrc(Cb);
    const __amdgpu_buffer_rsrc_t rs_o = buffer_rsrc(ob), rs_oz = buffer_rsrc(ozb);
    auto load_elems = [&](int64_t pair_i, RawVec<T, E> &u, RawVec<T, E> &dl, RawVec<T, E> &z) {
        if constexpr (FULL) {
            const uint32_t sof = uint32_t((pair_i < n_pairs ? pair_i : n_pairs - 1) * (2 * kT1 * SZ));   // uniform
            u = buffer_load_raw<T, E>(rs_u, fo_u, sof);
            dl = buffer_load_raw<T, E>(rs_d, fo_d, sof);
            if (zb) z = buffer_load_raw<T, E>(rs_z, fo_z, sof);
            else z = {};
        } else {
            const uint32_t te = clamp4(pair_i * (2 * kT1) + kT1 * w + es);
            u = load_raw<T, E>(ub + (u_row + te));
            dl = load_raw<T, E>(db + (d_row + te));
            if (zb) z = load_raw<T, E>(zb + (z_row + te));
            else z = {};
        }
    };
    auto load_data = [&](int64_t i, K2Data<T> &dst) {
        if constexpr (FULL) {
            const uint32_t sof = uint32_t((i < n_pairs ? i : n_pairs - 1) * (2 * kT1 * SZ));              // uniform
            dst.b = buffer_load_raw<T, E>(rs_b, fo_b, sof);
            dst.c = buffer_load_raw<T, E>(rs_c, fo_c, sof);
        } else {
            const uint32_t tb = clamp4(i * (2 * kT1) + sb);
            dst.b = load_raw<T, E>(Bb + (B_row + tb));
            dst.c = load_raw<T, E>(Cb + (C_row + tb));
        }
        load_elems(i + 1, dst.u, dst.dl, dst.z);
    };

    // This lane's u and z of the two tiles it owns that are in flight: tile t uses slot (t / 2) % 2
    // (wave 0: tile 2i+2 is prepared into slot 1-P while tile 2i, slot P, waits for its epilogue;
    // wave 1: tile 2i-1 is finished from slot 1-P, then tile 2i+3 is prepared into it).
    float uu[2][E], zz[2][E];

    // Prologue of tile t0 / 16 (this lane's slice): delta', delta' u -> dt/du, u and z -> slot.
    auto prologue = [&](const RawVec<T, E> &ru, const RawVec<T, E> &rd, const RawVec<T, E> &rz, int64_t t0,
                        float *dt, float *du, auto Slot) {
        constexpr int sl = decltype(Slot)::value;
        float dd[E], dtp[E];
        unpack_raw<T, E>(ru, uu[sl]);
        unpack_raw<T, E>(rd, dd);
        unpack_raw<T, E>(rz, zz[sl]);
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float x = dd[k] + bias;
            dtp[k] = SOFTPLUS ? softplus_fast(x) : x;
        }
        // Padded steps (L % 8 == 0: all four or none). With FULL only tiles past the last pair are
        // prepared beyond L, and those are never scanned.
        if (!FULL && t0 + es >= L) {
#pragma unroll
            for (int k = 0; k < E; ++k) dtp[k] = 0.f;
        }
        *reinterpret_cast<float4 *>(&dt[ce * kT1 + (((es >> 2) ^ swe) << 2)]) = make_float4(dtp[0], dtp[1], dtp[2], dtp[3]);
        *reinterpret_cast<float4 *>(&du[ce * kT1 + (((es >> 2) ^ swe) << 2)]) =
            make_float4(dtp[0] * uu[sl][0], dtp[1] * uu[sl][1], dtp[2] * uu[sl][2], dtp[3] * uu[sl][3]);
    };

    // Epilogue of tile t0 / 16 (this lane's slice): the 8 row partials added in row order.
    auto epilogue = [&](int64_t t0, const float *yb, auto Slot) {
        constexpr int sl = decltype(Slot)::value;
        const int ecol = ((es >> 2) ^ swe) << 2;
        float4 a = *reinterpret_cast<const float4 *>(&yb[ce * kT1 + ecol]);
#pragma unroll
        for (int rr = 1; rr < NR; ++rr) {
            const float4 v = *reinterpret_cast<const float4 *>(&yb[(rr * kCh + ce) * kT1 + ecol]);
            a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
        }
        if (FULL || t0 + es < L) {   // FULL: only whole tiles are finished
            float o[E] = {__builtin_fmaf(Dv, uu[sl][0], a.x), __builtin_fmaf(Dv, uu[sl][1], a.y),
                          __builtin_fmaf(Dv, uu[sl][2], a.z), __builtin_fmaf(Dv, uu[sl][3], a.w)};
            const uint32_t t = uint32_t(t0 + es);
            if (ob) {
                if constexpr (FULL) buffer_store_vec<T, E>(rs_o, fo_o, uint32_t(t0 * SZ), o);
                else store_vec<T, E>(ob + (o_row + t), o);
            }
            if (zb) {
#pragma unroll
                for (int k = 0; k < E; ++k) o[k] *= silu_fast(zz[sl][k]);
                if constexpr (FULL) buffer_store_vec<T, E>(rs_oz, fo_oz, uint32_t(t0 * SZ), o);
                else store_vec<T, E>(ozb + (oz_row + t), o);
            }
        }
    };

    // Scan of one tile (pair half H) from dt/du into the row partials yb. B/C of state 2r + k at
    // step s of the pair sit in lane 8k + s / 4 of this row, register s % 4.
    // The tile's dt' / dt'u are read from LDS one 4-step group ahead of their use: groups 1-3 while
    // the group before computes, and group 0 of the next tile (dtn / dun, prepared two intervals
    // earlier and published by the last barrier) at the end of this one, so that its LDS latency
    // passes during the epilogue / prologue work and the barrier instead of stalling the next scan.
    float bv[E], cv[E];
    float4 pre_dt, pre_du;                 // group 0 of the tile about to be scanned
    auto scan_tile = [&](auto Hc, int64_t t0, const float *dt, const float *du, float *yb, const float *dtn,
                         const float *dun) {
        constexpr int H = decltype(Hc)::value;
        float4 dtq = pre_dt, duq = pre_du;
        static_for<0, kT1 / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            float4 ndt, ndu;
            if constexpr (s4 + 1 < kT1 / 4) {
                ndt = *reinterpret_cast<const float4 *>(&dt[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&du[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
            } else {
                ndt = *reinterpret_cast<const float4 *>(&dtn[c * kT1 + (swc << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&dun[c * kT1 + (swc << 2)]);
            }
            const float dts[4] = {dtq.x, dtq.y, dtq.z, dtq.w};
            const float dus[4] = {duq.x, duq.y, duq.z, duq.w};
            float av[4][2], bbv[4][2], pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                if (CHUNKS) cum_dt += dts[j];
                static_for<0, 2>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    av[j][k] = decay_exp2(dts[j], At[k]);
                    bbv[j][k] = row_bcast<k * LPS + s / E>(bv[s % E]) * dus[j];
                });
            });
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                h[0] = __builtin_fmaf(av[j][0], h[0], bbv[j][0]);
                h[1] = __builtin_fmaf(av[j][1], h[1], bbv[j][1]);
                float acc = row_bcast<s / E>(cv[s % E]) * h[0];
                fmac_row_bcast<LPS + s / E>(acc, cv[s % E], h[1]);
                pv[j] = acc;
            });
            *reinterpret_cast<float4 *>(&yb[(r * kCh + c) * kT1 + ((s4 ^ swc) << 2)]) =
                make_float4(pv[0], pv[1], pv[2], pv[3]);
            dtq = ndt;
            duq = ndu;
        });
        pre_dt = dtq;
        pre_du = duq;
        if (CHUNKS && p.chunk_states) {
            const int64_t tend = t0 + kT1 < L ? t0 + kT1 : L;
            if (t0 < L && (tend % MM_SCAN_CHUNK == 0 || tend == L)) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *csp = p.chunk_states + ((b * p.dim + d0 + c) * n_chunks + ci) * 32 + 4 * r;
                csp[0] = __builtin_amdgcn_exp2f(At[0] * cum_dt);
                csp[1] = h[0];
                csp[2] = __builtin_amdgcn_exp2f(At[1] * cum_dt);
                csp[3] = h[1];
            }
        }
        // The state after this tile = the checkpoint before the next one, for the backward (training
        // forwards only: those write chunk states; the inference variants carry no such code).
        if (CHUNKS && p.tile_states && t0 + kT1 < L) {
            float *ck = p.tile_states + ((t0 / kT1 + 1) * p.batch * p.dim + b * p.dim + d0 + c) * 16 + 2 * r;
            *reinterpret_cast<float2 *>(ck) = make_float2(h[0], h[1]);
        }
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if (CHUNKS && p.tile_states)           // the checkpoint before the first tile: zero
        *reinterpret_cast<float2 *>(p.tile_states + (b * p.dim + d0 + c) * 16 + 2 * r) = make_float2(0.f, 0.f);
    K2Data<T> ring[PF];
    {
        RawVec<T, E> u0, d0v, z0;
        load_elems(0, u0, d0v, z0);
#pragma unroll
        for (int s = 0; s < PF; ++s) load_data(s, ring[s]);
        // Tiles 0 and 1 are prepared before the first interval (slot 0 for both waves).
        if (w == 0) prologue(u0, d0v, z0, 0, DT(I0{}), DU(I0{}), I0{});
        else prologue(u0, d0v, z0, kT1, DT(I1{}), DU(I1{}), I0{});
    }
    __syncthreads();
    pre_dt = *reinterpret_cast<const float4 *>(&DT(I0{})[c * kT1 + (swc << 2)]);
    pre_du = *reinterpret_cast<const float4 *>(&DU(I0{})[c * kT1 + (swc << 2)]);

    for (int64_t i0 = 0; i0 < n_pairs; i0 += PF) {
        static_for<0, PF>([&](auto Sc) {
            constexpr int S = decltype(Sc)::value;
            constexpr int P = S & 1;       // parity of the pair index (PF is even)
            using IP = std::integral_constant<int, P>;
            using I1P = std::integral_constant<int, 1 - P>;
            const int64_t i = i0 + S;
            if (i < n_pairs) {
                const int64_t t0 = i * (2 * kT1);
                unpack_raw<T, E>(ring[S].b, bv);
                unpack_raw<T, E>(ring[S].c, cv);
                // Two wait states between the VALU writes of the DPP sources and their first DPP
                // read by the fmac inline asm (the compiler covers its own DPP instructions).
#pragma unroll
                for (int k = 0; k < E; ++k) asm volatile("s_nop 1" : "+v"(bv[k]), "+v"(cv[k]));
                const RawVec<T, E> nu = ring[S].u, nd = ring[S].dl, nz = ring[S].z;  // pair i + 1
                load_data(i + PF, ring[S]);
                // Interval 2i: wave 0 prepares tile 2i+2, wave 1 finishes tile 2i-1.
                scan_tile(I0{}, t0, DT(std::integral_constant<int, 2 * P>{}), DU(std::integral_constant<int, 2 * P>{}),
                          YB(I0{}), DT(std::integral_constant<int, 2 * P + 1>{}),
                          DU(std::integral_constant<int, 2 * P + 1>{}));
                if (w == 0) prologue(nu, nd, nz, t0 + 2 * kT1, DT(std::integral_constant<int, 2 * P + 2>{}),
                                     DU(std::integral_constant<int, 2 * P + 2>{}), I1P{});
                else if (i > 0) epilogue(t0 - kT1, YB(I1{}), I1P{});
                __syncthreads();
                // Interval 2i+1: wave 1 prepares tile 2i+3, wave 0 finishes tile 2i.
                scan_tile(I1{}, t0 + kT1, DT(std::integral_constant<int, 2 * P + 1>{}),
                          DU(std::integral_constant<int, 2 * P + 1>{}), YB(I1{}),
                          DT(std::integral_constant<int, 2 * P + 2>{}), DU(std::integral_constant<int, 2 * P + 2>{}));
                if (w == 1) prologue(nu, nd, nz, t0 + 3 * kT1, DT(std::integral_constant<int, 2 * P + 3>{}),
                                     DU(std::integral_constant<int, 2 * P + 3>{}), I1P{});
                else epilogue(t0, YB(I0{}), IP{});
                __syncthreads();
            }
        });
    }
    // The last tile, 2 n_pairs - 1, belongs to wave 1.
    if (w == 1) {
        const int64_t tl = (2 * n_pairs - 1) * kT1;
        if (((n_pairs - 1) & 1) == 0) epilogue(tl, YB(I1{}), I0{});
        else epilogue(tl, YB(I1{}), I1{});
    }
    if (p.last_state) {
        p.last_state[(b * p.dim + d0 + c) * 16 + 2 * r] = h[0];
        p.last_state[(b * p.dim + d0 + c) * 16 + 2 * r + 1] = h[1];
    }
}

template <typename T, int PF, bool FULL>
int launch_k2i_full(const mm_scan_fwd_params &p, hipStream_t stream) {
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / kCh), unsigned(p.batch));
    auto *kern = p.delta_softplus
                     ? (p.chunk_states ? scan_fwd_k2i<T, PF, true, true, FULL> : scan_fwd_k2i<T, PF, true, false, FULL>)
                     : (p.chunk_states ? scan_fwd_k2i<T, PF, false, true, FULL> : scan_fwd_k2i<T, PF, false, false, FULL>);
    hipLaunchKernelGGL(kern, grid, dim3(128), 0, stream, p, ratio);
    return launch_status("scan_fwd_k2i");
}

// FULL needs whole tile pairs and byte offsets (span x element size) below 2^32; the callers have
// checked that the element span is below 2^31 (pipe_offsets_ok) and T is a 16-bit type here.
template <typename T, int PF>
int launch_k2i(const mm_scan_fwd_params &p, hipStream_t stream) {
    static_assert(sizeof(T) == 2, "k2i runs 16-bit inputs");
    static const bool nofull = getenv("MM_SCAN_NOFULL") != nullptr;
    if (p.seqlen % (2 * kT1) == 0 && !nofull) return launch_k2i_full<T, PF, true>(p, stream);
    return launch_k2i_full<T, PF, false>(p, stream);
}

// ---------------------------------------------------------------------------------------------
// scan_fwd_k2s: the scan of k2i with the per-element work split evenly over both waves. Every lane
// owns 2 consecutive steps of one channel in every tile (lane = 8 x channel + step pair), so in
// interval j each lane prepares its elements of tile j + 2, scans tile j with its row, and finishes
// its elements of tile j - 1: the same straight-line code in both waves, with no wave-dependent
// branch between the scan and the element work, so the scheduler can fill the scan's latency gaps
// with softplus, the row-partial sums and the gating. Taken when L is a multiple of 32 (whole tile
// pairs, buffer addressing as k2i's FULL path).
//
// Sequence segments (SEG, blockIdx.z = segment of sg.pairs tile pairs), as the pipelined kernel's
// MODE 1 and 2: SEG 1 scans segments 0 .. n_seg-2 from a zero state for the states alone (YO false)
// and writes each segment's end state and sum of delta'; SEG 2 scans every segment from its carried
// state (and delta' prefix) and writes the outputs, last_state from the last segment.
// ---------------------------------------------------------------------------------------------
template <typename T>
struct K2SData {                       // one lane's global data for pair iteration i
    RawVec<T, 4> b, c;                 // B, C of one of the lane's row states: 4 steps of pair i
    RawVec<T, 2> u0, d0, z0, u1, d1, z1;   // u, delta, z: 2 steps of tiles 0 and 1 of pair i + 1
};

// LDS of one k2s group: dt' and dt'u of four tiles, and two buffers of the 8 row partials of y
// ([row][channel][16 steps]); every row of 16 floats holds four 4-float blocks permuted by swz16.
struct K2SLds {
    float dt[4][kCh * kT1];
    float du[4][kCh * kT1];
    float y[2][8 * kCh * kT1];
};

// One 16-channel group of batch row b on 128 lanes (tid 0..127, two waves): the body of scan_fwd_k2s,
// also run twice per workgroup by scan_fwd_mix. Every lane of the workgroup calls __syncthreads()
// the same number of times (once per 16-step tile, the same tile count for both groups).
template <typename T, int PF, bool SOFTPLUS, bool CHUNKS, bool HAS_Z, bool HAS_OUT, bool YO, int SEG>
__device__ __forceinline__ void k2s_group(const mm_scan_fwd_params &p, const int64_t ratio, const SegArgs &sg,
                                          const int tid, const int64_t b, const int64_t d0, const int seg,
                                          K2SLds &lds) {
    static_assert(PF % 2 == 0, "the pair loop is unrolled by PF and needs a static parity");
    static_assert(SEG != 1 || !YO, "the first segment pass computes the states alone");
    static_assert(SEG != 2 || YO, "the second segment pass writes the outputs");
    constexpr int E = 2, LPS = 8, NR = 8;
    auto DT = [&](auto I) -> float * { return lds.dt[decltype(I)::value & 3]; };
    auto DU = [&](auto I) -> float * { return lds.du[decltype(I)::value & 3]; };
    auto YB = [&](auto I) -> float * { return lds.y[decltype(I)::value & 1]; };

    const int lane = tid & 63;
    const int r = tid >> 4;                // row (states 2r, 2r+1) of this lane in the scan
    const int c = lane & 15;               // channel of this lane in the scan
    const int ce = tid >> 3;               // channel of this lane's elements
    const int es = E * (tid & 7);          // first step (within a tile) of its two elements
    const int swc = swz16(c), swe = swz16(ce);   // LDS block permutations of the two channels
    const int64_t g = d0 / ratio;
    const int64_t L = p.seqlen;
    const int32_t n_pairs = int32_t(L / (2 * kT1));   // L is a multiple of 32 here
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    const int32_t pb = SEG ? int32_t(seg * sg.pairs) : 0;                                 // first pair
    const int32_t pe = SEG ? (pb + int32_t(sg.pairs) < n_pairs ? pb + int32_t(sg.pairs) : n_pairs) : n_pairs;
    const int64_t srow = (b * p.dim + d0 + c) * int64_t(sg.n_seg) + seg;                 // segment slot

    const int64_t de = d0 + ce;
    const T *ub = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d0 * p.u_d_stride;
    const T *db = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d0 * p.delta_d_stride;
    const T *zb = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d0 * p.z_d_stride : nullptr;
    T *ob = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d0 * p.out_d_stride : nullptr;
    T *ozb = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d0 * p.out_z_d_stride : nullptr;
    const T *Bb = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cb = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;
    const int nl = 2 * r + c / LPS;        // the state whose B/C this lane loads
    const int sb = 4 * (c % LPS);          // first step (within a pair) of this lane's B/C slice

    float At[2], h[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        At[k] = p.A[(d0 + c) * p.A_d_stride + int64_t(2 * r + k) * p.A_dstate_stride] * kLog2e;
        h[k] = SEG == 2 ? sg.h[srow * 16 + 2 * r + k] : 0.f;
    }
    const float Dv = p.D ? p.D[de] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[de] : 0.f;
    float cum_dt = (SEG == 2 && CHUNKS) ? sg.cum[srow] : 0.f;

    // Buffer resources of the group's rows (the host checks that every byte offset of the group is
    // below 2^32) and this lane's byte offsets from them; tile and pair offsets are scalar.
    constexpr uint32_t SZ = sizeof(T);
    const uint32_t fo_u = uint32_t(ce * p.u_d_stride + es) * SZ, fo_d = uint32_t(ce * p.delta_d_stride + es) * SZ;
    const uint32_t fo_z = uint32_t(ce * p.z_d_stride + es) * SZ;
    const uint32_t fo_b = uint32_t(nl * p.B_dstate_stride + sb) * SZ, fo_c = uint32_t(nl * p.C_dstate_stride + sb) * SZ;
    const uint32_t fo_o = uint32_t(ce * p.out_d_stride + es) * SZ, fo_oz = uint32_t(ce * p.out_z_d_stride + es) * SZ;
    const __amdgpu_buffer_rsrc_t rs_u = buffer_rsrc(ub), rs_d = buffer_rsrc(db), rs_z = buffer_rsrc(zb);
    const __amdgpu_buffer_rsrc_t rs_b = buffer_rsrc(Bb), rs_c = buffer_rsrc(Cb);
    const __amdgpu_buffer_rsrc_t rs_o = buffer_rsrc(ob), rs_oz = buffer_rsrc(ozb);
    // Pair and tile indices past the end are clamped to the last ones (the data they bring is
    // never used): every access stays inside the rows.
    auto pair_off = [&](int32_t i) { return uint32_t(i < n_pairs ? i : n_pairs - 1) * uint32_t(2 * kT1 * SZ); };
    auto tile_off = [&](int32_t t) { return uint32_t(t < 2 * n_pairs ? t : 2 * n_pairs - 1) * uint32_t(kT1 * SZ); };
    auto load_tile = [&](int32_t t, RawVec<T, E> &u, RawVec<T, E> &dl, RawVec<T, E> &z) {
        const uint32_t sof = tile_off(t);
        u = buffer_load_raw<T, E>(rs_u, fo_u, sof);
        dl = buffer_load_raw<T, E>(rs_d, fo_d, sof);
        if constexpr (HAS_Z) z = buffer_load_raw<T, E>(rs_z, fo_z, sof);
        else z = {};
    };
    auto load_data = [&](int32_t i, K2SData<T> &dst) {
        const uint32_t sof = pair_off(i);
        dst.b = buffer_load_raw<T, 4>(rs_b, fo_b, sof);
        if constexpr (YO) dst.c = buffer_load_raw<T, 4>(rs_c, fo_c, sof);
        else dst.c = {};
        load_tile(2 * i + 2, dst.u0, dst.d0, dst.z0);
        load_tile(2 * i + 3, dst.u1, dst.d1, dst.z1);
    };

    // u (unpacked) and z of the tiles between their prologue and their epilogue: tile t in slot t % 4.
    float ru[4][E];
    RawVec<T, E> rz[4];

    // Prologue of tile t (slot S = t % 4): delta', delta' u of this lane's two elements -> LDS.
    auto prologue = [&](auto Slot, const RawVec<T, E> &u, const RawVec<T, E> &dl, const RawVec<T, E> &z) {
        constexpr int sl = decltype(Slot)::value & 3;
        float uu[E], dd[E], dtp[E];
        unpack_raw<T, E>(u, uu);
        unpack_raw<T, E>(dl, dd);
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float x = dd[k] + bias;
            dtp[k] = SOFTPLUS ? softplus_fast(x) : x;
        }
        *reinterpret_cast<float2 *>(&DT(Slot)[ce * kT1 + (((es >> 2) ^ swe) << 2) + (es & 3)]) = make_float2(dtp[0], dtp[1]);
        *reinterpret_cast<float2 *>(&DU(Slot)[ce * kT1 + (((es >> 2) ^ swe) << 2) + (es & 3)]) = make_float2(dtp[0] * uu[0], dtp[1] * uu[1]);
        if constexpr (YO) {
#pragma unroll
            for (int k = 0; k < E; ++k) ru[sl][k] = uu[k];
            rz[sl] = z;
        }
    };

    // Epilogue of tile t (slot S = t % 4, partials in yb): the 8 row partials added in row order,
    // D u, the silu(z) gate, one 2-element store. The first interval finishes no tile; it runs the
    // same code on the unused buffers and stores to tile 0, which the lane overwrites with tile 0's
    // real outputs one interval later (same lane, same addresses, program order), so that no branch
    // separates the scan from the element work.
    auto epilogue = [&](auto Slot, const float *yb, int32_t t) {
        constexpr int sl = decltype(Slot)::value & 3;
        const int ecol = (((es >> 2) ^ swe) << 2) + (es & 3);
        float2 a = *reinterpret_cast<const float2 *>(&yb[ce * kT1 + ecol]);
#pragma unroll
        for (int rr = 1; rr < NR; ++rr) {
            const float2 v = *reinterpret_cast<const float2 *>(&yb[(rr * kCh + ce) * kT1 + ecol]);
            a.x += v.x;
            a.y += v.y;
        }
        float zz[E];
        unpack_raw<T, E>(rz[sl], zz);
        float o[E] = {__builtin_fmaf(Dv, ru[sl][0], a.x), __builtin_fmaf(Dv, ru[sl][1], a.y)};
        const uint32_t sof = uint32_t(t) * uint32_t(kT1 * SZ);
        if constexpr (HAS_OUT) buffer_store_vec<T, E>(rs_o, fo_o, sof, o);
        if constexpr (HAS_Z) {
#pragma unroll
            for (int k = 0; k < E; ++k) o[k] *= silu_fast(zz[k]);
            buffer_store_vec<T, E>(rs_oz, fo_oz, sof, o);
        }
    };

    // Scan of one tile (pair half H) from dt/du into the row partials yb, as k2i's: B/C of state
    // 2r + k at step s of the pair sit in lane 8k + s / 4 of this row, register s % 4; dt' / dt'u
    // are read one 4-step group ahead (group 0 of the next tile at the end of this one).
    float bv[4], cv[4];
    float4 pre_dt, pre_du;
    auto scan_tile = [&](auto Hc, int64_t t0, const float *dt, const float *du, float *yb, const float *dtn,
                         const float *dun) {
        constexpr int H = decltype(Hc)::value;
        float4 dtq = pre_dt, duq = pre_du;
        static_for<0, kT1 / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            float4 ndt, ndu;
            if constexpr (s4 + 1 < kT1 / 4) {
                ndt = *reinterpret_cast<const float4 *>(&dt[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&du[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
            } else {
                ndt = *reinterpret_cast<const float4 *>(&dtn[c * kT1 + (swc << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&dun[c * kT1 + (swc << 2)]);
            }
            const float dts[4] = {dtq.x, dtq.y, dtq.z, dtq.w};
            const float dus[4] = {duq.x, duq.y, duq.z, duq.w};
            float av[4][2], bbv[4][2], pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                if (CHUNKS || SEG == 1) cum_dt += dts[j];
                static_for<0, 2>([&](auto KK) {
                    constexpr int k = decltype(KK)::value;
                    av[j][k] = decay_exp2(dts[j], At[k]);
                    bbv[j][k] = row_bcast<k * LPS + s / 4>(bv[s % 4]) * dus[j];
                });
            });
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                h[0] = __builtin_fmaf(av[j][0], h[0], bbv[j][0]);
                h[1] = __builtin_fmaf(av[j][1], h[1], bbv[j][1]);
                if constexpr (YO) {
                    float acc = row_bcast<s / 4>(cv[s % 4]) * h[0];
                    fmac_row_bcast<LPS + s / 4>(acc, cv[s % 4], h[1]);
                    pv[j] = acc;
                }
            });
            if constexpr (YO)
                *reinterpret_cast<float4 *>(&yb[(r * kCh + c) * kT1 + ((s4 ^ swc) << 2)]) =
                    make_float4(pv[0], pv[1], pv[2], pv[3]);
            // Without the y-partial chain the scheduler would hoist the exponentials of a whole
            // tile and run out of registers: the states-only scan stays in 4-step groups.
            if constexpr (!YO) __builtin_amdgcn_sched_barrier(0);
            dtq = ndt;
            duq = ndu;
        });
        pre_dt = dtq;
        pre_du = duq;
        if (CHUNKS && p.chunk_states) {
            const int64_t tend = t0 + kT1;
            if (tend % MM_SCAN_CHUNK == 0 || tend == L) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *csp = p.chunk_states + ((b * p.dim + d0 + c) * n_chunks + ci) * 32 + 4 * r;
                csp[0] = __builtin_amdgcn_exp2f(At[0] * cum_dt);
                csp[1] = h[0];
                csp[2] = __builtin_amdgcn_exp2f(At[1] * cum_dt);
                csp[3] = h[1];
            }
        }
        if (SEG == 0 && (CHUNKS || !YO) && p.tile_states && t0 + kT1 < L) {
            float *ck = p.tile_states + ((t0 / kT1 + 1) * p.batch * p.dim + b * p.dim + d0 + c) * 16 + 2 * r;
            *reinterpret_cast<float2 *>(ck) = make_float2(h[0], h[1]);
        }
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if (SEG == 0 && (CHUNKS || !YO) && p.tile_states)  // the checkpoint before the first tile: zero
        *reinterpret_cast<float2 *>(p.tile_states + (b * p.dim + d0 + c) * 16 + 2 * r) = make_float2(0.f, 0.f);
    // Tile t of the segment sits in slot (t - 2 pb) % 4: the slots and buffer parities below count
    // pairs from pb.
    K2SData<T> ring[PF];
    {
        RawVec<T, E> u0, dl0, z0, u1, dl1, z1;
        load_tile(2 * pb, u0, dl0, z0);
        load_tile(2 * pb + 1, u1, dl1, z1);
#pragma unroll
        for (int s = 0; s < PF; ++s) load_data(pb + s, ring[s]);
        prologue(I0{}, u0, dl0, z0);       // tiles 2 pb and 2 pb + 1, slots 0 and 1
        prologue(I1{}, u1, dl1, z1);
    }
    __syncthreads();
    pre_dt = *reinterpret_cast<const float4 *>(&DT(I0{})[c * kT1 + (swc << 2)]);
    pre_du = *reinterpret_cast<const float4 *>(&DU(I0{})[c * kT1 + (swc << 2)]);

    for (int32_t i0 = pb; i0 < pe; i0 += PF) {
        static_for<0, PF>([&](auto Sc) {
            constexpr int S = decltype(Sc)::value;
            constexpr int P = S & 1;       // parity of the pair index from pb (PF is even)
            using T2P = std::integral_constant<int, 2 * P>;
            using T2P1 = std::integral_constant<int, 2 * P + 1>;
            using T2P2 = std::integral_constant<int, 2 * P + 2>;
            using T2P3 = std::integral_constant<int, 2 * P + 3>;
            const int32_t i = i0 + S;
            if (i < pe) {
                const int64_t t0 = int64_t(i) * (2 * kT1);
                unpack_raw<T, 4>(ring[S].b, bv);
                // Two wait states between the VALU writes of the DPP sources and their first DPP
                // read by the fmac inline asm (the compiler covers its own DPP instructions).
                if constexpr (YO) {
                    unpack_raw<T, 4>(ring[S].c, cv);
#pragma unroll
                    for (int k = 0; k < 4; ++k) asm volatile("s_nop 1" : "+v"(bv[k]), "+v"(cv[k]));
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) asm volatile("s_nop 1" : "+v"(bv[k]));
                }
                // The ring entry is refilled with pair i + PF (B/C) and the elements of the pair
                // after it before this pair's scan starts, about two pairs ahead of their use; its
                // elements of pair i + 1 are kept in `nxt` for the two prologues below. Refilling
                // the entry after the second prologue instead (no copy, fewer registers) left only
                // one pair of distance and cost 2.3 % at config 2.
                const K2SData<T> nxt = ring[S];
                load_data(i + PF, ring[S]);
                // Interval 2i: scan tile 2i, prepare tile 2i + 2, finish tile 2i - 1.
                scan_tile(I0{}, t0, DT(T2P{}), DU(T2P{}), YB(I0{}), DT(T2P1{}), DU(T2P1{}));
                prologue(T2P2{}, nxt.u0, nxt.d0, nxt.z0);
                if constexpr (YO) epilogue(T2P3{}, YB(I1{}), i > pb ? 2 * i - 1 : 2 * pb);
                __syncthreads();
                // Interval 2i + 1: scan tile 2i + 1, prepare tile 2i + 3, finish tile 2i.
                scan_tile(I1{}, t0 + kT1, DT(T2P1{}), DU(T2P1{}), YB(I1{}), DT(T2P2{}), DU(T2P2{}));
                prologue(T2P3{}, nxt.u1, nxt.d1, nxt.z1);
                if constexpr (YO) epilogue(T2P{}, YB(I0{}), 2 * i);
                __syncthreads();
            }
        });
    }
    // The last tile, 2 pe - 1 (slot (2 (pe - pb) - 1) % 4: 1 or 3).
    if constexpr (YO) {
        if (((pe - 1 - pb) & 1) == 0) epilogue(I1{}, YB(I1{}), 2 * pe - 1);
        else epilogue(std::integral_constant<int, 3>{}, YB(I1{}), 2 * pe - 1);
    }
    if constexpr (SEG == 1) {
        sg.h[srow * 16 + 2 * r] = h[0];
        sg.h[srow * 16 + 2 * r + 1] = h[1];
        if (r == 0) sg.sumdt[srow] = cum_dt;
    } else if (p.last_state && (SEG == 0 || seg == sg.n_seg - 1)) {
        p.last_state[(b * p.dim + d0 + c) * 16 + 2 * r] = h[0];
        p.last_state[(b * p.dim + d0 + c) * 16 + 2 * r + 1] = h[1];
    }
}

template <typename T, int PF, bool SOFTPLUS, bool CHUNKS, bool HAS_Z, bool HAS_OUT, bool YO, int SEG = 0>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(3, 8)))
scan_fwd_k2s(const mm_scan_fwd_params p, const int64_t ratio, const SegArgs sg) {
    __shared__ __align__(16) K2SLds lds;
    k2s_group<T, PF, SOFTPLUS, CHUNKS, HAS_Z, HAS_OUT, YO, SEG>(p, ratio, sg, threadIdx.x, blockIdx.y,
                                                                int64_t(blockIdx.x) * kCh, SEG ? int(blockIdx.z) : 0, lds);
}

using K2SKernel = void (*)(const mm_scan_fwd_params, const int64_t, const SegArgs);
constexpr SegArgs kWholeRows{0, 1, nullptr, nullptr, nullptr};

// ---------------------------------------------------------------------------------------------
// k1s: one state per lane. A 16-channel group of batch row b on 256 lanes (four waves), lane
// 16 r + c holding state r of channel c, in k2s's interval structure: per 16-step tile j each lane
// prepares one element of tile j + 2 (channel r, step c), scans tile j (16 state updates) and
// finishes one element of tile j - 1, adding the 16 row partials of y in row order. Per state
// update it issues what k2s issues (exp2 and its argument, B dt'u and C h by DPP row broadcast, the
// state FMA) with the element work and the row partials spread over twice the lanes. scan_fwd_mix
// runs it beside k2s groups so that every SIMD of the device carries the same number of states.
// ---------------------------------------------------------------------------------------------
struct K1SLds {
    float dt[4][kCh * kT1];
    float du[4][kCh * kT1];
    float y[2][16 * kCh * kT1];
};

template <typename T>
struct K1SData {                       // one lane's global data for pair iteration i
    RawVec<T, 2> b, c;                 // B, C of the lane's state: steps 2c and 2c + 1 of pair i
    uint32_t u0, d0, z0, u1, d1, z1;   // u, delta, z: one element of tiles 0 and 1 of pair i + 1 (raw bits)
};

// One element of T through a buffer resource, as raw bits (16-bit types zero-extended).
template <typename T>
__device__ __forceinline__ uint32_t buffer_load_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (sizeof(T) == 4)
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    else
        return uint32_t(__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
}
template <typename T>
__device__ __forceinline__ float elem_f32(uint32_t w) {
    if constexpr (std::is_same_v<T, float>) return __uint_as_float(w);
    else if constexpr (std::is_same_v<T, bf16_t>) return __uint_as_float(w << 16);
    else return float(__builtin_bit_cast(_Float16, uint16_t(w)));
}
// One float stored as T (bf16 round-to-nearest-even, as buffer_store_vec converts).
template <typename T>
__device__ __forceinline__ void buffer_store_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float x) {
    if constexpr (std::is_same_v<T, float>)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, voff, soff, 0);
    else if constexpr (std::is_same_v<T, bf16_t>)
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(pack_bf16x2(x, 0.f) & 0xffffu), r, voff, soff, 0);
    else
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (_Float16)x), r, voff, soff, 0);
}

// CHUNKS: the training outputs as k2s writes them -- the chunk states (the product of the decays
// since step 0 and the state, at every chunk end) and, on request, the state after every 16-step
// tile for the backward. YO false: the states alone (no C, y or outputs), the tile states written,
// as k2s's states-only form.
template <typename T, int PF, bool SOFTPLUS, bool HAS_Z, bool HAS_OUT, bool CHUNKS = false, bool YO = true>
__device__ __forceinline__ void k1s_group(const mm_scan_fwd_params &p, const int64_t ratio, const int tid,
                                          const int64_t b, const int64_t d0, K1SLds &lds) {
    static_assert(PF % 2 == 0, "the pair loop is unrolled by PF and needs a static parity");
    constexpr int NR = 16;
    auto DT = [&](auto I) -> float * { return lds.dt[decltype(I)::value & 3]; };
    auto DU = [&](auto I) -> float * { return lds.du[decltype(I)::value & 3]; };
    auto YB = [&](auto I) -> float * { return lds.y[decltype(I)::value & 1]; };

    const int r = tid >> 4;                // state of this lane in the scan; channel of its element
    const int c = tid & 15;                // channel of this lane in the scan; step of its element
    const int ce = r, es = c;
    const int swc = swz16(c), swe = swz16(ce);
    const int64_t g = d0 / ratio;
    const int64_t L = p.seqlen;
    const int32_t n_pairs = int32_t(L / (2 * kT1));   // L is a multiple of 32 here

    const int64_t de = d0 + ce;
    const T *ub = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d0 * p.u_d_stride;
    const T *db = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d0 * p.delta_d_stride;
    const T *zb = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d0 * p.z_d_stride : nullptr;
    T *ob = p.out ? reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d0 * p.out_d_stride : nullptr;
    T *ozb = p.out_z ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d0 * p.out_z_d_stride : nullptr;
    const T *Bb = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cb = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;

    const float At = p.A[(d0 + c) * p.A_d_stride + int64_t(r) * p.A_dstate_stride] * kLog2e;
    float h = 0.f;
    float cum_dt = 0.f;                    // CHUNKS: sum of dt' since step 0
    const int64_t n_chunks = (L + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    const float Dv = p.D ? p.D[de] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[de] : 0.f;

    // Buffer resources of the group's rows (the host checks that every byte offset of the group is
    // below 2^32) and this lane's byte offsets from them; tile and pair offsets are scalar.
    constexpr uint32_t SZ = sizeof(T);
    const uint32_t fo_u = uint32_t(ce * p.u_d_stride + es) * SZ, fo_d = uint32_t(ce * p.delta_d_stride + es) * SZ;
    const uint32_t fo_z = uint32_t(ce * p.z_d_stride + es) * SZ;
    const uint32_t fo_b = uint32_t(r * p.B_dstate_stride + 2 * c) * SZ, fo_c = uint32_t(r * p.C_dstate_stride + 2 * c) * SZ;
    const uint32_t fo_o = uint32_t(ce * p.out_d_stride + es) * SZ, fo_oz = uint32_t(ce * p.out_z_d_stride + es) * SZ;
    const __amdgpu_buffer_rsrc_t rs_u = buffer_rsrc(ub), rs_d = buffer_rsrc(db), rs_z = buffer_rsrc(zb);
    const __amdgpu_buffer_rsrc_t rs_b = buffer_rsrc(Bb), rs_c = buffer_rsrc(Cb);
    const __amdgpu_buffer_rsrc_t rs_o = buffer_rsrc(ob), rs_oz = buffer_rsrc(ozb);
    // Pair and tile indices past the end are clamped to the last ones (their data is never used).
    auto pair_off = [&](int32_t i) { return uint32_t(i < n_pairs ? i : n_pairs - 1) * uint32_t(2 * kT1 * SZ); };
    auto tile_off = [&](int32_t t) { return uint32_t(t < 2 * n_pairs ? t : 2 * n_pairs - 1) * uint32_t(kT1 * SZ); };
    auto load_tile = [&](int32_t t, uint32_t &u, uint32_t &dl, uint32_t &z) {
        const uint32_t sof = tile_off(t);
        u = buffer_load_elem<T>(rs_u, fo_u, sof);
        dl = buffer_load_elem<T>(rs_d, fo_d, sof);
        z = HAS_Z ? buffer_load_elem<T>(rs_z, fo_z, sof) : 0u;
    };
    auto load_data = [&](int32_t i, K1SData<T> &dst) {
        const uint32_t sof = pair_off(i);
        dst.b = buffer_load_raw<T, 2>(rs_b, fo_b, sof);
        if constexpr (YO) dst.c = buffer_load_raw<T, 2>(rs_c, fo_c, sof);
        else dst.c = {};
        load_tile(2 * i + 2, dst.u0, dst.d0, dst.z0);
        load_tile(2 * i + 3, dst.u1, dst.d1, dst.z1);
    };

    // u (unpacked) and z of the tiles between their prologue and their epilogue: tile t in slot t % 4.
    float ru[4];
    uint32_t rz[4];
    auto prologue = [&](auto Slot, uint32_t u, uint32_t dl, uint32_t z) {
        constexpr int sl = decltype(Slot)::value & 3;
        const float uu = elem_f32<T>(u);
        const float x = elem_f32<T>(dl) + bias;
        const float dtp = SOFTPLUS ? softplus_fast(x) : x;
        const int pos = ce * kT1 + (((es >> 2) ^ swe) << 2) + (es & 3);
        DT(Slot)[pos] = dtp;
        DU(Slot)[pos] = dtp * uu;
        ru[sl] = uu;
        rz[sl] = z;
    };
    // Epilogue of tile t: the 16 row partials added in row order, D u, the silu(z) gate, one store.
    // The first interval runs it on the unused buffers and stores to tile 0, which the same lane
    // overwrites with tile 0's outputs one interval later (as k2s does).
    auto epilogue = [&](auto Slot, const float *yb, int32_t t) {
        if constexpr (!YO) return;
        constexpr int sl = decltype(Slot)::value & 3;
        const int ecol = (((es >> 2) ^ swe) << 2) + (es & 3);
        float a = yb[ce * kT1 + ecol];
#pragma unroll
        for (int rr = 1; rr < NR; ++rr) a += yb[(rr * kCh + ce) * kT1 + ecol];
        float o = __builtin_fmaf(Dv, ru[sl], a);
        const uint32_t sof = uint32_t(t) * uint32_t(kT1 * SZ);
        if constexpr (HAS_OUT) buffer_store_elem<T>(rs_o, fo_o, sof, o);
        if constexpr (HAS_Z) {
            o *= silu_fast(elem_f32<T>(rz[sl]));
            buffer_store_elem<T>(rs_oz, fo_oz, sof, o);
        }
    };

    // Scan of one tile (pair half H): B/C of the lane's state at step s of the pair sit in lane s / 2
    // of its row, register s % 2; dt' / dt'u are read one 4-step group ahead.
    float bv[2], cv[2];
    float4 pre_dt, pre_du;
    auto scan_tile = [&](auto Hc, int64_t t0, const float *dt, const float *du, float *yb, const float *dtn,
                         const float *dun) {
        constexpr int H = decltype(Hc)::value;
        float4 dtq = pre_dt, duq = pre_du;
        static_for<0, kT1 / 4>([&](auto S4) {
            constexpr int s4 = decltype(S4)::value;
            float4 ndt, ndu;
            if constexpr (s4 + 1 < kT1 / 4) {
                ndt = *reinterpret_cast<const float4 *>(&dt[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&du[c * kT1 + (((s4 + 1) ^ swc) << 2)]);
            } else {
                ndt = *reinterpret_cast<const float4 *>(&dtn[c * kT1 + (swc << 2)]);
                ndu = *reinterpret_cast<const float4 *>(&dun[c * kT1 + (swc << 2)]);
            }
            const float dts[4] = {dtq.x, dtq.y, dtq.z, dtq.w};
            const float dus[4] = {duq.x, duq.y, duq.z, duq.w};
            float av[4], bbv[4], pv[4];
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                if constexpr (CHUNKS) cum_dt += dts[j];
                av[j] = decay_exp2(dts[j], At);
                bbv[j] = row_bcast<s / 2>(bv[s % 2]) * dus[j];
            });
            static_for<0, 4>([&](auto J) {
                constexpr int j = decltype(J)::value;
                constexpr int s = kT1 * H + 4 * s4 + j;
                h = __builtin_fmaf(av[j], h, bbv[j]);
                if constexpr (YO) pv[j] = row_bcast<s / 2>(cv[s % 2]) * h;
            });
            if constexpr (YO)
                *reinterpret_cast<float4 *>(&yb[(r * kCh + c) * kT1 + ((s4 ^ swc) << 2)]) =
                    make_float4(pv[0], pv[1], pv[2], pv[3]);
            dtq = ndt;
            duq = ndu;
        });
        pre_dt = dtq;
        pre_du = duq;
        if constexpr (CHUNKS || !YO) {
            const int64_t tend = t0 + kT1;
            if (CHUNKS && p.chunk_states && (tend % MM_SCAN_CHUNK == 0 || tend == L)) {
                const int64_t ci = (tend - 1) / MM_SCAN_CHUNK;
                float *csp = p.chunk_states + ((b * p.dim + d0 + c) * n_chunks + ci) * 32 + 2 * r;
                csp[0] = __builtin_amdgcn_exp2f(At * cum_dt);
                csp[1] = h;
            }
            if (p.tile_states && tend < L)
                p.tile_states[((t0 / kT1 + 1) * p.batch * p.dim + b * p.dim + d0 + c) * 16 + r] = h;
        }
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if ((CHUNKS || !YO) && p.tile_states)  // the checkpoint before the first tile: zero
        p.tile_states[(b * p.dim + d0 + c) * 16 + r] = 0.f;
    K1SData<T> ring[PF];
    {
        uint32_t u0, dl0, z0, u1, dl1, z1;
        load_tile(0, u0, dl0, z0);
        load_tile(1, u1, dl1, z1);
#pragma unroll
        for (int s = 0; s < PF; ++s) load_data(s, ring[s]);
        prologue(I0{}, u0, dl0, z0);
        prologue(I1{}, u1, dl1, z1);
    }
    __syncthreads();
    pre_dt = *reinterpret_cast<const float4 *>(&DT(I0{})[c * kT1 + (swc << 2)]);
    pre_du = *reinterpret_cast<const float4 *>(&DU(I0{})[c * kT1 + (swc << 2)]);

    for (int32_t i0 = 0; i0 < n_pairs; i0 += PF) {
        static_for<0, PF>([&](auto Sc) {
            constexpr int S = decltype(Sc)::value;
            constexpr int P = S & 1;
            using T2P = std::integral_constant<int, 2 * P>;
            using T2P1 = std::integral_constant<int, 2 * P + 1>;
            using T2P2 = std::integral_constant<int, 2 * P + 2>;
            using T2P3 = std::integral_constant<int, 2 * P + 3>;
            const int32_t i = i0 + S;
            if (i < n_pairs) {
                const int64_t t0 = int64_t(i) * (2 * kT1);
                unpack_raw<T, 2>(ring[S].b, bv);
                unpack_raw<T, 2>(ring[S].c, cv);
                const K1SData<T> nxt = ring[S];
                load_data(i + PF, ring[S]);
                // Interval 2i: scan tile 2i, prepare tile 2i + 2, finish tile 2i - 1.
                scan_tile(I0{}, t0, DT(T2P{}), DU(T2P{}), YB(I0{}), DT(T2P1{}), DU(T2P1{}));
                prologue(T2P2{}, nxt.u0, nxt.d0, nxt.z0);
                epilogue(T2P3{}, YB(I1{}), i > 0 ? 2 * i - 1 : 0);
                __syncthreads();
                // Interval 2i + 1: scan tile 2i + 1, prepare tile 2i + 3, finish tile 2i.
                scan_tile(I1{}, t0 + kT1, DT(T2P1{}), DU(T2P1{}), YB(I1{}), DT(T2P2{}), DU(T2P2{}));
                prologue(T2P3{}, nxt.u1, nxt.d1, nxt.z1);
                epilogue(T2P{}, YB(I0{}), 2 * i);
                __syncthreads();
            }
        });
    }
    // The last tile, 2 n_pairs - 1 (slot 1 or 3).
    if (((n_pairs - 1) & 1) == 0) epilogue(I1{}, YB(I1{}), 2 * n_pairs - 1);
    else epilogue(std::integral_constant<int, 3>{}, YB(I1{}), 2 * n_pairs - 1);
    if (p.last_state) p.last_state[(b * p.dim + d0 + c) * 16 + r] = h;
}

// scan_fwd_mix: blocks [0, n_double) run two k2s groups each (waves 0-1 and 2-3), the blocks after
// them one k1s group each; every block has four waves. The grid is sized so that each compute unit
// holds n_double / CUs two-group blocks and one one-group block at once (the hardware places a
// block's four waves on the four SIMDs of a CU and deals the blocks out round-robin), which puts
// the same number of (channel, state) rows on every SIMD: at 5 groups per CU, 2 x 2 + 1 x 1 states
// per lane; at 3 groups per CU, 1 x 2 + 1 x 1. Groups are numbered batch-major; group g always takes
// the same path for a given shape and device, so results do not depend on scheduling.
union MixLds {
    K2SLds k2[2];
    K1SLds k1;
};

// CHUNKS: the training form (chunk states and, on request, tile states), 16-bit inputs. YO false:
// the states alone (the backward's checkpoints), 16-bit inputs.
template <typename T, bool SOFTPLUS, bool HAS_Z, bool HAS_OUT, bool CHUNKS, bool YO = true>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8)))
scan_fwd_mix(const mm_scan_fwd_params p, const int64_t ratio, const int32_t n_double) {
    __shared__ __align__(16) MixLds lds;
    const int64_t gpb = p.dim / kCh;   // 16-channel groups per batch row
    if (int32_t(blockIdx.x) < n_double) {
        // Waves 0-1 take the first group, waves 2-3 the second: uniform per wave, made scalar so
        // that the group's buffer resources stay in SGPRs.
        const int half = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 7));
        const int64_t grp = 2 * int64_t(blockIdx.x) + half;
        k2s_group<T, 2, SOFTPLUS, CHUNKS, HAS_Z, HAS_OUT, YO, 0>(p, ratio, kWholeRows, threadIdx.x & 127, grp / gpb,
                                                                 (grp % gpb) * kCh, 0, lds.k2[half]);
    } else {
        const int64_t grp = 2 * int64_t(n_double) + (int64_t(blockIdx.x) - n_double);
        k1s_group<T, 2, SOFTPLUS, HAS_Z, HAS_OUT, CHUNKS, YO>(p, ratio, threadIdx.x, grp / gpb, (grp % gpb) * kCh,
                                                              lds.k1);
    }
}

template <typename T, bool HAS_Z, bool HAS_OUT>
int launch_mix_io(const mm_scan_fwd_params &p, hipStream_t stream, int32_t n_double, int32_t n_single) {
    const int64_t ratio = p.dim / p.n_groups;
    using K = void (*)(const mm_scan_fwd_params, const int64_t, const int32_t);
    K kern;
    if constexpr (sizeof(T) == 4) {
        if (p.chunk_states || p.tile_states) return MM_ERR_UNSUPPORTED;   // no fp32 training instance
        kern = p.delta_softplus ? scan_fwd_mix<T, true, HAS_Z, HAS_OUT, false> : scan_fwd_mix<T, false, HAS_Z, HAS_OUT, false>;
    } else {
        kern = p.chunk_states ? (p.delta_softplus ? scan_fwd_mix<T, true, HAS_Z, HAS_OUT, true>
                                                  : scan_fwd_mix<T, false, HAS_Z, HAS_OUT, true>)
                              : (p.delta_softplus ? scan_fwd_mix<T, true, HAS_Z, HAS_OUT, false>
                                                  : scan_fwd_mix<T, false, HAS_Z, HAS_OUT, false>);
    }
    hipLaunchKernelGGL(kern, dim3(unsigned(n_double + n_single)), dim3(256), 0, stream, p, ratio, n_double);
    return launch_status("scan_fwd_mix");
}

template <typename T>
int launch_mix(const mm_scan_fwd_params &p, hipStream_t stream, int32_t n_double, int32_t n_single) {
    if (p.z) return p.out ? launch_mix_io<T, true, true>(p, stream, n_double, n_single)
                          : launch_mix_io<T, true, false>(p, stream, n_double, n_single);
    return launch_mix_io<T, false, true>(p, stream, n_double, n_single);
}

// fp32 rows: only the instances without chunk states (the training variants' chunk and tile state
// stores take them past 168 VGPRs, where they spill); the caller routes chunk states elsewhere.
template <typename T, int PF, bool HAS_Z, bool HAS_OUT>
int launch_k2s_io(const mm_scan_fwd_params &p, hipStream_t stream) {
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / kCh), unsigned(p.batch));
    K2SKernel kern;
    if constexpr (sizeof(T) == 4) {
        if (p.chunk_states || p.tile_states) return MM_ERR_UNSUPPORTED;
        kern = p.delta_softplus ? scan_fwd_k2s<T, PF, true, false, HAS_Z, HAS_OUT, true>
                                : scan_fwd_k2s<T, PF, false, false, HAS_Z, HAS_OUT, true>;
    } else {
        kern = p.delta_softplus ? (p.chunk_states ? scan_fwd_k2s<T, PF, true, true, HAS_Z, HAS_OUT, true>
                                                  : scan_fwd_k2s<T, PF, true, false, HAS_Z, HAS_OUT, true>)
                                : (p.chunk_states ? scan_fwd_k2s<T, PF, false, true, HAS_Z, HAS_OUT, true>
                                                  : scan_fwd_k2s<T, PF, false, false, HAS_Z, HAS_OUT, true>);
    }
    hipLaunchKernelGGL(kern, grid, dim3(128), 0, stream, p, ratio, kWholeRows);
    return launch_status("scan_fwd_k2s");
}

template <typename T, int PF>
int launch_k2s(const mm_scan_fwd_params &p, hipStream_t stream) {
    if (p.z) return p.out ? launch_k2s_io<T, PF, true, true>(p, stream) : launch_k2s_io<T, PF, true, false>(p, stream);
    return launch_k2s_io<T, PF, false, true>(p, stream);   // without z the pre-gate out is the output
}

// The states alone (L a multiple of 32): p.tile_states, and p.last_state when given; on the
// balanced mixed grid when the caller found a plan for it (n_double + n_single > 0, 16-bit inputs).
template <typename T>
int launch_k2s_states(const mm_scan_fwd_params &p, hipStream_t stream, int32_t n_double, int32_t n_single) {
    const int64_t ratio = p.dim / p.n_groups;
    if constexpr (sizeof(T) == 2) {
        if (n_double + n_single > 0) {
            auto *kern = p.delta_softplus ? scan_fwd_mix<T, true, false, false, false, false>
                                          : scan_fwd_mix<T, false, false, false, false, false>;
            hipLaunchKernelGGL(kern, dim3(unsigned(n_double + n_single)), dim3(256), 0, stream, p, ratio, n_double);
            return launch_status("scan_fwd_mix_states");
        }
    }
    dim3 grid(unsigned(p.dim / kCh), unsigned(p.batch));
    auto *kern = p.delta_softplus ? scan_fwd_k2s<T, 2, true, false, false, false, false>
                                  : scan_fwd_k2s<T, 2, false, false, false, false, false>;
    hipLaunchKernelGGL(kern, grid, dim3(128), 0, stream, p, ratio, kWholeRows);
    return launch_status("scan_fwd_k2s_states");
}

// The full pass of the segmented k2s (SEG 2) for one output set; fp32 has no chunk-state instance.
template <typename T, bool HAS_Z, bool HAS_OUT>
K2SKernel k2s_seg_full(bool softplus, bool chunks) {
    if constexpr (sizeof(T) == 4)
        return softplus ? scan_fwd_k2s<T, 2, true, false, HAS_Z, HAS_OUT, true, 2>
                        : scan_fwd_k2s<T, 2, false, false, HAS_Z, HAS_OUT, true, 2>;
    else
        return softplus ? (chunks ? scan_fwd_k2s<T, 2, true, true, HAS_Z, HAS_OUT, true, 2>
                                  : scan_fwd_k2s<T, 2, true, false, HAS_Z, HAS_OUT, true, 2>)
                        : (chunks ? scan_fwd_k2s<T, 2, false, true, HAS_Z, HAS_OUT, true, 2>
                                  : scan_fwd_k2s<T, 2, false, false, HAS_Z, HAS_OUT, true, 2>);
}

// Segmented scan on k2s (L a multiple of 32): the states of segments 0 .. n_seg-2 (SEG 1), the
// carry chain, every segment with its outputs (SEG 2). Requests that write both out and out_z, and
// fp32 requests with chunk states, return MM_ERR_UNSUPPORTED before launching anything (the
// pipelined kernel's segments serve them).
template <typename T>
int launch_k2s_segmented(const mm_scan_fwd_params &p, hipStream_t stream, const SegArgs &sg) {
    const bool chunks = p.chunk_states != nullptr;
    if ((p.z && p.out) || (sizeof(T) == 4 && chunks) || p.tile_states) return MM_ERR_UNSUPPORTED;
    const K2SKernel states = p.delta_softplus ? scan_fwd_k2s<T, 2, true, false, false, false, false, 1>
                                              : scan_fwd_k2s<T, 2, false, false, false, false, false, 1>;
    const K2SKernel full = p.z ? k2s_seg_full<T, true, false>(p.delta_softplus, chunks)
                               : k2s_seg_full<T, false, true>(p.delta_softplus, chunks);
    const int64_t ratio = p.dim / p.n_groups;
    hipLaunchKernelGGL(states, dim3(unsigned(p.dim / kCh), unsigned(p.batch), unsigned(sg.n_seg - 1)), dim3(128), 0,
                       stream, p, ratio, sg);
    int rc = launch_status("scan_fwd_k2s_seg_states");
    if (rc != MM_OK) return rc;
    const int64_t rows = p.batch * p.dim;
    hipLaunchKernelGGL(seg_carry_kernel, dim3(unsigned((rows * 16 + 255) / 256)), dim3(256), 0, stream, p.A,
                       p.A_d_stride, p.A_dstate_stride, rows, p.dim, sg);
    rc = launch_status("seg_carry");
    if (rc != MM_OK) return rc;
    hipLaunchKernelGGL(full, dim3(unsigned(p.dim / kCh), unsigned(p.batch), unsigned(sg.n_seg)), dim3(128), 0, stream,
                       p, ratio, sg);
    return launch_status("scan_fwd_k2s_seg");
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

// Kernel choice for dstate 16: by default 16-bit inputs take k2s (L a multiple of 32) or k2i; fp32
// inputs take k2s for L a multiple of 32 without chunk or tile states (inference), else the
// pipelined k2. MM_SCAN_KERNEL in the environment selects "k2i" (two states per lane, per-element
// work alternating between the waves), "k2" / "k1" (two / one state per lane, alternating
// prologue/epilogue phases), or "nw1" / "nw2" / "nw4" (multi-state-per-lane kernel without
// pipelining, 1, 2 or 4 waves per group). MM_SCAN_PF (1, 2, 3; default 2) sets the load distance in
// 32-step tile pairs of k2 / k1 (k2i loads 2 pairs ahead).
static int tiled_variant() {
    static int v = [] {
        const char *e = getenv("MM_SCAN_KERNEL");
        if (!e) return 0;
        if (!strcmp(e, "k1")) return 10;
        if (!strcmp(e, "k2")) return 20;
        if (!strcmp(e, "k2i")) return 31;
        if (!strcmp(e, "nw1")) return 1;
        if (!strcmp(e, "nw2")) return 2;
        if (!strcmp(e, "nw4")) return 4;
        return 0;
    }();
    return v;
}

static int pipe_prefetch() {
    static int pf = [] {
        const char *e = getenv("MM_SCAN_PF");
        const int v = e ? atoi(e) : 2;
        return (v >= 1 && v <= 3) ? v : 2;
    }();
    return pf;
}

template <typename T, int K>
static int launch_pipe_pf(const mm_scan_fwd_params &p, hipStream_t stream) {
    switch (pipe_prefetch()) {
        case 1: return tiled::launch_pipe<T, K, 1>(p, stream);
        case 3: return tiled::launch_pipe<T, K, 3>(p, stream);
        default: return tiled::launch_pipe<T, K, 2>(p, stream);
    }
}

// Shape conditions of the dstate-16 kernels that do not depend on pointer alignment.
static bool tiled_shape_ok(const mm_scan_fwd_params &p) {
    if (p.dstate != 16 || !p.is_variable_B || !p.is_variable_C) return false;
    if (p.dim % tiled::kCh != 0 || (p.dim / p.n_groups) % tiled::kCh != 0) return false;
    return p.seqlen >= 8 && p.seqlen % 8 == 0 && p.batch <= 65535;
}

// The pipelined kernels address a 16-channel group with 32-bit element offsets from a per-group base.
static bool pipe_offsets_ok(const mm_scan_fwd_params &p) {
    const int64_t span = p.seqlen + 15 * std::max({p.u_d_stride, p.delta_d_stride, p.z_d_stride, p.out_d_stride,
                                                   p.out_z_d_stride, p.B_dstate_stride, p.C_dstate_stride});
    return span < (int64_t(1) << 31);
}

// k2s, k1s and k2i address a 16-channel group with 32-bit BYTE offsets from a per-group buffer base
// (lane offset + tile or pair offset): every byte they touch must lie below 2^32 from the base. For
// 16-bit inputs pipe_offsets_ok implies it; fp32 rows whose channel stride puts the group's span
// at or above 2^30 elements go to the pipelined kernel, which uses element offsets.
static bool k2s_bytes_ok(const mm_scan_fwd_params &p) {
    const int64_t span = p.seqlen + 15 * std::max({p.u_d_stride, p.delta_d_stride, p.z_d_stride, p.out_d_stride,
                                                   p.out_z_d_stride, p.B_dstate_stride, p.C_dstate_stride});
    const int64_t size = p.itype == MM_FLOAT32 ? 4 : 2;
    return span * size < (int64_t(1) << 32);
}

// Whether a segmented request runs on k2s: every 32-step pair whole, byte offsets in range, and
// neither a request that writes both out and out_z nor fp32 with chunk states (the pipelined
// kernel's segments serve those; MM_SCAN_KERNEL=k2 selects them always).
static bool k2s_segments_ok(const mm_scan_fwd_params &p) {
    return p.seqlen % (2 * tiled::kT1) == 0 && tiled_variant() != 20 && !(p.z && p.out) &&
           !(p.itype == MM_FLOAT32 && p.chunk_states) && k2s_bytes_ok(p);
}

#ifdef MM_TILED_COMMON
// SIMDs of the current device (4 per CU), or 1024 (the MI355X's) when it cannot be queried.
int64_t device_simds() {
    static std::atomic<int64_t> cache[64] = {};   // per device; every thread computes the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
    int64_t v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return 1024;
        v = 4 * int64_t(cus);
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Sequence segments for shapes whose (batch, 16-channel) groups give fewer than one wave per SIMD
// (two waves per group): enough segments for ~5 waves per SIMD in the full pass, each at least 512
// steps. Measured at config 3 (160 groups, L 65,536, fp32, k2s segments): 6, 8, 9, 10, 12, 15, 16,
// 19, 24 and 32 segments take 1.42, 1.44, 1.31, 1.48, 1.40, 1.29, 1.24, 1.24, 1.25 and 1.25 ms -- a
// full pass just past one round of workgroups (10, 12) or a few long segments at 2 waves per SIMD
// (6, 8) cost most, and from ~5 waves per SIMD on the time is flat. MM_SCAN_SEGMENTS=n sets the count
// (for measurements).
int64_t segment_count(const mm_scan_fwd_params &p) {
    if (!tiled_shape_ok(p) || !fwd_vector_ok(&p) || !pipe_offsets_ok(p) || p.tile_states) return 1;
    const int64_t waves = 2 * p.batch * (p.dim / tiled::kCh);
    const int64_t n_pairs = (p.seqlen + 2 * tiled::kT1 - 1) / (2 * tiled::kT1);
    int64_t n_seg;
    if (const char *e = std::getenv("MM_SCAN_SEGMENTS"); e && std::atoll(e) >= 1) {
        n_seg = std::min<int64_t>(std::atoll(e), n_pairs);
    } else {
        const int64_t simds = device_simds();
        if (waves >= simds) return 1;
        n_seg = std::min((5 * simds + waves - 1) / waves, n_pairs / 16);
    }
    if (n_seg < 2) return 1;
    const int64_t pairs = (n_pairs + n_seg - 1) / n_seg;
    return (n_pairs + pairs - 1) / pairs;   // every segment holds at least one pair
}

int64_t segment_workspace_bytes(const mm_scan_fwd_params &p, int64_t n_seg) {
    return n_seg > 1 ? p.batch * p.dim * n_seg * (16 + 2) * int64_t(sizeof(float)) : 0;
}

// Whether the diagonal forward can write tile_states for this request (the kernels below).
bool tile_states_ok(const mm_scan_fwd_params &p) {
    return tiled_shape_ok(p) && fwd_vector_ok(&p) && pipe_offsets_ok(p);
}
#endif  // MM_TILED_COMMON

// Balanced launch of one-pass inference requests (scan_fwd_mix): when the 16-channel groups give an
// odd number q in {3, 5} per compute unit, k2s alone would put 3 waves on half the SIMDs and 2 on
// the others (q = 5) or 2 and 1 (q = 3). The mixed grid runs (q - 1) / 2 two-group blocks and one
// one-group (k1s) block per CU instead, the same states on every SIMD. MM_SCAN_MIX=0 turns it off
// (for comparison).
static bool mix_plan(const mm_scan_fwd_params &p, int32_t &n_double, int32_t &n_single) {
    static const int mode = [] {   // 0: off, 1: default, 2: one-state groups only (q = 3)
        const char *e = getenv("MM_SCAN_MIX");
        if (!e) return 1;
        if (!strcmp(e, "0")) return 0;
        if (!strcmp(e, "k1")) return 2;
        return 1;
    }();
    // The training form (chunk and tile states) is built for 16-bit inputs only.
    if (mode == 0 || ((p.chunk_states || p.tile_states) && p.itype == MM_FLOAT32)) return false;
    const int64_t groups = p.batch * (p.dim / tiled::kCh);
    const int64_t cus = device_simds() / 4;
    if (cus <= 0 || groups % cus != 0) return false;
    const int64_t q = groups / cus;
    if (q != 3 && q != 5) return false;
    if (mode == 2 && q == 3) {
        n_double = 0;
        n_single = int32_t(3 * cus);
        return true;
    }
    n_double = int32_t((q / 2) * cus);
    n_single = int32_t(cus);
    return true;
}

// The two-states-per-lane kernels: k2s (symmetric element work, or the balanced mixed grid) when L
// is a multiple of 32 and the byte offsets fit, else k2i for 16-bit inputs (MM_SCAN_KERNEL=k2i
// selects k2i always, for comparison) and the pipelined kernel for fp32.
template <typename T>
static int launch_k2x(const mm_scan_fwd_params &p, hipStream_t stream) {
    static const bool nofull = getenv("MM_SCAN_NOFULL") != nullptr;
    const bool whole_pairs = p.seqlen % (2 * tiled::kT1) == 0 && !nofull && k2s_bytes_ok(p);
    int32_t n_double = 0, n_single = 0;
    if constexpr (sizeof(T) == 4) {
        // fp32: k2s for the inference requests it compiles for (no chunk or tile states), the
        // pipelined kernel for the rest.
        if (whole_pairs && !p.chunk_states && !p.tile_states) {
            if (mix_plan(p, n_double, n_single)) return tiled::launch_mix<T>(p, stream, n_double, n_single);
            return tiled::launch_k2s<T, 2>(p, stream);
        }
        return launch_pipe_pf<T, 2>(p, stream);
    } else {
        if (tiled_variant() != 31 && whole_pairs) {
            if (mix_plan(p, n_double, n_single)) return tiled::launch_mix<T>(p, stream, n_double, n_single);
            return tiled::launch_k2s<T, 2>(p, stream);
        }
        return tiled::launch_k2i<T, 2>(p, stream);
    }
}

template <typename T>
int try_launch_tiled(const mm_scan_fwd_params &p, hipStream_t stream) {
    if (!tiled_shape_ok(p) || !fwd_vector_ok(&p)) return MM_ERR_UNSUPPORTED;
    const bool pipe_ok = pipe_offsets_ok(p);
    if (p.tile_states) {
        // The backward's checkpoints are written by the default kernels only (one pass, no segments).
        if (!pipe_ok) return MM_ERR_UNSUPPORTED;
        if constexpr (std::is_same_v<T, float>) return launch_pipe_pf<T, 2>(p, stream);
        else return launch_k2x<T>(p, stream);
    }
    const int64_t n_seg = pipe_ok ? segment_count(p) : 1;
    if (n_seg > 1 && p.workspace && p.workspace_bytes >= segment_workspace_bytes(p, n_seg) &&
        (reinterpret_cast<uintptr_t>(p.workspace) & 15u) == 0) {
        const int64_t n_pairs = (p.seqlen + 2 * tiled::kT1 - 1) / (2 * tiled::kT1);
        const int64_t rows = p.batch * p.dim;
        float *ws = static_cast<float *>(p.workspace);
        const tiled::SegArgs sg{(n_pairs + n_seg - 1) / n_seg, int32_t(n_seg), ws, ws + rows * n_seg * 16,
                                ws + rows * n_seg * 17};
        if (k2s_segments_ok(p)) {
            const int rc = tiled::launch_k2s_segmented<T>(p, stream, sg);
            if (rc != MM_ERR_UNSUPPORTED) return rc;
        }
        return tiled::launch_pipe_segmented<T>(p, stream, sg);
    }
    switch (pipe_ok ? tiled_variant() : 2) {
        case 1: return tiled::launch_nw<T, 1>(p, stream);
        case 2: return tiled::launch_nw<T, 2>(p, stream);
        case 4: return tiled::launch_nw<T, 4>(p, stream);
        case 10: return launch_pipe_pf<T, 1>(p, stream);
        case 20: return launch_pipe_pf<T, 2>(p, stream);
        default: return launch_k2x<T>(p, stream);
    }
}


// The states-only forward the backward runs when no tile states were saved; MM_ERR_UNSUPPORTED
// (nothing launched) when the request falls outside the dstate-16 pipelined kernels. Inputs with L
// a multiple of 32 take k2s without outputs, others the pipelined kernel's MODE 3
// (MM_STATES_KERNEL=pipe selects it always, for comparison). Both compute the states with the
// same operations in the same order.
template <typename T>
int launch_states_only(const mm_scan_fwd_params &p, hipStream_t stream) {
    if (!p.tile_states || !tile_states_ok(p)) return MM_ERR_UNSUPPORTED;
    static const bool pipe = [] {
        const char *e = getenv("MM_STATES_KERNEL");
        return e && !strcmp(e, "pipe");
    }();
    if (!pipe && p.seqlen % (2 * tiled::kT1) == 0 && k2s_bytes_ok(p)) {
        int32_t n_double = 0, n_single = 0;
        if (!mix_plan(p, n_double, n_single)) n_double = n_single = 0;
        return tiled::launch_k2s_states<T>(p, stream, n_double, n_single);
    }
    return tiled::launch_fwd_states<T>(p, stream);
}
template int launch_states_only<MM_TILED_TYPE>(const mm_scan_fwd_params &, hipStream_t);
template int try_launch_tiled<MM_TILED_TYPE>(const mm_scan_fwd_params &, hipStream_t);

}  // namespace mm
