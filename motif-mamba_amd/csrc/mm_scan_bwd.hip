// mm_scan_bwd.hip -- gfx950 backward of the diagonal selective scan.
//
// Reference behaviour: selective_scan_cuda.bwd (csrc/selective_scan/selective_scan.cpp:415-612) and
// selective_scan_bwd_kernel (csrc/selective_scan/selective_scan_bwd_kernel.cuh:405-880): the
// gradients of u, delta, A, B, C, D, z and delta_bias for a gradient `dout` of the forward's output.
// Per (batch, channel) row and state n, with g_t = dout_t silu(z_t):
//
//   gh_t = C_t g_t + a_{t+1} gh_{t+1}                     (adjoint of h_t, a reverse scan)
//   dC_t += g_t h_t,  dB_t += gh_t dt_t u_t,  dA += gh_t dt_t (a_t h_{t-1}),
//   du_t = D g_t + dt_t sum_n gh_t B_t,  ddt_t = sum_n gh_t (u_t B_t + A (a_t h_{t-1})),
//
// with a_t h_{t-1} = h_t - dt_t u_t B_t. The reverse scan needs h_t again; this file's design:
// a first pass recomputes the forward states and stores them at every 16-step tile start in the
// caller's workspace, and the reverse pass recomputes each tile from its checkpoint (keeping the
// tile's states and decays in registers) and walks it backwards.
//
//   scan_bwd_tiled16<T, CARRY, CH>   dstate 16, variable B/C (the Mamba shape): CH channels (16
//       or 32) x 16 states per workgroup of 8 CH lanes, sums over states and over the block's
//       channels through LDS, dB/dC as per-block partials reduced by scan_bwd_reduce_bc (no
//       atomics on them).
//   scan_bwd_general<T>   any shape: a 256-lane workgroup holds 256/NP rows, one lane per state
//       (NP = next power of two >= dstate); sums over states go through LDS, sums over rows
//       (dB, dC, dA, dD, ddelta_bias) are float32 device atomics.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace bwd {

constexpr int kBT = 16;          // steps per checkpoint tile
constexpr int kGenThreads = 256;

// Zero up to 8 float32 tensors of up to 4 dimensions with arbitrary element strides, in one launch
// (the gradients a backward accumulates into).
struct FillSet {
    float *ptr[8];
    int64_t n[8][4], st[8][4];
    int count;
};
__global__ void __launch_bounds__(256) fill_zero_set(const FillSet fs) {
    for (int k = 0; k < fs.count; ++k) {
        const int64_t n1 = fs.n[k][1], n2 = fs.n[k][2], n3 = fs.n[k][3];
        const int64_t total = fs.n[k][0] * n1 * n2 * n3;
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
            int64_t r = i;
            const int64_t i3 = r % n3; r /= n3;
            const int64_t i2 = r % n2; r /= n2;
            const int64_t i1 = r % n1; r /= n1;
            fs.ptr[k][r * fs.st[k][0] + i1 * fs.st[k][1] + i2 * fs.st[k][2] + i3 * fs.st[k][3]] = 0.f;
        }
    }
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + expf(-x)); }

template <typename T>
__global__ void __launch_bounds__(kGenThreads)
scan_bwd_general(const mm_scan_bwd_params p, const int64_t ratio, const int np_log2, float *const partB,
                 float *const partC) {
    __shared__ float sDu[kBT * kGenThreads];   // [step][lane]: per-state partials of sum_n gh B
    __shared__ float sDdt[kBT * kGenThreads];  // [step][lane]: per-state partials of ddt
    __shared__ float sB[kBT * kGenThreads];    // [step][lane]: variable dB terms of the tile
    __shared__ float sC[kBT * kGenThreads];    // [step][lane]: variable dC terms of the tile
    const int NP = 1 << np_log2;
    const int tid = threadIdx.x;
    const int slot = tid >> np_log2;
    const int n = tid & (NP - 1);
    const int N = int(p.dstate);
    const int64_t rows = p.batch * p.dim;
    const int64_t r = int64_t(blockIdx.x) * (kGenThreads >> np_log2) + slot;
    const bool row_ok = r < rows;
    const int64_t rr = row_ok ? r : rows - 1;       // clamped for loads; stores are predicated
    const int64_t b = rr / p.dim;
    const int64_t d = rr - b * p.dim;
    const int64_t g = d / ratio;
    const bool on = row_ok && n < N;
    const int nn = n < N ? n : N - 1;
    const int64_t L = p.seqlen;
    const int64_t n_tiles = (L + kBT - 1) / kBT;

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    const T *outp = p.z ? reinterpret_cast<const T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    const T *gop = reinterpret_cast<const T *>(p.dout) + b * p.dout_batch_stride + d * p.dout_d_stride;
    T *dup = reinterpret_cast<T *>(p.du) + b * p.du_batch_stride + d * p.du_d_stride;
    T *ddp = reinterpret_cast<T *>(p.ddelta) + b * p.ddelta_batch_stride + d * p.ddelta_d_stride;
    T *dzp = p.z ? reinterpret_cast<T *>(p.dz) + b * p.dz_batch_stride + d * p.dz_d_stride : nullptr;
    T *ozp = (p.z && p.out_z) ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    const T *Bv = p.is_variable_B ? reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride + nn * p.B_dstate_stride : nullptr;
    const T *Cv = p.is_variable_C ? reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride + nn * p.C_dstate_stride : nullptr;
    float *dBv = p.is_variable_B ? p.dB + b * p.dB_batch_stride + g * p.dB_group_stride + nn * p.dB_dstate_stride : nullptr;
    float *dCv = p.is_variable_C ? p.dC + b * p.dC_batch_stride + g * p.dC_group_stride + nn * p.dC_dstate_stride : nullptr;
    const float Bc = p.is_variable_B ? 0.f : reinterpret_cast<const float *>(p.B)[d * p.B_d_stride + nn * p.B_dstate_stride];
    const float Cc = p.is_variable_C ? 0.f : reinterpret_cast<const float *>(p.C)[d * p.C_d_stride + nn * p.C_dstate_stride];
    const float An = p.A[d * p.A_d_stride + nn * p.A_dstate_stride];
    const float A2 = An * kLog2e;
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    float *ck = reinterpret_cast<float *>(p.workspace) + rr * n_tiles * N;

    auto dt_at = [&](int64_t t, float &raw) {
        raw = to_f32(dp[t]) + bias;
        return p.delta_softplus ? softplus_fast(raw) : raw;
    };
    auto b_at = [&](int64_t t) { return Bv ? to_f32(Bv[t]) : Bc; };
    auto c_at = [&](int64_t t) { return Cv ? to_f32(Cv[t]) : Cc; };
    // g_t = dout_t silu(z_t) (or dout_t); the lane of state 0 also writes dz_t (and out_z_t).
    auto g_at = [&](int64_t t, bool writer) {
        float go = to_f32(gop[t]);
        if (zp) {
            const float zz = to_f32(zp[t]);
            const float sg = sigmoid_f32(zz);
            if (writer) {
                const float o = to_f32(outp[t]);
                dzp[t] = from_f32<T>(go * o * sg * (1.f + zz * (1.f - sg)));
                if (ozp) ozp[t] = from_f32<T>(o * zz * sg);
            }
            go *= zz * sg;
        }
        return go;
    };

    // Pass 1: the forward states at every tile start.
    float h = 0.f;
    for (int64_t t = 0; t < L; ++t) {
        if (t % kBT == 0 && on) ck[(t / kBT) * N + n] = h;
        float raw;
        const float dt = dt_at(t, raw);
        h = __builtin_fmaf(decay_exp2(dt, A2), h, dt * to_f32(up[t]) * b_at(t));
    }
    __syncthreads();  // orders this lane's checkpoint stores before its reloads (same lane, global memory)

    // Pass 2: tiles in reverse order.
    float gh = 0.f, a_next = 0.f, dA_acc = 0.f, dBc = 0.f, dCc = 0.f, dD_acc = 0.f, dbias_acc = 0.f;
    for (int64_t j = n_tiles - 1; j >= 0; --j) {
        const int64_t t0 = j * kBT;
        const int cnt = int(L - t0 < kBT ? L - t0 : kBT);
        float hs[kBT], as[kBT], dts[kBT], us[kBT];
        float hh = on ? ck[j * N + n] : 0.f;
        float dA_tile = 0.f, dB_tile = 0.f, dC_tile = 0.f;  // per-tile partial sums (shorter chains)
#pragma unroll
        for (int s = 0; s < kBT; ++s) {
            if (s < cnt) {
                float raw;
                const int64_t t = t0 + s;
                dts[s] = dt_at(t, raw);
                us[s] = to_f32(up[t]);
                as[s] = decay_exp2(dts[s], A2);
                hh = __builtin_fmaf(as[s], hh, dts[s] * us[s] * b_at(t));
                hs[s] = hh;
            }
        }
#pragma unroll
        for (int s = kBT - 1; s >= 0; --s) {
            float du_part = 0.f, ddt_part = 0.f;
            if (s < cnt) {
                const int64_t t = t0 + s;
                const float gt = g_at(t, row_ok && n == 0);
                const float bn = b_at(t);
                const float dtu = dts[s] * us[s];
                gh = __builtin_fmaf(c_at(t), gt, a_next * gh);
                const float ah = hs[s] - dtu * bn;        // a_t h_{t-1}
                const float dcv = gt * hs[s];
                const float dbv = gh * dtu;
                sB[s * kGenThreads + tid] = dbv;
                sC[s * kGenThreads + tid] = dcv;
                dC_tile += dcv;
                dB_tile += dbv;
                du_part = gh * bn;
                ddt_part = gh * __builtin_fmaf(An, ah, us[s] * bn);
                dA_tile = __builtin_fmaf(gh * dts[s], ah, dA_tile);
                a_next = as[s];
            }
            sDu[s * kGenThreads + tid] = on ? du_part : 0.f;
            sDdt[s * kGenThreads + tid] = on ? ddt_part : 0.f;
        }
        dA_acc += dA_tile;
        dBc += dB_tile;
        dCc += dC_tile;
        __syncthreads();
        // The variable dB / dC of the tile: per (step, state), the terms of consecutive rows of one
        // (batch, group) added in row order -- into this workgroup's slab when there is one (its
        // rows are then all of one (batch, group)), else one float32 atomic per such run.
        if (partB || partC) {
            const int rpb = kGenThreads >> np_log2;
            const int64_t row0 = int64_t(blockIdx.x) * rpb;
            const int64_t b0 = row0 / p.dim, d0 = row0 - b0 * p.dim, g0 = d0 / ratio;
            const int64_t blk = (d0 - g0 * ratio) / rpb;
            float *const slabB = partB ? partB + ((blk * p.batch + b0) * p.n_groups + g0) * N * L : nullptr;
            float *const slabC = partC ? partC + ((blk * p.batch + b0) * p.n_groups + g0) * N * L : nullptr;
            for (int e = tid; e < kBT * NP; e += kGenThreads) {
                const int se = e >> np_log2, ne = e & (NP - 1);
                if (se >= cnt || ne >= N) continue;
                float accB = 0.f, accC = 0.f;
                for (int sl = 0; sl < rpb; ++sl) {
                    accB += sB[se * kGenThreads + sl * NP + ne];
                    accC += sC[se * kGenThreads + sl * NP + ne];
                }
                if (slabB) slabB[ne * L + t0 + se] = accB;
                if (slabC) slabC[ne * L + t0 + se] = accC;
            }
        } else if (dBv || dCv) {
            const int rpb = kGenThreads >> np_log2;
            const int64_t row0 = int64_t(blockIdx.x) * rpb;
            for (int e = tid; e < kBT * NP; e += kGenThreads) {
                const int se = e >> np_log2, ne = e & (NP - 1);
                if (se >= cnt || ne >= N) continue;
                const int64_t t = t0 + se;
                float accB = 0.f, accC = 0.f;
                int64_t key = -1, kb = 0, kg = 0;
                auto flush = [&]() {
                    if (key < 0) return;
                    if (dBv) atomicAdd(p.dB + kb * p.dB_batch_stride + kg * p.dB_group_stride + ne * p.dB_dstate_stride + t, accB);
                    if (dCv) atomicAdd(p.dC + kb * p.dC_batch_stride + kg * p.dC_group_stride + ne * p.dC_dstate_stride + t, accC);
                };
                for (int sl = 0; sl < rpb; ++sl) {
                    const int64_t rw = row0 + sl;
                    if (rw >= rows) break;
                    const int64_t bw = rw / p.dim, gw = (rw - bw * p.dim) / ratio;
                    const int64_t kw = bw * p.n_groups + gw;
                    if (kw != key) {
                        flush();
                        key = kw; kb = bw; kg = gw; accB = 0.f; accC = 0.f;
                    }
                    accB += sB[se * kGenThreads + sl * NP + ne];
                    accC += sC[se * kGenThreads + sl * NP + ne];
                }
                flush();
            }
        }
        // Per step: sums over the row's states; the lane of state s % NP finishes step s.
        float dD_tile = 0.f, dbias_tile = 0.f;
        for (int s = n; s < cnt; s += NP) {
            float su = 0.f, sd = 0.f;
            for (int k = 0; k < N; ++k) {
                su += sDu[s * kGenThreads + slot * NP + k];
                sd += sDdt[s * kGenThreads + slot * NP + k];
            }
            if (row_ok) {
                const int64_t t = t0 + s;
                float raw;
                const float dt = dt_at(t, raw);
                const float gt = g_at(t, false);
                const float uu = to_f32(up[t]);
                const float dd = (p.delta_softplus && raw <= 20.f) ? sd * sigmoid_f32(raw) : sd;
                dup[t] = from_f32<T>(__builtin_fmaf(Dv, gt, dt * su));
                ddp[t] = from_f32<T>(dd);
                dD_tile = __builtin_fmaf(gt, uu, dD_tile);
                dbias_tile += dd;
            }
        }
        dD_acc += dD_tile;
        dbias_acc += dbias_tile;
        __syncthreads();
    }
    if (on) {
        atomicAdd(p.dA + d * p.dA_d_stride + n * p.dA_dstate_stride, dA_acc);
        if (!p.is_variable_B) atomicAdd(p.dB + d * p.dB_d_stride + n * p.dB_dstate_stride, dBc);
        if (!p.is_variable_C) atomicAdd(p.dC + d * p.dC_d_stride + n * p.dC_dstate_stride, dCc);
    }
    if (row_ok && n < kBT) {
        if (p.dD) atomicAdd(p.dD + d, dD_acc);
        if (p.ddelta_bias) atomicAdd(p.ddelta_bias + d, dbias_acc);
    }
}


// ------------------------------------------------------------------------------------------------
// dstate-16 backward: a workgroup of 8 CH lanes owns CH channels x 16 states of one (batch, group)
// -- lane (slot rs = lane / CH, channel c = lane % CH) holds states 2 rs and 2 rs + 1 of channel c.
// Per 16-step tile: the lane owning steps 2 rs, 2 rs + 1 of channel c computes dt', dt'u, u and
// g = dout silu(z) (and writes dz) into LDS; B and C of the tile are staged in LDS as float32; the
// tile is recomputed from its checkpoint with states and decays kept in registers, then walked
// backwards in two halves of 8 steps. Per half, the dB/dC contributions (per state, step and
// channel) go to LDS and are summed over the CH channels, the sums written as this channel block's
// partials (reduced over blocks by scan_bwd_reduce_bc, in a fixed order); the per-slot partial sums
// over states of gh B and of the delta' derivative go to LDS and the owner of each step adds the 8
// slots in order and finishes du and ddelta.
// ------------------------------------------------------------------------------------------------
constexpr int kFT = 16;          // steps per tile
constexpr int kFH = 8;           // steps per reduction half
constexpr int kPS = 8;           // step stride (floats) of sPart rows
constexpr int kXS = kFT + 1;     // step stride (float4) of sX rows
constexpr int kBufs = 1;         // sX / sBC buffers (one: 4 workgroups fit a CU's LDS)
// sBC row stride (floats): B 16 | C 16 | 2 pad. 34 (2 mod 32 banks) puts the four step rows that
// one 32-lane staging store touches on disjoint banks; the 8-byte reads stay aligned.
constexpr int kBCS = 34;

// sRed address of (tensor, state n, step t of the half, channel c) for CH channels per workgroup:
// a block of 8 rows of CH channels per (tensor, state). Rows are CH + 4 floats apart (CH = 16: 20),
// so that the 8 consecutive steps of one state that 8 lanes read as 16-byte pieces in the reduction
// fall in distinct 16-byte bank groups; blocks are an odd multiple of 8 such groups apart (CH = 16:
// 168 floats, 8 mod 16 banks), which puts the next state's 8 steps in the other groups.
template <int CH> constexpr int kRedRow = CH + 4;
template <int CH> constexpr int kRedBlock = CH == 16 ? 168 : 288;
template <int CH>
__device__ __forceinline__ int red_at(int tensor, int n, int t, int c) {
    return (tensor * 16 + n) * kRedBlock<CH> + t * kRedRow<CH> + c;
}
template <int CH> constexpr int kRedFloats = 32 * kRedBlock<CH>;

// The per-slot state sums: the two slots a wave holds per channel (lanes l and l + 32 of the wave,
// slots rs and rs ^ kPairBit) are added before the LDS exchange, with one v_permlane32_swap per
// step: the lower lane ends with the pair's gh B sum, the upper lane with its ddt sum. Each lane
// then stores one value per step instead of two, and the owners add 4 pair sums instead of 8
// slot sums.
#ifndef MM_BWD_PAIR_SUMS
#define MM_BWD_PAIR_SUMS 1
#endif
constexpr bool kPairSums = MM_BWD_PAIR_SUMS != 0;
template <int CH> constexpr int kPairBit = 32 / CH;             // slot bit that lane bit 5 carries
template <int CH> constexpr int kPartSlots = kPairSums ? 4 : 8;  // sPart rows per tensor and channel

// Lower half of the wave: pu + the upper lane's pu; upper half: the lower lane's pd + pd.
__device__ __forceinline__ float pair_sum(float pu, float pd) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(pu), __float_as_uint(pd), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
static_assert((kFH - 1) * kRedRow<16> + 16 <= kRedBlock<16>, "sRed rows overlap");
static_assert((kFH - 1) * kRedRow<32> + 32 <= kRedBlock<32>, "sRed rows overlap");

template <typename T>
__device__ __forceinline__ void unpack2(const RawVec<T, 2> &r, float &a, float &b) {
    float o[2];
    unpack_raw<T, 2>(r, o);
    a = o[0];
    b = o[1];
}

template <typename T>
__device__ __forceinline__ void store2(T *p, float a, float b) {
    const float x[2] = {a, b};
    store_vec<T, 2>(p, x);
}

struct FastWs {
    float *ck;      // [n_tiles][batch][dim][16]: states before each tile
    float *partB;   // [block][batch][group][16][L]: dB summed over one 16-channel block
    float *partC;
    // State split (dstate a multiple of 16 above 16: one launch sequence per 16 states): the sums
    // over states of gh B and of the delta' term, float32 [batch][dim][L], carried from part to
    // part. part 0: no split; 1: the first part (stores its sums); 2: a middle part (adds its
    // own); 3: the last part (adds the carried sums to its own and finishes du, ddelta, dD and
    // ddelta_bias, which the other parts leave alone).
    float *acc_su = nullptr;
    float *acc_sd = nullptr;
    int part = 0;
};

// Sequence segments. A launch covers the units (batch row, CH-channel block) unit0, unit0 + 1, ...
// (unit = b * dim / CH + d0 / CH), each as n_seg segments of seg_tiles tiles. With n_seg > 1 the
// CARRY launch walks segments 1 .. n_seg-1 of each unit from a zero adjoint and stores, per channel
// and state, (a_t0 gh_t0, prod of a over the segment): the adjoint the segment hands to the one
// before it, and the factor that carries a later adjoint through it. The gradient launch then
// starts each segment from the combination of those of the segments after it.
//
// The CARRY launch also reduces the dB/dC slab rows that the whole-row launch before it completed:
// its workgroups past carry_blocks sum rows [0, red_rows) of both slabs over their n_blocks channel
// blocks, memory-bound work beside the carries' latency-bound walks.
struct BwdSeg {
    int64_t unit0;
    int64_t n_seg;
    int64_t seg_tiles;
    float2 *carry;      // [unit - unit0][n_seg * csplit][CH channels][16 states]
    int64_t csplit;     // carry pieces per segment
    int64_t carry_blocks, red_rows, n_blocks;
};

// dB or dC rows [row0, row1) (row = (b * n_groups + g) * 16 + n), by workgroup wg of n_wg, each of
// NTH lanes: an element is four steps of a row, the sum of its n_blocks channel-block partials. The
// blocks are split into K contiguous ranges summed by separate lanes (with K > 1 a short row range
// still keeps enough loads in flight), each range in block order, and the range sums added in range
// order through `scratch` (NTH float4, unused with K = 1). Each element is reduced by one call, whose
// K the plan fixes, so the result is deterministic.
constexpr int kRedChunks = 8;
// The row stride (floats) of the partial slabs: L rounded up to whole float4s.
__host__ __device__ __forceinline__ int64_t slab_row(int64_t L) { return (L + 3) & ~int64_t(3); }
template <int NTH, int K>
__device__ __forceinline__ void reduce_slab_rows(const mm_scan_bwd_params &p, const float *part, float *dst,
                                                 int64_t bs, int64_t gs, int64_t ns, int64_t n_blocks, int64_t row0,
                                                 int64_t row1, int64_t wg, int64_t n_wg, float4 *scratch) {
    constexpr int E = NTH / K;   // elements per workgroup pass
    const int tid = threadIdx.x, e = tid % E, k = tid / E;
    const int64_t Lp = slab_row(p.seqlen), L4 = Lp / 4;
    const int64_t st = p.batch * p.n_groups * 16 * L4;   // one block's slab, in float4
    const int64_t b_lo = n_blocks * k / K, b_hi = n_blocks * (k + 1) / K;
    const int64_t end = row1 * L4;
    for (int64_t base = row0 * L4 + wg * E; base < end; base += n_wg * E) {   // uniform over the workgroup
        const int64_t i = base + e;
        const int64_t row = i / L4, t4 = i - row * L4;
        // Slab rows past dstate (P/Q with dstate < 16) are not written.
        const bool live = i < end && row % 16 < p.dstate;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) {
            const float4 *src = reinterpret_cast<const float4 *>(part + row * Lp) + t4;
            int64_t blk = b_lo;
            for (; blk + 8 <= b_hi; blk += 8) {   // eight loads in flight, added in block order
                float4 v[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = src[(blk + q) * st];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    acc.x += v[q].x; acc.y += v[q].y; acc.z += v[q].z; acc.w += v[q].w;
                }
            }
            for (; blk < b_hi; ++blk) {
                const float4 v = src[blk * st];
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
        }
        if constexpr (K > 1) {
            scratch[k * E + e] = acc;
            __syncthreads();
        }
        if (k == 0 && live) {
#pragma unroll
            for (int kk = 1; kk < K; ++kk) {
                const float4 v = scratch[kk * E + e];
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
            const int64_t n = row % 16, bg = row / 16;
            const int64_t gg = bg % p.n_groups, bb = bg / p.n_groups;
            float *o = dst + bb * bs + gg * gs + n * ns + 4 * t4;
            const float a4[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)   // the row's last float4 may reach past L (L % 4 = 2)
                if (4 * t4 + q < p.seqlen) o[q] = a4[q];
        }
        if constexpr (K > 1) __syncthreads();   // scratch reads done before the next pass rewrites it
    }
}

// B/C staging of one tile: the first kStageLanes<CH> lanes each load kStageVals<CH> consecutive steps
// of one state of B (first half of them) or C (second half): 2 x 16 states x 16 steps in all.
template <int CH> constexpr int kStageLanes = 8 * CH < 256 ? 8 * CH : 256;
template <int CH> constexpr int kStageVals = 512 / kStageLanes<CH>;

// Global data of one tile for one lane, loaded a tile ahead of its use.
template <typename T, int CH>
struct TileRaw {
    RawVec<T, 2> d, u, go, z, o;             // this lane's two steps of one channel
    RawVec<T, 2> bc[kStageVals<CH> / 2];     // B or C values of one state (staging lanes)
    float2 hc;                               // checkpoint of the lane's two states (pass 2)
};

// CH channels (16 or 32) x 16 states per workgroup of 8 CH lanes.
// SPLIT: a part of a state-split request (FastWs::part 1-3); its own instance, so that the whole
// requests' kernel carries none of the split's code.
template <typename T, bool CARRY, int CH, bool SPLIT = false>
__global__ void __launch_bounds__(8 * CH)
scan_bwd_tiled16(const mm_scan_bwd_params p, const int64_t ratio, const FastWs ws, const BwdSeg sg) {
    constexpr int NT = 8 * CH;
    constexpr int SL = kStageLanes<CH>, SV = kStageVals<CH>;
    __shared__ __align__(16) float4 sX[kBufs][CH * kXS];       // [buf][c][t]: (dt', dt'u, u, g)
    __shared__ __align__(16) float sBC[kBufs][kFT * kBCS];      // [buf][t][B 16 | C 16 | pad]
    __shared__ __align__(16) float sRed[kRedFloats<CH>];        // red_at<CH>(tensor, n, t, c)
    __shared__ __align__(16) float sPart[kPartSlots<CH> * 2 * CH * kPS];   // [slot (pair)][gh B | ddt][c][t]

    const int tid = threadIdx.x;
    if constexpr (CARRY) {
        if (int64_t(blockIdx.x) >= sg.carry_blocks) {   // a slab-reduction workgroup: one lane per element
            const int64_t wg = int64_t(blockIdx.x) - sg.carry_blocks, n_wg = int64_t(gridDim.x) - sg.carry_blocks;
            reduce_slab_rows<NT, 1>(p, ws.partB, p.dB, p.dB_batch_stride, p.dB_group_stride, p.dB_dstate_stride,
                                    sg.n_blocks, 0, sg.red_rows, wg, n_wg, nullptr);
            reduce_slab_rows<NT, 1>(p, ws.partC, p.dC, p.dC_batch_stride, p.dC_group_stride, p.dC_dstate_stride,
                                    sg.n_blocks, 0, sg.red_rows, wg, n_wg, nullptr);
            return;
        }
    }
    const int rs = tid / CH;               // state slot: states 2 rs, 2 rs + 1; prologue steps 2 rs, 2 rs + 1
    const int c = tid % CH;                // channel within the block
    const int n0 = 2 * rs;
    const int pswz = (c >> 2) & 3;         // sPart step-pair permutation of this channel
    // The CARRY launch walks segments 1 .. n_seg-1 (segment 0 hands nothing on), each as csplit
    // pieces: piece cs is part cs % csplit of segment cs / csplit.
    const int64_t nsw = CARRY ? (sg.n_seg - 1) * sg.csplit : sg.n_seg;
    const int64_t uo = int64_t(blockIdx.x) / nsw;
    const int64_t seg = int64_t(blockIdx.x) - uo * nsw + (CARRY ? sg.csplit : 0);   // CARRY: the piece cs
    const int64_t per_b = p.dim / CH;
    const int64_t b = (sg.unit0 + uo) / per_b;
    const int64_t d0 = (sg.unit0 + uo - b * per_b) * CH;
    const int64_t d = d0 + c;
    const int64_t g = d0 / ratio;
    const int64_t blk = (d0 - g * ratio) / CH;
    const int64_t L = p.seqlen;
    const int64_t Lp = slab_row(L);
    const int64_t n_tiles = (L + kFT - 1) / kFT;
    int64_t j_lo = seg * sg.seg_tiles;
    int64_t j_hi = j_lo + sg.seg_tiles < n_tiles ? j_lo + sg.seg_tiles : n_tiles;
    if constexpr (CARRY) {   // the tiles of piece seg (empty when the segment is short)
        const int64_t s_lo = (seg / sg.csplit) * sg.seg_tiles;
        const int64_t s_hi = s_lo + sg.seg_tiles < n_tiles ? s_lo + sg.seg_tiles : n_tiles;
        const int64_t piece = (sg.seg_tiles + sg.csplit - 1) / sg.csplit;
        j_lo = std::min(s_lo + (seg % sg.csplit) * piece, s_hi);
        j_hi = std::min(j_lo + piece, s_hi);
    }

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    const T *outp = p.z ? reinterpret_cast<const T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    const T *gop = reinterpret_cast<const T *>(p.dout) + b * p.dout_batch_stride + d * p.dout_d_stride;
    T *dup = reinterpret_cast<T *>(p.du) + b * p.du_batch_stride + d * p.du_d_stride;
    T *ddp = reinterpret_cast<T *>(p.ddelta) + b * p.ddelta_batch_stride + d * p.ddelta_d_stride;
    T *dzp = p.z ? reinterpret_cast<T *>(p.dz) + b * p.dz_batch_stride + d * p.dz_d_stride : nullptr;
    T *ozp = (p.z && p.out_z) ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    // B/C staging (lanes tid < SL): lane -> tensor tid / (SL / 2), state, steps SV q .. SV q + SV - 1.
    const bool stager = tid < SL;
    const int st_li = tid % (SL / 2);
    const int st_tensor = (tid / (SL / 2)) & 1, st_n = st_li / (16 / SV), st_q = st_li % (16 / SV);
    const T *stp = st_tensor == 0
        ? reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride + st_n * p.B_dstate_stride
        : reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride + st_n * p.C_dstate_stride;
    float *ckp = ws.ck + (b * p.dim + d) * 16 + n0;
    const int64_t ck_tile = p.batch * p.dim * 16;

    const float A0 = p.A[d * p.A_d_stride + n0 * p.A_dstate_stride];
    const float A1 = p.A[d * p.A_d_stride + (n0 + 1) * p.A_dstate_stride];
    const float A20 = A0 * kLog2e, A21 = A1 * kLog2e;
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;

    // Loads of tile j (clamped into the row: always in bounds). Steps past L are padding, made
    // inert in commit(): dt' = g = 0 and B = C = 0 leave every state and gradient unchanged.
    // The carry walk (CARRY) reads only delta', g and C: it loads neither u, the pre-gate out, B
    // nor the checkpoint (their registers stay zero).
    auto load = [&](int64_t j, bool full) {
        TileRaw<T, CH> r;
        const int64_t jj = j < 0 ? 0 : (j >= n_tiles ? n_tiles - 1 : j);
        const int64_t te = jj * kFT + 2 * rs;
        const int64_t tl = te < L ? te : L - 2;
        r.d = load_raw<T, 2>(dp + tl);
        r.u = {};
        if constexpr (!CARRY) r.u = load_raw<T, 2>(up + tl);
        r.go = {};
        r.z = {};
        r.o = {};
        if (full) {
            r.go = load_raw<T, 2>(gop + tl);
            if (zp) {
                r.z = load_raw<T, 2>(zp + tl);
                if constexpr (!CARRY) r.o = load_raw<T, 2>(outp + tl);
            }
        }
        const int64_t ts0 = jj * kFT + SV * st_q;
#pragma unroll
        for (int i = 0; i < SV / 2; ++i) r.bc[i] = {};
        if (stager && (CARRY ? st_tensor == 1 : (full || st_tensor == 0))) {
#pragma unroll
            for (int i = 0; i < SV / 2; ++i) {   // each step pair clamped into the row on its own
                const int64_t ts = ts0 + 2 * i < L ? ts0 + 2 * i : L - 2;
                r.bc[i] = load_raw<T, 2>(stp + ts);
            }
        }
        r.hc = (full && !CARRY) ? *reinterpret_cast<const float2 *>(ckp + jj * ck_tile) : make_float2(0.f, 0.f);
        return r;
    };
    // Tile j's per-step values into LDS buffer `buf`; the lane's own steps kept for the epilogue;
    // dz (and out_z) written.
    float e_raw[2], e_dt[2], e_u[2], e_g[2];
    auto commit = [&](const TileRaw<T, CH> &r, int64_t j, int buf, bool full) {
        const int64_t te = j * kFT + 2 * rs;
        const bool ev = te < L;            // L is even: both steps exist or neither
        float dd[2], go[2] = {0.f, 0.f};
        unpack2<T>(r.d, dd[0], dd[1]);
        unpack2<T>(r.u, e_u[0], e_u[1]);
        if (full) {
            unpack2<T>(r.go, go[0], go[1]);
            if (zp) {
                float zz[2], oo[2], dz[2], oz[2];
                unpack2<T>(r.z, zz[0], zz[1]);
                unpack2<T>(r.o, oo[0], oo[1]);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-zz[i] * kLog2e));
                    dz[i] = go[i] * oo[i] * sg * (1.f + zz[i] * (1.f - sg));
                    oz[i] = oo[i] * zz[i] * sg;
                    go[i] *= zz[i] * sg;
                }
                if (ev && !CARRY) {
                    store2(dzp + te, dz[0], dz[1]);
                    if (ozp) store2(ozp + te, oz[0], oz[1]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            e_raw[i] = dd[i] + bias;
            e_dt[i] = ev ? (p.delta_softplus ? softplus_fast(e_raw[i]) : e_raw[i]) : 0.f;
            e_g[i] = ev ? go[i] : 0.f;
            sX[buf][c * kXS + 2 * rs + i] = make_float4(e_dt[i], e_dt[i] * e_u[i], e_u[i], e_g[i]);
        }
        if (stager) {
            float v[SV];
#pragma unroll
            for (int i = 0; i < SV / 2; ++i) unpack2<T>(r.bc[i], v[2 * i], v[2 * i + 1]);
#pragma unroll
            for (int i = 0; i < SV; ++i) {   // L is even: a step pair exists whole or not at all
                const bool bv_ok = j * kFT + SV * st_q + (i & ~1) < L;
                sBC[buf][(SV * st_q + i) * kBCS + st_tensor * 16 + st_n] = bv_ok ? v[i] : 0.f;
            }
        }
    };

    if constexpr (CARRY) {
        // The segment's adjoint from a zero carry, gh_t = C_t g_t + a_{t+1} gh_{t+1}, and the
        // product of its decays. Steps past L (last segment only) have dt' = g = 0: a = 1, inert.
        float gh0 = 0.f, gh1 = 0.f, an0 = 0.f, an1 = 0.f, pa0 = 1.f, pa1 = 1.f;
        TileRaw<T, CH> nx = load(j_hi - 1, true);
        for (int64_t j = j_hi - 1; j >= j_lo; --j) {
            commit(nx, j, 0, true);
            nx = load(j - 1, true);
            __syncthreads();
#pragma unroll
            for (int t = kFT - 1; t >= 0; --t) {
                const float4 x = sX[0][c * kXS + t];
                const float2 cv = *reinterpret_cast<const float2 *>(&sBC[0][t * kBCS + 16 + n0]);
                gh0 = __builtin_fmaf(an0, gh0, x.w * cv.x);
                gh1 = __builtin_fmaf(an1, gh1, x.w * cv.y);
                an0 = decay_exp2(x.x, A20);
                an1 = decay_exp2(x.x, A21);
                pa0 *= an0;
                pa1 *= an1;
            }
            __syncthreads();   // reads done before the next commit rewrites the buffer
        }
        float4 *cp = reinterpret_cast<float4 *>(sg.carry + ((uo * sg.n_seg * sg.csplit + seg) * CH + c) * 16 + n0);
        *cp = make_float4(an0 * gh0, pa0, an1 * gh1, pa1);
        return;
    }

    // Pass 1: the states before every tile, into the checkpoint workspace (skipped when the
    // forward wrote them: ws.ck then points at its tile_states; segmented launches always have them).
    float h0 = 0.f, h1 = 0.f;
    TileRaw<T, CH> nxt = load(0, false);
    for (int64_t j = 0; j < (p.tile_states ? 0 : n_tiles); ++j) {
        const int buf = int(j % kBufs);
        *reinterpret_cast<float2 *>(ckp + j * ck_tile) = make_float2(h0, h1);
        commit(nxt, j, buf, false);
        nxt = load(j + 1, false);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < kFT; ++t) {
            const float4 x = sX[buf][c * kXS + t];
            const float2 bv = *reinterpret_cast<const float2 *>(&sBC[buf][t * kBCS + n0]);
            h0 = __builtin_fmaf(decay_exp2(x.x, A20), h0, x.y * bv.x);
            h1 = __builtin_fmaf(decay_exp2(x.x, A21), h1, x.y * bv.y);
        }
        if (kBufs == 1) __syncthreads();   // reads done before the next commit rewrites the buffer
    }
    __syncthreads();   // the checkpoints stored above are read back by this lane only

    // Pass 2: tiles in reverse order.
    float gh0 = 0.f, gh1 = 0.f, an0 = 0.f, an1 = 0.f;   // state adjoints, decays of the step after
    if (seg + 1 < sg.n_seg) {
        // The adjoint entering from the later segments: c_{S-1} = 0, c_{s-1} = e_s + P_s c_s.
        // Pieces compose like segments (c entering a piece = e + P c leaving it), so the carry is
        // the same chain over the pieces of the later segments.
        const float4 *cp =
            reinterpret_cast<const float4 *>(sg.carry + ((uo * sg.n_seg * sg.csplit) * CH + c) * 16 + n0);
        float c0 = 0.f, c1 = 0.f;
        for (int64_t s2 = sg.n_seg * sg.csplit - 1; s2 >= (seg + 1) * sg.csplit; --s2) {
            const float4 v = cp[s2 * CH * 8];   // one piece: CH channels x 16 states x (e, P)
            c0 = __builtin_fmaf(v.y, c0, v.x);
            c1 = __builtin_fmaf(v.w, c1, v.z);
        }
        gh0 = c0;
        gh1 = c1;
        an0 = 1.f;
        an1 = 1.f;
    }
    float dA0 = 0.f, dA1 = 0.f, dD_acc = 0.f, dbias_acc = 0.f;
    // Two tiles in flight: the loads of tile j - 2 are issued once tile j is committed. The two ring
    // entries keep their registers (the loop is unrolled by two below): a copy of an entry whose
    // loads are still in flight would wait for them.
    TileRaw<T, CH> ra = load(j_hi - 1, true), rb = load(j_hi - 2, true);
    auto tile = [&](const int64_t j, TileRaw<T, CH> &cur) {
        const int64_t t0 = j * kFT;
        const int buf = int(j % kBufs);
        const float2 hc = cur.hc;
        commit(cur, j, buf, true);
        cur = load(j - 2, true);
        __syncthreads();
        float hs0[kFT], hs1[kFT], as0[kFT], as1[kFT];
        {
            float x0 = hc.x, x1 = hc.y;
#pragma unroll
            for (int t = 0; t < kFT; ++t) {
                const float4 x = sX[buf][c * kXS + t];
                const float2 bv = *reinterpret_cast<const float2 *>(&sBC[buf][t * kBCS + n0]);
                as0[t] = decay_exp2(x.x, A20);
                as1[t] = decay_exp2(x.x, A21);
                x0 = __builtin_fmaf(as0[t], x0, x.y * bv.x);
                x1 = __builtin_fmaf(as1[t], x1, x.y * bv.y);
                hs0[t] = x0;
                hs1[t] = x1;
            }
        }
#pragma unroll
        for (int half = 1; half >= 0; --half) {
            float pu[kFH], pd[kFH];
            float dA_t0 = 0.f, dA_t1 = 0.f;
#pragma unroll
            for (int s = kFH - 1; s >= 0; --s) {
                const int t = half * kFH + s;
                const float4 x = sX[buf][c * kXS + t];     // dt', dt'u, u, g
                const float2 bv = *reinterpret_cast<const float2 *>(&sBC[buf][t * kBCS + n0]);
                const float2 cv = *reinterpret_cast<const float2 *>(&sBC[buf][t * kBCS + 16 + n0]);
                gh0 = __builtin_fmaf(an0, gh0, x.w * cv.x);
                gh1 = __builtin_fmaf(an1, gh1, x.w * cv.y);
                const float ah0 = __builtin_fmaf(-x.y, bv.x, hs0[t]);   // a_t h_{t-1}
                const float ah1 = __builtin_fmaf(-x.y, bv.y, hs1[t]);
                sRed[red_at<CH>(0, n0, s, c)] = gh0 * x.y;          // dB contributions
                sRed[red_at<CH>(0, n0 + 1, s, c)] = gh1 * x.y;
                sRed[red_at<CH>(1, n0, s, c)] = x.w * hs0[t];       // dC contributions
                sRed[red_at<CH>(1, n0 + 1, s, c)] = x.w * hs1[t];
                // sum_n gh (u B + A a h_{t-1}) = u sum_n gh B + sum_n A (gh a h_{t-1}); the products
                // gh a h_{t-1} also give dA.
                const float w0 = gh0 * ah0, w1 = gh1 * ah1;
                pu[s] = __builtin_fmaf(gh1, bv.y, gh0 * bv.x);
                pd[s] = __builtin_fmaf(x.z, pu[s], __builtin_fmaf(A1, w1, A0 * w0));
                dA_t0 = __builtin_fmaf(x.x, w0, dA_t0);
                dA_t1 = __builtin_fmaf(x.x, w1, dA_t1);
                an0 = as0[t];
                an1 = as1[t];
            }
            dA0 += dA_t0;
            dA1 += dA_t1;
            // sPart rows hold 4 step pairs; pair q of channel c sits at pair position q ^ pswz, so
            // that 16 consecutive channels (what one 64-bit LDS cycle serves) hit 16 distinct bank
            // pairs, for these stores and for the owners' reads below (8-float rows alone put 4
            // channels on each).
            if constexpr (kPairSums) {
                // Pair index of the slot pair (rs, rs ^ kPairBit), 0 .. 3; the lower lane writes the
                // gh B row, the upper lane the ddt row.
                constexpr int PB = kPairBit<CH>;
                const int pi = (rs & (PB - 1)) | ((rs >> 1) & ~(PB - 1));
                const int tz = (rs & PB) ? 1 : 0;
                float2 *pw = reinterpret_cast<float2 *>(&sPart[((pi * 2 + tz) * CH + c) * kPS]);
#pragma unroll
                for (int q = 0; q < kFH / 2; ++q)
                    pw[q ^ pswz] = make_float2(pair_sum(pu[2 * q], pd[2 * q]), pair_sum(pu[2 * q + 1], pd[2 * q + 1]));
            } else {
                float2 *pp = reinterpret_cast<float2 *>(&sPart[((rs * 2 + 0) * CH + c) * kPS]);
                float2 *pq = reinterpret_cast<float2 *>(&sPart[((rs * 2 + 1) * CH + c) * kPS]);
#pragma unroll
                for (int q = 0; q < kFH / 2; ++q) {
                    pp[q ^ pswz] = make_float2(pu[2 * q], pu[2 * q + 1]);
                    pq[q ^ pswz] = make_float2(pd[2 * q], pd[2 * q + 1]);
                }
            }
            __syncthreads();
            // dB / dC of this half summed over the block's CH channels: the 256 rows (tensor, state,
            // step), step fastest, one per lane (two per lane with 128 lanes; lanes past 256 idle),
            // so consecutive lanes read consecutive steps.
            constexpr int kRowsPerLane = NT >= 256 ? 1 : 256 / NT;
#pragma unroll
            for (int k = 0; k < kRowsPerLane; ++k) {
                const int row = tid + NT * k;
                if (NT > 256 && row >= 256) break;
                const int tz = row >> 7, tn = (row >> 3) & 15, tt = row & 7;
                const float4 *rv = reinterpret_cast<const float4 *>(&sRed[red_at<CH>(tz, tn, tt, 0)]);
                float q4[CH / 4];
#pragma unroll
                for (int q = 0; q < CH / 4; ++q) {   // pairwise: short dependency chains, fixed order
                    const float4 v = rv[q];
                    q4[q] = (v.x + v.y) + (v.z + v.w);
                }
#pragma unroll
                for (int w = 1; w < CH / 4; w *= 2) {
#pragma unroll
                    for (int q = 0; q < CH / 4; q += 2 * w) q4[q] += q4[q + w];
                }
                const float acc = q4[0];
                const int64_t ts = t0 + half * kFH + tt;
                if (ts < L)
                    (tz == 0 ? ws.partB : ws.partC)[(((blk * p.batch + b) * p.n_groups + g) * 16 + tn) * Lp + ts] = acc;
            }
            // du / ddelta of the steps this lane owns, if they are in this half: the partial sums
            // over states of the 4 slot pairs (or 8 slots), added in order.
            if ((rs >> 2) == half) {
                const int sl = 2 * (rs & 3);               // first owned step within the half
                const int64_t te = t0 + 2 * rs;
                float su[2] = {0.f, 0.f}, sd[2] = {0.f, 0.f};
#pragma unroll
                for (int k = 0; k < kPartSlots<CH>; ++k) {
                    const int pos = 2 * ((sl >> 1) ^ pswz);
                    const float2 a = *reinterpret_cast<const float2 *>(&sPart[((k * 2 + 0) * CH + c) * kPS + pos]);
                    const float2 bq = *reinterpret_cast<const float2 *>(&sPart[((k * 2 + 1) * CH + c) * kPS + pos]);
                    su[0] += a.x; su[1] += a.y;
                    sd[0] += bq.x; sd[1] += bq.y;
                }
                if (SPLIT && te < L) {   // state split: carry the sums over states
                    float2 *const asu = reinterpret_cast<float2 *>(ws.acc_su + (b * p.dim + d) * L + te);
                    float2 *const asd = reinterpret_cast<float2 *>(ws.acc_sd + (b * p.dim + d) * L + te);
                    if (ws.part != 1) {
                        const float2 x = *asu, y = *asd;
                        su[0] = x.x + su[0]; su[1] = x.y + su[1];
                        sd[0] = y.x + sd[0]; sd[1] = y.y + sd[1];
                    }
                    if (ws.part != 3) {
                        *asu = make_float2(su[0], su[1]);
                        *asd = make_float2(sd[0], sd[1]);
                    }
                }
                if (te < L && (!SPLIT || ws.part == 3)) {
                    float du[2], ddl[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        du[i] = __builtin_fmaf(Dv, e_g[i], e_dt[i] * su[i]);
                        const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-e_raw[i] * kLog2e));
                        ddl[i] = (p.delta_softplus && e_raw[i] <= 20.f) ? sd[i] * sg : sd[i];
                        dD_acc = __builtin_fmaf(e_g[i], e_u[i], dD_acc);
                        dbias_acc += ddl[i];
                    }
                    store2(dup + te, du[0], du[1]);
                    store2(ddp + te, ddl[0], ddl[1]);
                }
            }
            __syncthreads();
        }
    };
    for (int64_t j = j_hi - 1; j >= j_lo; j -= 2) {
        tile(j, ra);
        if (j - 1 >= j_lo) tile(j - 1, rb);
    }
    atomicAdd(p.dA + d * p.dA_d_stride + n0 * p.dA_dstate_stride, dA0);
    atomicAdd(p.dA + d * p.dA_d_stride + (n0 + 1) * p.dA_dstate_stride, dA1);
    if (p.dD) atomicAdd(p.dD + d, dD_acc);
    if (p.ddelta_bias) atomicAdd(p.ddelta_bias + d, dbias_acc);
}

// dB and dC rows [row0, rows) = the sums of the channel blocks' partials, in a fixed order.
__global__ void __launch_bounds__(256)
scan_bwd_reduce_bc(const mm_scan_bwd_params p, const float *partB, const float *partC, int64_t n_blocks,
                   int64_t row0, int64_t rows) {
    __shared__ float4 scratch[256];
    reduce_slab_rows<256, kRedChunks>(p, partB, p.dB, p.dB_batch_stride, p.dB_group_stride, p.dB_dstate_stride,
                                      n_blocks, row0, rows, blockIdx.x, gridDim.x, scratch);
    reduce_slab_rows<256, kRedChunks>(p, partC, p.dC, p.dC_batch_stride, p.dC_group_stride, p.dC_dstate_stride,
                                      n_blocks, row0, rows, blockIdx.x, gridDim.x, scratch);
}

// dB / dC from the general kernels' slabs [block][batch][group][dstate][seqlen]: each element the
// sum of its n_blocks partials in block order.
__global__ void __launch_bounds__(256)
gen_slab_reduce(const mm_scan_bwd_params p, const float *partB, const float *partC, int64_t n_blocks) {
    const int64_t L = p.seqlen, N = p.dstate;
    const int64_t total = p.batch * p.n_groups * N * L;
    for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t t = e % L, n = (e / L) % N, bg = e / (L * N);
        const int64_t b = bg / p.n_groups, g = bg % p.n_groups;
        if (partB) {
            float acc = 0.f;
            for (int64_t k = 0; k < n_blocks; ++k) acc += partB[k * total + e];
            p.dB[b * p.dB_batch_stride + g * p.dB_group_stride + n * p.dB_dstate_stride + t] = acc;
        }
        if (partC) {
            float acc = 0.f;
            for (int64_t k = 0; k < n_blocks; ++k) acc += partC[k * total + e];
            p.dC[b * p.dC_batch_stride + g * p.dC_group_stride + n * p.dC_dstate_stride + t] = acc;
        }
    }
}

int gen_rows_per_block(const mm_scan_bwd_params &p) {
    int np_log2 = 0;
    while ((1 << np_log2) < p.dstate) ++np_log2;
    return kGenThreads >> np_log2;
}

template <typename T>
int launch_general(const mm_scan_bwd_params &p, hipStream_t s) {
    int np_log2 = 0;
    while ((1 << np_log2) < p.dstate) ++np_log2;
    const int64_t rows_per_block = kGenThreads >> np_log2;
    const int64_t rows = p.batch * p.dim;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    if (blocks >= (int64_t(1) << 32) / kGenThreads)   // gridDim.x * blockDim.x must stay below 2^32
        return set_error(MM_ERR_UNSUPPORTED, "mm_scan_bwd: batch * dim too large for one launch of the general kernel");
    // Workspace: the checkpoints, then the dB / dC slabs when this shape has them.
    const int64_t n_tiles = (p.seqlen + kBT - 1) / kBT;
    float *const ws = static_cast<float *>(p.workspace);
    const int64_t slab = gen_slab_floats(p, rows_per_block);
    float *const partB = slab && p.is_variable_B ? ws + rows * n_tiles * p.dstate : nullptr;
    float *const partC = slab && p.is_variable_C ? ws + rows * n_tiles * p.dstate + slab : nullptr;
    const dim3 grid(static_cast<unsigned>(blocks));
    hipLaunchKernelGGL((scan_bwd_general<T>), grid, dim3(kGenThreads), 0, s, p, p.dim / p.n_groups, np_log2, partB,
                       partC);
    const int rc = launch_status("scan_bwd_general");
    if (rc != MM_OK || !slab) return rc;
    return launch_gen_slab_reduce(p, s, partB, partC, rows_per_block);
}

// Tensors to zero, collected and cleared by one launch of fill_zero_set.
struct Fills {
    FillSet fs{};
    int64_t largest = 0;
    void add(float *ptr, int64_t n0, int64_t n1, int64_t n2, int64_t n3, int64_t s0, int64_t s1, int64_t s2,
             int64_t s3) {
        const int64_t total = n0 * n1 * n2 * n3;
        if (!ptr || total == 0) return;
        const int k = fs.count++;
        fs.ptr[k] = ptr;
        const int64_t n[4] = {n0, n1, n2, n3}, st[4] = {s0, s1, s2, s3};
        for (int i = 0; i < 4; ++i) {
            fs.n[k][i] = n[i];
            fs.st[k][i] = st[i];
        }
        largest = std::max(largest, total);
    }
    int launch(hipStream_t s) const {
        if (fs.count == 0) return MM_OK;
        const int64_t blocks = std::min<int64_t>((largest + 255) / 256, 4096);
        hipLaunchKernelGGL(fill_zero_set, dim3(unsigned(blocks)), dim3(256), 0, s, fs);
        return launch_status("fill_zero_set");
    }
};

// The dstate-16 kernel's requirements: variable B/C, 16-channel blocks inside one group, L even,
// two-element-aligned activation and B/C rows (each lane moves step pairs).
bool fast_ok(const mm_scan_bwd_params &p) {
    if (p.P || p.dstate != 16 || !p.is_variable_B || !p.is_variable_C) return false;
    if (p.dim % 16 != 0 || (p.dim / p.n_groups) % 16 != 0 || p.seqlen < 2 || p.seqlen % 2 != 0) return false;
    // One 128-lane workgroup per unit in a 1-D grid: gridDim.x * blockDim.x must stay below 2^32.
    if (p.batch * (p.dim / 16) >= (int64_t(1) << 25)) return false;
    const int64_t eb = p.itype == MM_FLOAT32 ? 4 : 2;
    auto al = [](const void *ptr, int64_t bytes) { return (reinterpret_cast<uintptr_t>(ptr) % uintptr_t(bytes)) == 0; };
    auto row2 = [&](const void *ptr, int64_t s0, int64_t s1) {
        return ptr == nullptr || (al(ptr, 2 * eb) && s0 % 2 == 0 && s1 % 2 == 0);
    };
    bool ok = row2(p.u, p.u_batch_stride, p.u_d_stride) && row2(p.delta, p.delta_batch_stride, p.delta_d_stride) &&
              row2(p.z, p.z_batch_stride, p.z_d_stride) && row2(p.out, p.out_batch_stride, p.out_d_stride) &&
              row2(p.dout, p.dout_batch_stride, p.dout_d_stride) && row2(p.du, p.du_batch_stride, p.du_d_stride) &&
              row2(p.ddelta, p.ddelta_batch_stride, p.ddelta_d_stride) && row2(p.dz, p.dz_batch_stride, p.dz_d_stride) &&
              row2(p.out_z, p.out_z_batch_stride, p.out_z_d_stride);
    ok = ok && al(p.B, 2 * eb) && al(p.C, 2 * eb) && p.B_batch_stride % 2 == 0 && p.B_group_stride % 2 == 0 &&
         p.B_dstate_stride % 2 == 0 && p.C_batch_stride % 2 == 0 && p.C_group_stride % 2 == 0 &&
         p.C_dstate_stride % 2 == 0;
    return ok;
}

int64_t fast_ck_floats(const mm_scan_bwd_params &p) {
    return ((p.seqlen + kFT - 1) / kFT) * p.batch * p.dim * 16;
}
int64_t fast_part_floats(const mm_scan_bwd_params &p) {
    return (p.dim / 16) * p.batch * 16 * slab_row(p.seqlen);   // blocks per group x groups = dim / 16
}

// Workgroups of scan_bwd_tiled16<T, false, CH> that the current device runs at once (one round), or
// 0 when the device cannot be queried. MM_BWD_SLOTS overrides it (tests exercise the segmented tail
// with it).
template <typename T, int CH>
int64_t round_slots() {
    if (const char *e = std::getenv("MM_BWD_SLOTS")) {
        const long long v = std::atoll(e);
        if (v > 0) return v;
    }
    static std::atomic<int64_t> cache[64] = {};   // per device; every thread computes the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int64_t v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, scan_bwd_tiled16<T, false, CH>, 8 * CH, 0) !=
            hipSuccess)
            return 0;
        v = int64_t(cus) * per_cu;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}
template <typename T>
int64_t round_slots_ch(int ch) {
    return ch == 32 ? round_slots<T, 32>() : round_slots<T, 16>();
}

// Channels per workgroup. Every workgroup writes its own dB/dC partial slab (16 x L floats per
// tensor and batch row), which the reduction reads back, so wider workgroups move fewer bytes: at
// the Mamba-2.8B layer shape the 16-channel slabs (670 MB) exceed the 256 MB Infinity Cache. 32
// channels are taken when the group's channels divide into 32-channel blocks and those fill at
// least one whole round (two 32-channel workgroups share a CU where four 16-channel ones do, and
// a partial round of them costs more); otherwise 16. MM_BWD_CH=16/32 forces a width the group
// allows.
template <typename T>
int pick_ch(const mm_scan_bwd_params &p) {
    const int64_t ratio = p.dim / p.n_groups;
    if (const char *e = std::getenv("MM_BWD_CH")) {
        const int v = std::atoi(e);
        if ((v == 16 || v == 32) && ratio % v == 0) return v;
    }
    if (ratio % 32 == 0) {
        const int64_t slots = round_slots_ch<T>(32);
        if (slots > 0 && p.batch * (p.dim / 32) >= slots) return 32;
    }
    return 16;
}

// How the dstate-16 backward covers its units. The kernel is latency-bound, so a last round with
// few workgroups per CU costs nearly as much as a full one. With the forward's tile states the
// units of that last round (or all of them, when they fill at most half a round) are instead cut
// along the sequence into n_seg segments, enough to fill a round, joined by a carry pass.
// A unit is (batch row, block of ch channels).
struct SegPlan {
    int64_t main_units, tail_units, n_seg, seg_tiles;
    int ch;
    int64_t csplit;   // carry pieces per segment (more, shorter carry walks)
};
template <typename T>
SegPlan seg_plan(const mm_scan_bwd_params &p) {
    const int ch = pick_ch<T>(p);
    const int64_t units = p.batch * (p.dim / ch);
    const int64_t n_tiles = (p.seqlen + kFT - 1) / kFT;
    const SegPlan whole{units, 0, 1, n_tiles, ch, 1};
    const char *off = std::getenv("MM_BWD_SEGMENTS");
    if (!p.tile_states || (off && off[0] == '0')) return whole;
    const int64_t slots = round_slots_ch<T>(ch);
    if (slots <= 0 || units == 0) return whole;
    const int64_t tail = units % slots;
    if (tail == 0) return whole;
    int64_t n_seg = std::min<int64_t>({slots / tail, 8, n_tiles / 4});
    if (n_seg < 2) return whole;
    const int64_t seg_tiles = (n_tiles + n_seg - 1) / n_seg;
    n_seg = (n_tiles + seg_tiles - 1) / seg_tiles;   // every segment holds at least one tile
    if (n_seg < 2) return whole;
    // Two carry pieces per segment halve the carry launch's walk (config 2: 1.535 -> 1.505 ms; three
    // or four pieces, more workgroups than one round holds, measured 1.53 and 1.52).
    // MM_BWD_CARRY_SPLIT=n sets the count (tests cover uneven and empty pieces with it).
    int64_t csplit = seg_tiles >= 8 ? 2 : 1;
    if (const char *e = std::getenv("MM_BWD_CARRY_SPLIT")) {
        const long long v = std::atoll(e);
        if (v >= 1 && v <= 8) csplit = v;
    }
    return {units - tail, tail, n_seg, seg_tiles, ch, csplit};
}
SegPlan seg_plan_for(const mm_scan_bwd_params &p) {
    if (p.itype == MM_FLOAT32) return seg_plan<float>(p);
    if (p.itype == MM_FLOAT16) return seg_plan<f16_t>(p);
    return seg_plan<bf16_t>(p);
}
int64_t carry_floats(const SegPlan &pl) { return pl.tail_units * pl.n_seg * pl.csplit * pl.ch * 16 * 2; }

// The forward parameter block of the states-only pass the backward runs when no tile states were
// handed to it: the scan's inputs, no outputs, tile_states = the checkpoint region `ck`.
mm_scan_fwd_params states_params(const mm_scan_bwd_params &p, float *ck) {
    mm_scan_fwd_params f;
    memset(&f, 0, sizeof(f));
    f.batch = p.batch; f.dim = p.dim; f.seqlen = p.seqlen; f.dstate = p.dstate; f.n_groups = p.n_groups;
    f.itype = p.itype;
    f.is_variable_B = p.is_variable_B; f.is_variable_C = p.is_variable_C; f.delta_softplus = p.delta_softplus;
    f.u = p.u; f.delta = p.delta; f.A = p.A; f.B = p.B; f.C = p.C; f.delta_bias = p.delta_bias;
    f.u_batch_stride = p.u_batch_stride; f.u_d_stride = p.u_d_stride;
    f.delta_batch_stride = p.delta_batch_stride; f.delta_d_stride = p.delta_d_stride;
    f.A_d_stride = p.A_d_stride; f.A_dstate_stride = p.A_dstate_stride;
    f.B_batch_stride = p.B_batch_stride; f.B_group_stride = p.B_group_stride;
    f.B_dstate_stride = p.B_dstate_stride; f.B_d_stride = p.B_d_stride;
    f.C_batch_stride = p.C_batch_stride; f.C_group_stride = p.C_group_stride;
    f.C_dstate_stride = p.C_dstate_stride; f.C_d_stride = p.C_d_stride;
    f.tile_states = ck;
    return f;
}


// Whether `p` (no tile states handed in) is better served by a states-only forward first: only
// when that forward can write the checkpoints (the dstate-16 pipelined kernel's shape and alignment
// conditions) and the backward, given them, would cut its last round into sequence segments.
// Otherwise the backward's own first pass computes the same states at the same cost.
// MM_BWD_STATES_PASS=0 turns the states pass off (for measurements).
bool states_pass_ok(const mm_scan_bwd_params &p) {
    static const bool off = [] {
        const char *e = std::getenv("MM_BWD_STATES_PASS");
        return e && e[0] == '0';
    }();
    if (off || p.tile_states || p.P) return false;
    float dummy;
    if (!tile_states_ok(states_params(p, &dummy))) return false;
    mm_scan_bwd_params q = p;
    q.tile_states = &dummy;
    return seg_plan_for(q).tail_units > 0;
}

// dB and dC rows [row0, row1): the n_blocks channel-block partials of each element summed in a
// fixed order, one launch.
int launch_reduce(const mm_scan_bwd_params &p, hipStream_t s, const float *partB, const float *partC,
                  int64_t n_blocks, int64_t row0, int64_t row1) {
    const int64_t total = (row1 - row0) * (slab_row(p.seqlen) / 4);
    if (total <= 0) return MM_OK;
    constexpr int64_t per_wg = 256 / kRedChunks;   // elements per workgroup pass
    const unsigned blocks = unsigned(std::min<int64_t>((total + per_wg - 1) / per_wg, 8192));
    hipLaunchKernelGGL(scan_bwd_reduce_bc, dim3(blocks), dim3(256), 0, s, p, partB, partC, n_blocks, row0, row1);
    return launch_status("scan_bwd_reduce_bc");
}

// The launches of the dstate-16 kernel with CH channels per workgroup: the whole rows of the full
// rounds, then (segmented tail) the carries and every segment of the cut units. *red_rows returns
// the dB/dC slab rows already reduced (by the carry launch): those of the (batch, group) pairs whose
// units all ran in the whole-row launch.
template <typename T, int CH, bool SPLIT>
int launch_units(const mm_scan_bwd_params &p, hipStream_t s, int64_t ratio, const FastWs &fw, const SegPlan &pl,
                 float *carry, int64_t *red_rows) {
    int rc = MM_OK;
    *red_rows = 0;
    if (pl.main_units > 0) {
        hipLaunchKernelGGL((scan_bwd_tiled16<T, false, CH, SPLIT>), dim3(unsigned(pl.main_units)), dim3(8 * CH), 0, s, p,
                           ratio, fw, BwdSeg{0, 1, (p.seqlen + kFT - 1) / kFT, nullptr, 1, 0, 0, 0});
        rc = launch_status("scan_bwd_tiled16");
        if (rc != MM_OK) return rc;
    }
    if (pl.tail_units > 0) {
        // Units run (batch, group)-major: the pairs below main_units / (blocks per group) are complete.
        // (Measured at config 2: this beats a separate reduction launch before or after the carries.)
        const int64_t rows = pl.main_units / (ratio / CH) * 16;
        const int64_t carry_blocks = pl.tail_units * (pl.n_seg - 1) * pl.csplit;
        const int64_t red_blocks = std::min<int64_t>((rows * (slab_row(p.seqlen) / 4) + 8 * CH - 1) / (8 * CH), 8192);
        const BwdSeg sg{pl.main_units, pl.n_seg, pl.seg_tiles, reinterpret_cast<float2 *>(carry), pl.csplit,
                        carry_blocks, rows, ratio / CH};
        hipLaunchKernelGGL((scan_bwd_tiled16<T, true, CH>), dim3(unsigned(carry_blocks + red_blocks)), dim3(8 * CH),
                           0, s, p, ratio, fw, sg);
        rc = launch_status("scan_bwd_tiled16 (carries)");
        if (rc != MM_OK) return rc;
        *red_rows = rows;
        hipLaunchKernelGGL((scan_bwd_tiled16<T, false, CH, SPLIT>), dim3(unsigned(pl.tail_units * pl.n_seg)), dim3(8 * CH),
                           0, s, p, ratio, fw, sg);
        rc = launch_status("scan_bwd_tiled16 (segments)");
    }
    return rc;
}

template <typename T>
int launch_fast(const mm_scan_bwd_params &p_in, hipStream_t s, float *acc_su = nullptr, float *acc_sd = nullptr,
                int part = 0) {
    float *ws = static_cast<float *>(p_in.workspace);
    const bool own_ck = p_in.tile_states == nullptr;
    float *ck = own_ck ? ws : const_cast<float *>(p_in.tile_states);
    float *partB = own_ck ? ws + fast_ck_floats(p_in) : ws;
    const FastWs fw{ck, partB, partB + fast_part_floats(p_in), acc_su, acc_sd, part};
    const int64_t ratio = p_in.dim / p_in.n_groups;
    // Without the forward's tile states, a states-only forward writes them into the head of the
    // workspace first (the same states the backward's own first pass would compute, from a kernel
    // that runs the whole grid at the forward's occupancy); the backward then reads them, as it
    // reads a training forward's, and may cut its last round into sequence segments.
    mm_scan_bwd_params p = p_in;
    if (own_ck && states_pass_ok(p_in)) {
        const mm_scan_fwd_params f = states_params(p_in, ck);
        const int rc = launch_states_only<T>(f, s);
        if (rc != MM_OK) return rc;
        p.tile_states = ck;
    }
    SegPlan pl = seg_plan<T>(p);
    const int64_t need = ((own_ck ? fast_ck_floats(p) : 0) + 2 * fast_part_floats(p) + carry_floats(pl)) *
                         int64_t(sizeof(float));
    // A workspace without room for the segment carries (sized by bwd_workspace_min_bytes, or queried
    // under another round size: MM_BWD_SLOTS or another device) runs every unit as a whole row.
    if (pl.tail_units > 0 && p.workspace_bytes < need)
        pl = {pl.main_units + pl.tail_units, 0, 1, (p.seqlen + kFT - 1) / kFT, pl.ch, 1};
    int64_t red_rows = 0;
    float *const carry = partB + 2 * fast_part_floats(p);
    const int rc = part != 0 ? (pl.ch == 32 ? launch_units<T, 32, true>(p, s, ratio, fw, pl, carry, &red_rows)
                                            : launch_units<T, 16, true>(p, s, ratio, fw, pl, carry, &red_rows))
                             : (pl.ch == 32 ? launch_units<T, 32, false>(p, s, ratio, fw, pl, carry, &red_rows)
                                            : launch_units<T, 16, false>(p, s, ratio, fw, pl, carry, &red_rows));
    if (rc != MM_OK) return rc;
    return launch_reduce(p, s, fw.partB, fw.partC, ratio / pl.ch, red_rows, p.batch * p.n_groups * 16);
}

// State split: a diagonal request with dstate a multiple of 16 above 16 (the Mamba presets with
// d_state 32 and 64) is the dstate-16 backward of each group of 16 states -- the recurrences of
// different states are independent; only du and ddelta sum over all states, which the parts carry
// in float32 (FastWs::acc_su / acc_sd) and the last part finishes. Part k sees A, B, C, dA, dB
// and dC from state 16 k on. MM_BWD_SPLIT=0 keeps such requests on the general kernel.
mm_scan_bwd_params split_part(const mm_scan_bwd_params &p, int k) {
    mm_scan_bwd_params q = p;
    const int64_t n0 = 16 * int64_t(k);
    const int64_t eb = p.itype == MM_FLOAT32 ? 4 : 2;
    q.dstate = 16;
    q.A = p.A + n0 * p.A_dstate_stride;
    q.B = p.is_variable_B ? static_cast<const void *>(static_cast<const char *>(p.B) + n0 * p.B_dstate_stride * eb)
                          : static_cast<const void *>(static_cast<const float *>(p.B) + n0 * p.B_dstate_stride);
    q.C = p.is_variable_C ? static_cast<const void *>(static_cast<const char *>(p.C) + n0 * p.C_dstate_stride * eb)
                          : static_cast<const void *>(static_cast<const float *>(p.C) + n0 * p.C_dstate_stride);
    q.dA = p.dA + n0 * p.dA_dstate_stride;
    q.dB = p.dB + n0 * p.dB_dstate_stride;
    q.dC = p.dC + n0 * p.dC_dstate_stride;
    return q;
}
bool split_ok(const mm_scan_bwd_params &p) {
    if (p.P || p.dstate <= 16 || p.dstate % 16 != 0 || p.tile_states || p.seqlen == 0) return false;
    const char *e = std::getenv("MM_BWD_SPLIT");
    if (e && e[0] == '0') return false;
    return fast_ok(split_part(p, 0));
}
int64_t split_acc_floats(const mm_scan_bwd_params &p) { return 2 * p.batch * p.dim * p.seqlen; }

template <typename T>
int launch_split(const mm_scan_bwd_params &p, hipStream_t s) {
    const int parts = int(p.dstate / 16);
    mm_scan_bwd_params q0 = split_part(p, 0);
    const int64_t part_bytes = bwd_workspace_bytes(q0);
    float *const acc = reinterpret_cast<float *>(static_cast<char *>(p.workspace) + ((part_bytes + 255) & ~int64_t(255)));
    float *const acc_su = acc, *const acc_sd = acc + p.batch * p.dim * p.seqlen;
    for (int k = 0; k < parts; ++k) {
        mm_scan_bwd_params q = split_part(p, k);
        q.workspace_bytes = (part_bytes + 255) & ~int64_t(255);
        const int part = k == 0 ? 1 : (k == parts - 1 ? 3 : 2);
        const int rc = launch_fast<T>(q, s, acc_su, acc_sd, part);
        if (rc != MM_OK) return rc;
    }
    return MM_OK;
}

// The P/Q backward (mm_scan_pq_bwd.hip) with the dB / dC block partials reduced in block order.
template <typename T>
int launch_pq(const mm_scan_bwd_params &p, hipStream_t s) {
    if (!pq_bwd_ok(p)) {   // the general P/Q backward: checkpoints, then the dB / dC slabs if any
        float *const ck = static_cast<float *>(p.workspace);
        const int64_t rpb = pq_general_rows_per_block(p), slab = gen_slab_floats(p, rpb);
        float *const partB = slab && p.is_variable_B ? ck + pq_general_ck_floats(p) : nullptr;
        float *const partC = slab && p.is_variable_C ? ck + pq_general_ck_floats(p) + slab : nullptr;
        const int rc = launch_pq_general<T>(p, s, ck, partB, partC);
        if (rc != MM_OK || !slab) return rc;
        return launch_gen_slab_reduce(p, s, partB, partC, rpb);
    }
    // Checkpoints: the forward's tile_states when given, else the head of the workspace.
    float *ws = static_cast<float *>(p.workspace);
    float *ck = p.tile_states ? const_cast<float *>(p.tile_states) : ws;
    float *partB = p.tile_states ? ws : ws + fast_ck_floats(p), *partC = partB + fast_part_floats(p);
    const int rc = launch_pq_bwd<T>(p, s, ck, partB, partC);
    if (rc != MM_OK) return rc;
    // Slab rows past dstate are never written; the reduction reads only rows n < 16 of each slab
    // and writes rows n < dstate (dB / dC hold dstate rows).
    return launch_reduce(p, s, partB, partC, p.dim / p.n_groups / 16, 0, p.batch * p.n_groups * 16);
}

}  // namespace bwd

int64_t gen_slab_floats(const mm_scan_bwd_params &p, int64_t rpb) {
    if (!p.is_variable_B && !p.is_variable_C) return 0;
    if (p.n_groups < 1 || p.dim % p.n_groups || (p.dim / p.n_groups) % rpb) return 0;
    const int64_t floats = (p.dim / rpb) * p.batch * p.dstate * p.seqlen;
    return 2 * floats * int64_t(sizeof(float)) <= (int64_t(1) << 32) ? floats : 0;
}

int launch_gen_slab_reduce(const mm_scan_bwd_params &p, hipStream_t s, const float *partB, const float *partC,
                           int64_t rpb) {
    const int64_t total = p.batch * p.n_groups * p.dstate * p.seqlen;
    if (total <= 0) return MM_OK;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 255) / 256, 16384));
    hipLaunchKernelGGL(bwd::gen_slab_reduce, dim3(blocks), dim3(256), 0, s, p, partB, partC,
                       p.dim / p.n_groups / rpb);
    return launch_status("gen_slab_reduce");
}

int64_t bwd_workspace_bytes(const mm_scan_bwd_params &p) {
    if (bwd::split_ok(p))   // one part's workspace (reused by every part), then the carried sums
        return ((bwd_workspace_bytes(bwd::split_part(p, 0)) + 255) & ~int64_t(255)) +
               bwd::split_acc_floats(p) * int64_t(sizeof(float));
    if (p.P && !pq_bwd_ok(p))   // the general P/Q backward: its own checkpoints and the slabs
        return (pq_general_ck_floats(p) + 2 * gen_slab_floats(p, pq_general_rows_per_block(p))) * int64_t(sizeof(float));
    if (diag_via_pq_bwd(p))   // the P/Q backward with the zero pair (its own checkpoints without tile states)
        return ((p.tile_states ? 0 : bwd::fast_ck_floats(p)) + 2 * bwd::fast_part_floats(p)) * int64_t(sizeof(float));
    if (!p.P && bwd::fast_ok(p) && p.tile_states)
        return (2 * bwd::fast_part_floats(p) + bwd::carry_floats(bwd::seg_plan_for(p))) * int64_t(sizeof(float));
    if (!p.P && bwd::fast_ok(p) && bwd::states_pass_ok(p)) {
        // The states-only forward writes the checkpoints into the workspace; segment carries follow.
        mm_scan_bwd_params q = p;
        float dummy;
        q.tile_states = &dummy;
        return (bwd::fast_ck_floats(p) + 2 * bwd::fast_part_floats(p) + bwd::carry_floats(bwd::seg_plan_for(q))) *
               int64_t(sizeof(float));
    }
    if (p.P && p.tile_states) return 2 * bwd::fast_part_floats(p) * int64_t(sizeof(float));
    if (p.P || bwd::fast_ok(p)) return (bwd::fast_ck_floats(p) + 2 * bwd::fast_part_floats(p)) * int64_t(sizeof(float));
    const int64_t n_tiles = (p.seqlen + bwd::kBT - 1) / bwd::kBT;
    return (p.batch * p.dim * n_tiles * p.dstate + 2 * gen_slab_floats(p, bwd::gen_rows_per_block(p))) *
           int64_t(sizeof(float));
}

int64_t bwd_workspace_min_bytes(const mm_scan_bwd_params &p) {
    if (diag_via_pq_bwd(p) || bwd::split_ok(p)) return bwd_workspace_bytes(p);
    if (!p.P && bwd::fast_ok(p) && p.tile_states) return 2 * bwd::fast_part_floats(p) * int64_t(sizeof(float));
    if (!p.P && bwd::fast_ok(p)) return (bwd::fast_ck_floats(p) + 2 * bwd::fast_part_floats(p)) * int64_t(sizeof(float));
    return bwd_workspace_bytes(p);
}

template <typename T>
int launch_bwd(const mm_scan_bwd_params &p_in, hipStream_t s) {
    // Diagonal requests with dstate < 16 run the P/Q backward with a zero rank-1 pair.
    mm_scan_bwd_params p = p_in;
    if (diag_via_pq_bwd(p_in) && attach_zero_pair(p) != MM_OK) p = p_in;
    // The accumulated gradients start from zero on the launch stream (the dstate-16 kernel writes
    // dB and dC whole and only accumulates dA, dD and ddelta_bias).
    const bool fast = bwd::fast_ok(p) && p.seqlen > 0;
    bwd::Fills f;
    f.add(p.dA, 1, 1, p.dim, p.dstate, 0, 0, p.dA_d_stride, p.dA_dstate_stride);
    if (p.is_variable_B && !fast)
        f.add(p.dB, p.batch, p.n_groups, p.dstate, p.seqlen, p.dB_batch_stride, p.dB_group_stride, p.dB_dstate_stride, 1);
    if (!p.is_variable_B) f.add(p.dB, 1, 1, p.dim, p.dstate, 0, 0, p.dB_d_stride, p.dB_dstate_stride);
    if (p.is_variable_C && !fast)
        f.add(p.dC, p.batch, p.n_groups, p.dstate, p.seqlen, p.dC_batch_stride, p.dC_group_stride, p.dC_dstate_stride, 1);
    if (!p.is_variable_C) f.add(p.dC, 1, 1, p.dim, p.dstate, 0, 0, p.dC_d_stride, p.dC_dstate_stride);
    if (p.dD) f.add(p.dD, 1, 1, 1, p.dim, 0, 0, 0, 1);
    if (p.ddelta_bias) f.add(p.ddelta_bias, 1, 1, 1, p.dim, 0, 0, 0, 1);
    // dP / dQ: one (dstate, rank) slice per channel unless their d stride is 0 (one shared slice).
    if (p.P) {
        f.add(p.dP, 1, p.dP_d_stride ? p.dim : 1, p.dstate, p.pq_rank, 0, p.dP_d_stride, p.dP_dstate_stride,
              p.dP_r_stride);
        f.add(p.dQ, 1, p.dQ_d_stride ? p.dim : 1, p.pq_rank, p.dstate, 0, p.dQ_d_stride, p.dQ_r_stride,
              p.dQ_dstate_stride);
    }
    const int rc = f.launch(s);
    if (rc != MM_OK) return rc;
    if (p.seqlen == 0) return MM_OK;
    if (p.P) return bwd::launch_pq<T>(p, s);
    if (bwd::fast_ok(p)) return bwd::launch_fast<T>(p, s);
    if (bwd::split_ok(p)) return bwd::launch_split<T>(p, s);
    return bwd::launch_general<T>(p, s);
}

template int launch_bwd<float>(const mm_scan_bwd_params &, hipStream_t);
template int launch_bwd<f16_t>(const mm_scan_bwd_params &, hipStream_t);
template int launch_bwd<bf16_t>(const mm_scan_bwd_params &, hipStream_t);

}  // namespace mm
