// mm_conv1d.hip -- gfx950 causal depthwise conv1d (forward and decode update), the step before the
// selective scan in every Mamba block.
//
// Reference behaviour: causal_conv1d_fn / causal_conv1d_update of the package causal-conv1d that the
// reference imports (mamba_simplemotif.py:16-19; pinned >= 1.2.0, not vendored), whose in-tree
// fallback is mamba_simplemotif.py:298-299 (forward) and :353-358 (update):
//   out[b,d,t] = act(bias[d] + sum_{k<W} w[d,k] x[b,d,t-(W-1)+k]),  x before t = 0 from
//   initial_states (or 0); the update appends each new token to the state and takes the dot of the
//   state's last W entries with w.
// Both are HBM-bound (2 bytes in, 2 out per element for 16-bit data): the forward gives each lane 8
// consecutive outputs of one row -- one 16-byte load of its inputs, one of the 8 before them (the
// halo of W-1 <= 7 inputs), the row's W weights in registers, one 16-byte store; the update gives
// each lane one (batch, channel) row and keeps the last W-1 inputs in registers.
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "mm_common.h"
#include "mm_conv1d.h"
#include "mm_internal.h"

namespace mm {
namespace conv {

constexpr int kThreads = 256;
constexpr int kChunk = 8;        // outputs per lane

// One element of a tensor whose dtype is known only at run time (weights, bias, states).
__device__ __forceinline__ float load_any(const void *p, mm_dtype dt, int64_t i) {
    switch (dt) {
        case MM_FLOAT32: return reinterpret_cast<const float *>(p)[i];
        case MM_FLOAT16: return to_f32(reinterpret_cast<const f16_t *>(p)[i]);
        default: return to_f32(reinterpret_cast<const bf16_t *>(p)[i]);
    }
}
__device__ __forceinline__ void store_any(void *p, mm_dtype dt, int64_t i, float v) {
    switch (dt) {
        case MM_FLOAT32: reinterpret_cast<float *>(p)[i] = v; break;
        case MM_FLOAT16: reinterpret_cast<f16_t *>(p)[i] = from_f32<f16_t>(v); break;
        default: reinterpret_cast<bf16_t *>(p)[i] = from_f32<bf16_t>(v); break;
    }
}

// VEC: rows 16-byte aligned, seqlen a multiple of 8 (every chunk is whole and vector-movable).
// Each lane computes NC consecutive chunks of 8 outputs: all NC + 1 loads (the 8 inputs before the
// first chunk carry its halo) are issued before any arithmetic.
template <typename T, int W, bool VEC, int NC>
__global__ void __launch_bounds__(kThreads)
conv1d_fwd_kernel(const mm_conv1d_fwd_params p) {
    const int64_t t0 = (int64_t(blockIdx.x) * kThreads + threadIdx.x) * (kChunk * NC);
    const int64_t d = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t L = p.seqlen;
    if (t0 >= L) return;
    const T *xr = reinterpret_cast<const T *>(p.x) + b * p.x_batch_stride + d * p.x_d_stride;
    T *orow = reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride;

    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = load_any(p.weight, p.wtype, d * p.weight_d_stride + k * p.weight_w_stride);
    const float bias = p.bias ? load_any(p.bias, p.wtype, d * p.bias_stride) : 0.f;

    // xs[0..7]: the 8 inputs before the first chunk (initial states or 0 before t = 0); then the chunks.
    float xs[kChunk * (NC + 1)];
    if (VEC) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (t0 + c * kChunk < L) load8(xr + t0 + c * kChunk, xs + kChunk * (c + 1));
            else {
#pragma unroll
                for (int i = 0; i < kChunk; ++i) xs[kChunk * (c + 1) + i] = 0.f;
            }
        if (t0 >= kChunk) load8(xr + t0 - kChunk, xs);
    } else {
#pragma unroll
        for (int i = 0; i < kChunk * NC; ++i) xs[kChunk + i] = t0 + i < L ? to_f32(xr[t0 + i]) : 0.f;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) xs[i] = t0 >= kChunk ? to_f32(xr[t0 - kChunk + i]) : 0.f;
    }
    if (t0 < kChunk) {  // the first chunk of the row: the W - 1 positions before t = 0
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int j = i - kChunk + (W - 1);   // index into initial_states
            xs[i] = (p.initial_states && j >= 0)
                ? load_any(p.initial_states, p.itype, b * p.init_batch_stride + d * p.init_d_stride + j * p.init_w_stride)
                : 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t tc = t0 + c * kChunk;
        float o[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            float acc = bias;
#pragma unroll
            for (int k = 0; k < W; ++k) acc = __builtin_fmaf(w[k], xs[kChunk * (c + 1) + i - (W - 1) + k], acc);
            o[i] = p.silu ? acc * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-acc * kLog2e)) : acc;
        }
        if (VEC) {
            if (tc < L) store8(orow + tc, o);
        } else {
#pragma unroll
            for (int i = 0; i < kChunk; ++i)
                if (tc + i < L) orow[tc + i] = from_f32<T>(o[i]);
        }
        // The last W - 1 inputs (initial states where the row is shorter): written by the lane
        // holding position L - 1; all of them lie in xs.
        if (p.final_states && tc <= L - 1 && L - 1 < tc + kChunk) {
#pragma unroll
            for (int j = 0; j < W - 1; ++j) {
                const int64_t pos = L - (W - 1) + j;          // position in the row, may be negative
                const int idx = int(pos - tc) + kChunk * (c + 1);   // index into xs (pos >= tc - 7)
                store_any(p.final_states, p.itype, b * p.final_batch_stride + d * p.final_d_stride + j * p.final_w_stride,
                          xs[idx]);
            }
        }
    }
}

// One lane per (batch, channel) row. VEC4: the state rows are 4 contiguous entries of the input
// dtype, aligned for one 4-element vector load and store (the module's layout, state_len = d_conv = 4),
// and the width is at most 5.
template <typename T, bool VEC4>
__global__ void __launch_bounds__(kThreads)
conv1d_update_kernel(const mm_conv1d_update_params p) {
    const int64_t row = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (row >= p.batch * p.dim) return;
    const int64_t b = row / p.dim;
    const int64_t d = row - b * p.dim;
    const int W = int(p.width);
    const int64_t S = p.state_len;
    const T *xr = reinterpret_cast<const T *>(p.x) + b * p.x_batch_stride + d * p.x_d_stride;
    T *orow = reinterpret_cast<T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride;
    const int64_t sbase = b * p.state_batch_stride + d * p.state_d_stride;

    float st4[4] = {0.f, 0.f, 0.f, 0.f};
    if (VEC4) {
        const RawVec<T, 4> r = load_raw<T, 4>(reinterpret_cast<const T *>(p.conv_state) + sbase);
        unpack_raw<T, 4>(r, st4);
    }
    float w[MM_CONV1D_MAX_WIDTH], win[MM_CONV1D_MAX_WIDTH];
#pragma unroll
    for (int k = 0; k < MM_CONV1D_MAX_WIDTH; ++k) {
        w[k] = k < W ? load_any(p.weight, p.wtype, d * p.weight_d_stride + k * p.weight_w_stride) : 0.f;
        // Window slot k holds the input k steps before the current token once the token is shifted
        // in (slot 0: the token itself); before the first shift slot k holds state[S - 1 - k].
        if (VEC4)
            win[k] = (k < W - 1) ? st4[3 - k] : 0.f;
        else
            win[k] = (k < W - 1) ? load_any(p.conv_state, p.stype, sbase + (S - 1 - k) * p.state_l_stride) : 0.f;
    }
    const float bias = p.bias ? load_any(p.bias, p.wtype, d * p.bias_stride) : 0.f;
    for (int64_t t = 0; t < p.seqlen; ++t) {
#pragma unroll
        for (int k = MM_CONV1D_MAX_WIDTH - 1; k >= 1; --k) win[k] = win[k - 1];
        win[0] = to_f32(xr[t * p.x_l_stride]);
        float acc = bias;
#pragma unroll
        for (int k = 0; k < MM_CONV1D_MAX_WIDTH; ++k)
            if (k < W) acc = __builtin_fmaf(w[W - 1 - k], win[k], acc);
        const float o = p.silu ? acc * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-acc * kLog2e)) : acc;
        orow[t * p.out_l_stride] = from_f32<T>(o);
    }
    // New state: the last S entries of (old state ++ new tokens). Ascending j reads position
    // j + seqlen of the old state before anything at or above it is written.
    if (VEC4) {
        float ns[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t src = j + p.seqlen;
            ns[j] = src < 4 ? st4[src] : to_f32(xr[(src - 4) * p.x_l_stride]);
        }
        store_vec<T, 4>(reinterpret_cast<T *>(p.conv_state) + sbase, ns);
    } else {
        for (int64_t j = 0; j < S; ++j) {
            const int64_t src = j + p.seqlen;
            const float v = src < S ? load_any(p.conv_state, p.stype, sbase + src * p.state_l_stride)
                                    : to_f32(xr[(src - S) * p.x_l_stride]);
            store_any(p.conv_state, p.stype, sbase + j * p.state_l_stride, v);
        }
    }
}


// The decode form of the Mamba block (one new token, width 4, a contiguous 4-entry state per row,
// weight rows of 4 contiguous elements): one lane per (batch, channel) row; a workgroup covers 256
// consecutive channels of U consecutive batch rows, so a lane loads its channel's weights and bias
// once for U rows, and every load of the U rows is issued before any arithmetic. blockIdx.x = batch
// block * n_dblk + channel block (no 64-bit division per lane); channels past `dim` and rows past
// `batch` reload the last one and store nothing.
template <typename T, typename WT, int U>
__global__ void __launch_bounds__(kThreads)
conv1d_update_tok4(const mm_conv1d_update_params p, const uint32_t n_dblk) {
    const uint32_t bb = blockIdx.x / n_dblk;
    const uint32_t jd = blockIdx.x - bb * n_dblk;
    const uint32_t dim = uint32_t(p.dim), batch = uint32_t(p.batch);
    const uint32_t dr = jd * uint32_t(kThreads) + threadIdx.x;
    const uint32_t d = dr < dim ? dr : dim - 1;
    const WT *bptr = reinterpret_cast<const WT *>(p.bias);
    float w4[4];
    unpack_raw<WT, 4>(load_raw<WT, 4>(reinterpret_cast<const WT *>(p.weight) + int64_t(d) * p.weight_d_stride), w4);
    const float bias = bptr ? to_f32(bptr[int64_t(d) * p.bias_stride]) : 0.f;

    RawVec<T, 4> st[U];
    T xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t b0 = bb * U + u;
        const uint32_t b = b0 < batch ? b0 : batch - 1;
        st[u] = load_raw<T, 4>(reinterpret_cast<const T *>(p.conv_state) + int64_t(b) * p.state_batch_stride +
                               int64_t(d) * p.state_d_stride);
        xv[u] = reinterpret_cast<const T *>(p.x)[int64_t(b) * p.x_batch_stride + int64_t(d) * p.x_d_stride];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t b = bb * U + u;
        float s4[4];
        unpack_raw<T, 4>(st[u], s4);
        const float x = to_f32(xv[u]);
        // The window after the shift is (s1, s2, s3, x); weight k multiplies window entry k.
        float acc = bias;
        acc = __builtin_fmaf(w4[0], s4[1], acc);
        acc = __builtin_fmaf(w4[1], s4[2], acc);
        acc = __builtin_fmaf(w4[2], s4[3], acc);
        acc = __builtin_fmaf(w4[3], x, acc);
        const float o = p.silu ? acc * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-acc * kLog2e)) : acc;
        if (dr < dim && b < batch) {
            const float ns[4] = {s4[1], s4[2], s4[3], x};
            store_vec<T, 4>(reinterpret_cast<T *>(p.conv_state) + int64_t(b) * p.state_batch_stride +
                                int64_t(dr) * p.state_d_stride, ns);
            reinterpret_cast<T *>(p.out)[int64_t(b) * p.out_batch_stride + int64_t(dr) * p.out_d_stride] = from_f32<T>(o);
        }
    }
}

// Backward: one workgroup per channel d walks every (batch row, tile of kThreads * 8 * NC steps) of
// that channel; in each tile a lane owns NC chunks of 8 positions. It recomputes the pre-activation y
// at its positions and the next W - 1 (x from W - 1 before to W - 1 after, as 8-element chunks),
// forms dy = dout silu'(y) and writes dx[s] = sum_k w[k] dy[s + W - 1 - k]. Its shares of
// dweight[d, k] = sum dy[t] x[t - (W - 1) + k] and dbias[d] = sum dy[t] stay in registers over the
// whole walk; at the end the workgroup adds them (waves by shuffles, then LDS, in a fixed order)
// and one lane per k stores them: no atomics, no clearing launch, and the same bits on every run.
template <typename T, int W, bool VEC, int NC>
__global__ void __launch_bounds__(kThreads)
conv1d_bwd_kernel(const mm_conv1d_bwd_params p) {
    __shared__ float sRed[kThreads / 64][MM_CONV1D_MAX_WIDTH + 1];
    constexpr int64_t kTile = int64_t(kThreads) * kChunk * NC;   // steps per tile
    const int64_t d = blockIdx.x;
    const int64_t L = p.seqlen;
    const int64_t n_tiles = (L + kTile - 1) / kTile;

    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = load_any(p.weight, p.wtype, d * p.weight_d_stride + k * p.weight_w_stride);
    const float bias = p.bias ? load_any(p.bias, p.wtype, d * p.bias_stride) : 0.f;

    float dw[W], db = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) dw[k] = 0.f;
    // xs: chunk before, the NC chunks, chunk after; gs: dout of the NC chunks and the chunk after.
    constexpr int NX = kChunk * (NC + 2), NG = kChunk * (NC + 1);
    // One tile of a row: dy at positions t0 .. t0 + 8 (NC + 1) - 1 (0 past L), dx of the NC chunks,
    // and the lane's dweight / dbias terms.
    auto tile_math = [&](T *dxr, const int64_t t0, const float *xs, const float *gs) {
        float dy[NG];
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            float y = bias;
#pragma unroll
            for (int k = 0; k < W; ++k) y = __builtin_fmaf(w[k], xs[kChunk + i - (W - 1) + k], y);
            float g = gs[i];
            if (p.silu) {
                const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-y * kLog2e));
                g *= sg * (1.f + y * (1.f - sg));
            }
            dy[i] = (t0 + i < L) ? g : 0.f;
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float o[kChunk];
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                const int s = c * kChunk + i;
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < W; ++k) acc = __builtin_fmaf(w[k], dy[s + W - 1 - k], acc);
                o[i] = acc;
                db += dy[s];
#pragma unroll
                for (int k = 0; k < W; ++k) dw[k] = __builtin_fmaf(dy[s], xs[kChunk + s - (W - 1) + k], dw[k]);
            }
            const int64_t tc = t0 + c * kChunk;
            if (VEC && tc + kChunk <= L) {
                store8(dxr + tc, o);
            } else {
#pragma unroll
                for (int i = 0; i < kChunk; ++i)
                    if (tc + i < L) dxr[tc + i] = from_f32<T>(o[i]);
            }
        }
    };
    if constexpr (VEC) {
        // Rows in 16-byte vectors (L % 8 == 0, aligned rows): a chunk is wholly inside [0, L) or
        // wholly outside. The walk over (batch row, tile) pairs loads the next pair's raw vectors
        // before the current pair's arithmetic, so that their latency overlaps it.
        struct Raw {
            Vec8<T> x[NC + 2], g[NC + 1];
        };
        const int64_t n_it = p.batch * n_tiles;
        auto lane_t0 = [&](int64_t it) { return (it % n_tiles) * kTile + int64_t(threadIdx.x) * (kChunk * NC); };
        auto load_raw = [&](int64_t it, Raw &r) {
            const int64_t b = it / n_tiles, t0 = lane_t0(it);
            const T *xr = reinterpret_cast<const T *>(p.x) + b * p.x_batch_stride + d * p.x_d_stride;
            const T *gr = reinterpret_cast<const T *>(p.dout) + b * p.dout_batch_stride + d * p.dout_d_stride;
#pragma unroll
            for (int c = 0; c < NC + 2; ++c) {
                const int64_t t = t0 + (c - 1) * kChunk;
                r.x[c] = {};
                if (t >= 0 && t < L) r.x[c] = *reinterpret_cast<const Vec8<T> *>(xr + t);
            }
#pragma unroll
            for (int c = 0; c < NC + 1; ++c) {
                const int64_t t = t0 + c * kChunk;
                r.g[c] = {};
                if (t < L) r.g[c] = *reinterpret_cast<const Vec8<T> *>(gr + t);
            }
        };
        Raw cur, nxt;
        if (n_it > 0) load_raw(0, cur);
        for (int64_t it = 0; it < n_it; ++it) {
            if (it + 1 < n_it) load_raw(it + 1, nxt);
            const int64_t t0 = lane_t0(it);
            if (t0 < L) {   // lanes past the row's end (last tile only) have nothing to do
                float xs[NX], gs[NG];
#pragma unroll
                for (int c = 0; c < NC + 2; ++c) unpack8(cur.x[c], xs + c * kChunk);
#pragma unroll
                for (int c = 0; c < NC + 1; ++c) unpack8(cur.g[c], gs + c * kChunk);
                T *dxr = reinterpret_cast<T *>(p.dx) + (it / n_tiles) * p.dx_batch_stride + d * p.dx_d_stride;
                tile_math(dxr, t0, xs, gs);
            }
            cur = nxt;
        }
    } else {
        for (int64_t b = 0; b < p.batch; ++b) {
            const T *xr = reinterpret_cast<const T *>(p.x) + b * p.x_batch_stride + d * p.x_d_stride;
            const T *gr = reinterpret_cast<const T *>(p.dout) + b * p.dout_batch_stride + d * p.dout_d_stride;
            T *dxr = reinterpret_cast<T *>(p.dx) + b * p.dx_batch_stride + d * p.dx_d_stride;
            for (int64_t tile = 0; tile < n_tiles; ++tile) {
                const int64_t t0 = tile * kTile + int64_t(threadIdx.x) * (kChunk * NC);
                if (t0 >= L) continue;   // lanes past the row's end (last tile only)
                float xs[NX], gs[NG];
                auto ld = [&](const T *row, int64_t t, float *dst) {   // 8 elements at t (zeros outside [0, L))
#pragma unroll
                    for (int i = 0; i < kChunk; ++i) dst[i] = (t + i >= 0 && t + i < L) ? to_f32(row[t + i]) : 0.f;
                };
#pragma unroll
                for (int c = 0; c < NC + 2; ++c) ld(xr, t0 + (c - 1) * kChunk, xs + c * kChunk);
#pragma unroll
                for (int c = 0; c < NC + 1; ++c) ld(gr, t0 + c * kChunk, gs + c * kChunk);
                tile_math(dxr, t0, xs, gs);
            }
        }
    }
    // Workgroup sums of dweight / dbias: waves by shuffles, then the waves in order through LDS.
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k <= W; ++k) {
        float v = k < W ? dw[k] : db;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) sRed[wv][k] = v;
    }
    __syncthreads();
    if (threadIdx.x <= W) {
        const int k = threadIdx.x;
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < kThreads / 64; ++i) v += sRed[i][k];
        if (k < W) p.dweight[d * W + k] = v;
        else if (p.dbias) p.dbias[d] = v;
    }
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }


// Chunks of 8 positions per lane and tile: 2 (4,096-step tiles) unless 1 (2,048-step tiles) leaves
// fewer lanes past the end of the rows' last tiles (a 2,048-step row fills only half of a
// 4,096-step tile).
int bwd_chunks(int64_t L) {
    auto idle = [&](int64_t tile) { return ((L + tile - 1) / tile) * tile - L; };
    const int64_t t2 = int64_t(kThreads) * kChunk * 2;
    return idle(t2 / 2) < idle(t2) ? 1 : 2;
}

template <typename T, int W, int NC>
int launch_bwd_wn(const mm_conv1d_bwd_params &p, hipStream_t s) {
    const int64_t eb = int64_t(sizeof(T));
    auto row_ok = [&](const void *ptr, int64_t s0, int64_t s1) {
        return aligned16(ptr) && (s0 * eb) % 16 == 0 && (s1 * eb) % 16 == 0;
    };
    const bool vec = p.seqlen % kChunk == 0 && row_ok(p.x, p.x_batch_stride, p.x_d_stride) &&
                     row_ok(p.dout, p.dout_batch_stride, p.dout_d_stride) && row_ok(p.dx, p.dx_batch_stride, p.dx_d_stride);
    const dim3 grid(unsigned(p.dim));   // one workgroup per channel (dim < 2^24, checked on entry)
    if (vec)
        hipLaunchKernelGGL((conv1d_bwd_kernel<T, W, true, NC>), grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL((conv1d_bwd_kernel<T, W, false, NC>), grid, dim3(kThreads), 0, s, p);
    return launch_status("conv1d_bwd");
}

template <typename T, int W>
int launch_bwd_w(const mm_conv1d_bwd_params &p, hipStream_t s) {
    return bwd_chunks(p.seqlen) == 1 ? launch_bwd_wn<T, W, 1>(p, s) : launch_bwd_wn<T, W, 2>(p, s);
}

// dweight and dbias are written (not accumulated) by the one workgroup of each channel, also for
// an empty batch or sequence (zero sums).
template <typename T>
int launch_bwd(const mm_conv1d_bwd_params &p, hipStream_t s) {
    if (p.dim == 0) return MM_OK;
    switch (p.width) {
        case 1: return launch_bwd_w<T, 1>(p, s);
        case 2: return launch_bwd_w<T, 2>(p, s);
        case 3: return launch_bwd_w<T, 3>(p, s);
        case 4: return launch_bwd_w<T, 4>(p, s);
        case 5: return launch_bwd_w<T, 5>(p, s);
        case 6: return launch_bwd_w<T, 6>(p, s);
        case 7: return launch_bwd_w<T, 7>(p, s);
        default: return launch_bwd_w<T, 8>(p, s);
    }
}

template <typename T, int W>
int launch_fwd_w(const mm_conv1d_fwd_params &p, hipStream_t s) {
    const int64_t eb = int64_t(sizeof(T));
    const bool vec = p.seqlen % kChunk == 0 && aligned16(p.x) && aligned16(p.out) && (p.x_batch_stride * eb) % 16 == 0 &&
                     (p.x_d_stride * eb) % 16 == 0 && (p.out_batch_stride * eb) % 16 == 0 && (p.out_d_stride * eb) % 16 == 0;
    const char *e = getenv("MM_CONV_NC");
    const int nc = e ? atoi(e) : 2;
    auto go = [&](auto ncc) {
        constexpr int NC = decltype(ncc)::value;
        const int64_t per_lane = int64_t(kChunk) * NC;
        const int64_t lanes = (p.seqlen + per_lane - 1) / per_lane;
        dim3 grid(unsigned((lanes + kThreads - 1) / kThreads), unsigned(p.dim), unsigned(p.batch));
        if (vec)
            hipLaunchKernelGGL((conv1d_fwd_kernel<T, W, true, NC>), grid, dim3(kThreads), 0, s, p);
        else
            hipLaunchKernelGGL((conv1d_fwd_kernel<T, W, false, NC>), grid, dim3(kThreads), 0, s, p);
    };
    if (nc == 1) go(std::integral_constant<int, 1>{});
    else if (nc == 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 2>{});
    return launch_status("conv1d_fwd");
}

template <typename T>
int launch_fwd(const mm_conv1d_fwd_params &p, hipStream_t s) {
    switch (p.width) {
        case 1: return launch_fwd_w<T, 1>(p, s);
        case 2: return launch_fwd_w<T, 2>(p, s);
        case 3: return launch_fwd_w<T, 3>(p, s);
        case 4: return launch_fwd_w<T, 4>(p, s);
        case 5: return launch_fwd_w<T, 5>(p, s);
        case 6: return launch_fwd_w<T, 6>(p, s);
        case 7: return launch_fwd_w<T, 7>(p, s);
        default: return launch_fwd_w<T, 8>(p, s);
    }
}

template <typename T>
int launch_update(const mm_conv1d_update_params &p, hipStream_t s) {
    const int64_t rows = p.batch * p.dim;
    const int64_t vb = 4 * int64_t(sizeof(T));
    const bool vec4 = p.state_len == 4 && p.width <= 5 && p.state_l_stride == 1 && p.stype == p.itype &&
                      reinterpret_cast<uintptr_t>(p.conv_state) % uintptr_t(vb) == 0 && p.state_batch_stride % 4 == 0 &&
                      p.state_d_stride % 4 == 0;
    if (vec4 && p.seqlen == 1 && p.width == 4 && p.weight_w_stride == 1 && p.dim < (int64_t(1) << 31)) {
        const int64_t wb = 4 * (p.wtype == MM_FLOAT32 ? 4 : 2);
        const bool w_ok = reinterpret_cast<uintptr_t>(p.weight) % uintptr_t(wb) == 0 && p.weight_d_stride % 4 == 0;
        if (w_ok && (p.wtype == MM_FLOAT32 || p.wtype == p.itype) && p.batch < (int64_t(1) << 31)) {
            // Four batch rows per workgroup share the weight and bias loads.
            const int U = p.batch >= 4 ? 4 : 1;
            const int64_t n_dblk = (p.dim + kThreads - 1) / kThreads;
            const int64_t n_bblk = (p.batch + U - 1) / U;
            if (n_bblk * n_dblk < (int64_t(1) << 31)) {
                const dim3 g1(unsigned(n_bblk * n_dblk));
                const bool wf = p.wtype == MM_FLOAT32;
                if (U == 4) {
                    if (wf) hipLaunchKernelGGL((conv1d_update_tok4<T, float, 4>), g1, dim3(kThreads), 0, s, p, uint32_t(n_dblk));
                    else hipLaunchKernelGGL((conv1d_update_tok4<T, T, 4>), g1, dim3(kThreads), 0, s, p, uint32_t(n_dblk));
                } else {
                    if (wf) hipLaunchKernelGGL((conv1d_update_tok4<T, float, 1>), g1, dim3(kThreads), 0, s, p, uint32_t(n_dblk));
                    else hipLaunchKernelGGL((conv1d_update_tok4<T, T, 1>), g1, dim3(kThreads), 0, s, p, uint32_t(n_dblk));
                }
                return launch_status("conv1d_update");
            }
        }
    }
    const dim3 grid(unsigned((rows + kThreads - 1) / kThreads));
    if (vec4)
        hipLaunchKernelGGL((conv1d_update_kernel<T, true>), grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL((conv1d_update_kernel<T, false>), grid, dim3(kThreads), 0, s, p);
    return launch_status("conv1d_update");
}

bool dtype_ok(mm_dtype t) { return t == MM_FLOAT32 || t == MM_FLOAT16 || t == MM_BFLOAT16; }

int invalid(const char *msg) { return set_error(MM_ERR_INVALID_ARGUMENT, msg); }

}  // namespace conv
}  // namespace mm

extern "C" {

int mm_causal_conv1d_fwd(const mm_conv1d_fwd_params *params, void *stream) {
    using namespace mm::conv;
    if (!params) return invalid("mm_causal_conv1d_fwd: params is NULL");
    const mm_conv1d_fwd_params &p = *params;
    if (!dtype_ok(p.itype) || !dtype_ok(p.wtype)) return invalid("mm_causal_conv1d_fwd: unknown dtype");
    if (p.batch < 0 || p.dim < 0 || p.seqlen < 0) return invalid("mm_causal_conv1d_fwd: negative size");
    if (p.width < 1 || p.width > MM_CONV1D_MAX_WIDTH)
        return invalid("mm_causal_conv1d_fwd: width must be in [1, 8]");
    if (p.batch > 65535 || p.dim > 65535)
        return mm::set_error(MM_ERR_UNSUPPORTED, "mm_causal_conv1d_fwd: batch and dim must be <= 65535");
    if (p.batch == 0 || p.dim == 0 || p.seqlen == 0) return MM_OK;
    if (!p.x || !p.weight || !p.out) return invalid("mm_causal_conv1d_fwd: x, weight and out are required");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return launch_fwd<float>(p, s);
        case MM_FLOAT16: return launch_fwd<mm::f16_t>(p, s);
        default: return launch_fwd<mm::bf16_t>(p, s);
    }
}

int mm_causal_conv1d_bwd(const mm_conv1d_bwd_params *params, void *stream) {
    using namespace mm::conv;
    if (!params) return invalid("mm_causal_conv1d_bwd: params is NULL");
    const mm_conv1d_bwd_params &p = *params;
    if (!dtype_ok(p.itype) || !dtype_ok(p.wtype)) return invalid("mm_causal_conv1d_bwd: unknown dtype");
    if (p.batch < 0 || p.dim < 0 || p.seqlen < 0) return invalid("mm_causal_conv1d_bwd: negative size");
    if (p.width < 1 || p.width > MM_CONV1D_MAX_WIDTH)
        return invalid("mm_causal_conv1d_bwd: width must be in [1, 8]");
    // One workgroup of kThreads lanes per channel on a one-dimensional grid: gridDim.x * blockDim.x
    // (the grid's lane count) must stay below 2^32.
    if (p.dim >= (int64_t(1) << 32) / mm::conv::kThreads)
        return mm::set_error(MM_ERR_UNSUPPORTED, "mm_causal_conv1d_bwd: dim must be < 2^24");
    if (p.dim == 0) return MM_OK;
    if (!p.weight || !p.dweight || (p.bias && !p.dbias))
        return invalid("mm_causal_conv1d_bwd: weight and dweight (and dbias with bias) are required");
    if (p.batch > 0 && p.seqlen > 0 && (!p.x || !p.dout || !p.dx))
        return invalid("mm_causal_conv1d_bwd: x, dout and dx are required");
    mm_conv1d_bwd_params q = p;
    if (q.batch == 0) q.seqlen = 0;   // nothing to add: the sums are written as zeros
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (q.itype) {
        case MM_FLOAT32: return launch_bwd<float>(q, s);
        case MM_FLOAT16: return launch_bwd<mm::f16_t>(q, s);
        default: return launch_bwd<mm::bf16_t>(q, s);
    }
}

int mm_causal_conv1d_update(const mm_conv1d_update_params *params, void *stream) {
    using namespace mm::conv;
    if (!params) return invalid("mm_causal_conv1d_update: params is NULL");
    const mm_conv1d_update_params &p = *params;
    if (!dtype_ok(p.itype) || !dtype_ok(p.wtype) || !dtype_ok(p.stype))
        return invalid("mm_causal_conv1d_update: unknown dtype");
    if (p.batch < 0 || p.dim < 0 || p.seqlen < 0) return invalid("mm_causal_conv1d_update: negative size");
    if (p.width < 1 || p.width > MM_CONV1D_MAX_WIDTH)
        return invalid("mm_causal_conv1d_update: width must be in [1, 8]");
    if (p.state_len < p.width - 1) return invalid("mm_causal_conv1d_update: state_len must be >= width - 1");
    if (p.batch == 0 || p.dim == 0) return MM_OK;
    if (!p.x || !p.conv_state || !p.weight || !p.out)
        return invalid("mm_causal_conv1d_update: x, conv_state, weight and out are required");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (p.itype) {
        case MM_FLOAT32: return launch_update<float>(p, s);
        case MM_FLOAT16: return launch_update<mm::f16_t>(p, s);
        default: return launch_update<mm::bf16_t>(p, s);
    }
}

}  // extern "C"
