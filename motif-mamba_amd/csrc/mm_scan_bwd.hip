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
//   scan_bwd_general<T>   any shape: a 256-lane workgroup holds 256/NP rows, one lane per state
//       (NP = next power of two >= dstate); sums over states go through LDS, sums over rows
//       (dB, dC, dA, dD, ddelta_bias) are float32 device atomics.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace bwd {

constexpr int kBT = 16;          // steps per checkpoint tile
constexpr int kGenThreads = 256;

// Zero a float32 tensor of up to 4 dimensions with arbitrary element strides.
__global__ void __launch_bounds__(256)
fill_zero4(float *p, int64_t n0, int64_t n1, int64_t n2, int64_t n3, int64_t s0, int64_t s1, int64_t s2, int64_t s3) {
    const int64_t total = n0 * n1 * n2 * n3;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t r = i;
        const int64_t i3 = r % n3; r /= n3;
        const int64_t i2 = r % n2; r /= n2;
        const int64_t i1 = r % n1; r /= n1;
        p[r * s0 + i1 * s1 + i2 * s2 + i3 * s3] = 0.f;
    }
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + expf(-x)); }

template <typename T>
__global__ void __launch_bounds__(kGenThreads)
scan_bwd_general(const mm_scan_bwd_params p, const int64_t ratio, const int np_log2) {
    __shared__ float sDu[kBT * kGenThreads];   // [step][lane]: per-state partials of sum_n gh B
    __shared__ float sDdt[kBT * kGenThreads];  // [step][lane]: per-state partials of ddt
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
        h = __builtin_fmaf(fast_exp2(dt * A2), h, dt * to_f32(up[t]) * b_at(t));
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
                as[s] = fast_exp2(dts[s] * A2);
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
                if (on) {
                    if (dCv) atomicAdd(dCv + t, dcv);
                    if (dBv) atomicAdd(dBv + t, dbv);
                }
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

template <typename T>
int launch_general(const mm_scan_bwd_params &p, hipStream_t s) {
    int np_log2 = 0;
    while ((1 << np_log2) < p.dstate) ++np_log2;
    const int64_t rows_per_block = kGenThreads >> np_log2;
    const int64_t rows = p.batch * p.dim;
    dim3 grid(unsigned((rows + rows_per_block - 1) / rows_per_block));
    hipLaunchKernelGGL((scan_bwd_general<T>), grid, dim3(kGenThreads), 0, s, p, p.dim / p.n_groups, np_log2);
    return launch_status("scan_bwd_general");
}

int launch_fill(float *ptr, int64_t n0, int64_t n1, int64_t n2, int64_t n3, int64_t s0, int64_t s1, int64_t s2,
                int64_t s3, hipStream_t s) {
    const int64_t total = n0 * n1 * n2 * n3;
    if (!ptr || total == 0) return MM_OK;
    const int64_t blocks = (total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096;
    hipLaunchKernelGGL(fill_zero4, dim3(unsigned(blocks)), dim3(256), 0, s, ptr, n0, n1, n2, n3, s0, s1, s2, s3);
    return launch_status("fill_zero4");
}

}  // namespace bwd

int64_t bwd_workspace_bytes(const mm_scan_bwd_params &p) {
    const int64_t n_tiles = (p.seqlen + bwd::kBT - 1) / bwd::kBT;
    return p.batch * p.dim * n_tiles * p.dstate * int64_t(sizeof(float));
}

template <typename T>
int launch_bwd(const mm_scan_bwd_params &p, hipStream_t s) {
    // The accumulated gradients start from zero on the launch stream.
    int rc = bwd::launch_fill(p.dA, 1, 1, p.dim, p.dstate, 0, 0, p.dA_d_stride, p.dA_dstate_stride, s);
    if (rc == MM_OK && p.is_variable_B)
        rc = bwd::launch_fill(p.dB, p.batch, p.n_groups, p.dstate, p.seqlen, p.dB_batch_stride, p.dB_group_stride,
                              p.dB_dstate_stride, 1, s);
    if (rc == MM_OK && !p.is_variable_B)
        rc = bwd::launch_fill(p.dB, 1, 1, p.dim, p.dstate, 0, 0, p.dB_d_stride, p.dB_dstate_stride, s);
    if (rc == MM_OK && p.is_variable_C)
        rc = bwd::launch_fill(p.dC, p.batch, p.n_groups, p.dstate, p.seqlen, p.dC_batch_stride, p.dC_group_stride,
                              p.dC_dstate_stride, 1, s);
    if (rc == MM_OK && !p.is_variable_C)
        rc = bwd::launch_fill(p.dC, 1, 1, p.dim, p.dstate, 0, 0, p.dC_d_stride, p.dC_dstate_stride, s);
    if (rc == MM_OK && p.dD) rc = bwd::launch_fill(p.dD, 1, 1, 1, p.dim, 0, 0, 0, 1, s);
    if (rc == MM_OK && p.ddelta_bias) rc = bwd::launch_fill(p.ddelta_bias, 1, 1, 1, p.dim, 0, 0, 0, 1, s);
    if (rc != MM_OK) return rc;
    if (p.seqlen == 0) return MM_OK;
    return bwd::launch_general<T>(p, s);
}

template int launch_bwd<float>(const mm_scan_bwd_params &, hipStream_t);
template int launch_bwd<f16_t>(const mm_scan_bwd_params &, hipStream_t);
template int launch_bwd<bf16_t>(const mm_scan_bwd_params &, hipStream_t);

}  // namespace mm
