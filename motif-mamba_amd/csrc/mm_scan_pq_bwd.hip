// mm_scan_pq_bwd.hip -- gfx950 backward of the MotifMamba low-rank coupled scan.
//
// Reference behaviour: the gradients torch autograd takes through selective_scan_full_matrix_cuda
// (mamba_ssm/ops/selective_scan_interface.py:262-350), the path selective_scan_fn takes for P/Q
// calls with z (selective_scan_interface.py:243-258, the Motif module always passes z), i.e. the
// exact gradients of
//
//     h_t = a_t * h_{t-1} + dt'_t P (Q h_{t-1}) + dt'_t u_t B_t,   a_t = exp(dt'_t A),
//     y_t = C_t . h_t,   out_t = y_t + D u_t,   out_z_t = out_t * silu(z_t).
//
// With g_t = dout_t * silu(z_t) and the state adjoint lam_t = dL / dh_t (a reverse recurrence
// through the transposed transition matrix M_{t+1} = diag(a_{t+1}) + dt'_{t+1} P Q):
//
//     lam_t  = C_t g_t + a_{t+1} * lam_{t+1} + dt'_{t+1} Q^T (P^T lam_{t+1}),     lam_{L-1} = C g
//     dt'_t  = sum_n lam_t (A a_t h_{t-1} + (P q_t) + u_t B_t),    q_t = Q h_{t-1}
//     du_t   = D g_t + dt'_t sum_n lam_t B_t
//     dA    += lam_t dt'_t a_t h_{t-1};  dP += dt'_t lam_t q_t^T;  dQ += dt'_t (P^T lam_t) h_{t-1}^T
//     dB_t  += lam_t dt'_t u_t;  dC_t += g_t h_t;  dD += g_t u_t;  dz, ddelta_bias as the diagonal case.
//
// The design of this file is its own. scan_bwd_pq16<T, S, R>: a workgroup owns 16 channels of one
// (batch, group) and dstate <= 16 states; the LPR = 16 / S consecutive lanes of a channel hold S
// states each (S = 2: 8 lanes per channel, two waves per workgroup), and the sums over a channel's
// states (Q h, P^T lam, and the per-step sums that give du and ddelta) are DPP butterflies inside
// those lanes, which leave bit-identical totals in all of them (the R sums of Q h and of P^T lam
// each as one transposed butterfly, lane_sums). P and Q of the lane's states live
// in registers. The states at every 16-step tile start come from the forward (its tile_states) or,
// without them, from a first pass that recomputes the forward into the caller's workspace. The
// second pass walks the tiles in reverse: it recomputes each tile from its checkpoint into LDS (the
// states read back by the same lane, Q h_{t-1} by the whole channel) and walks it backwards. The
// dB / dC contributions are summed over the block's 16 channels through LDS per 4 steps (so that
// the 37-39 KB of LDS let four workgroups share a CU) and written as the block's partials, which
// scan_bwd_reduce_bc adds in block order (no atomics on them); dA, dP, dQ, dD and ddelta_bias take
// float32 atomics once per lane at the end.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mm_common.h"
#include "mm_internal.h"

namespace mm {
namespace pqbwd {

constexpr int kT = 16;           // steps per tile
constexpr int kH = 4;            // steps per dB / dC reduction
constexpr int kXS = kT + 1;      // sX row stride (float4)
constexpr int kBCS = 36;         // sBC row stride (floats): B 16 | C 16 | pad 4
constexpr int kRow = 20;         // sRed row stride (floats): 16 channels + 4
constexpr int kRed = 2 * kH * 16 * kRow;   // sRed floats: [tensor][step of the half][state][channel]

template <typename T, int S, int R>
__global__ void __launch_bounds__(16 * (16 / S)) __attribute__((amdgpu_waves_per_eu(2)))
scan_bwd_pq16(const mm_scan_bwd_params p, const int64_t ratio, float *const ck, float *const partB,
              float *const partC) {
    constexpr int LPR = 16 / S;          // lanes per channel
    constexpr int NT = 16 * LPR;         // lanes per workgroup
    constexpr int E = kT / LPR;          // steps per lane of a tile's per-element work
    __shared__ __align__(16) float4 sX[16 * kXS];       // [c][t]: (dt', dt'u, u, g)
    __shared__ __align__(16) float sBC[kT * kBCS];       // [t][B 16 | C 16]
    __shared__ __align__(16) float sRed[kRed];           // [tensor][t % kH][n][c]
    __shared__ __align__(16) float sHS[kT * 16 * 16];    // [t][c][n]: the tile's states after step t
    __shared__ __align__(16) float sOwn[2 * 16 * kT];    // [sum of lam B | dt' term][c][t]
    __shared__ __align__(16) float sQ[kT * 16 * R];      // [t][c][r]: Q h_{t-1} of the tile's steps

    const int tid = threadIdx.x;
    const int cw = tid / LPR;              // channel of the block
    const int k = tid % LPR;               // states k S .. k S + S - 1
    const int64_t b = blockIdx.y;
    const int64_t d0 = int64_t(blockIdx.x) * 16;
    const int64_t d = d0 + cw;
    const int64_t g = d0 / ratio;
    const int64_t blk = (d0 - g * ratio) / 16;
    const int64_t L = p.seqlen;
    const int N = int(p.dstate);
    const int rank = int(p.pq_rank);
    const int64_t n_tiles = (L + kT - 1) / kT;
    const int es = E * k;                  // first step (within a tile) of this lane's elements

    const T *up = reinterpret_cast<const T *>(p.u) + b * p.u_batch_stride + d * p.u_d_stride;
    const T *dp = reinterpret_cast<const T *>(p.delta) + b * p.delta_batch_stride + d * p.delta_d_stride;
    const T *zp = p.z ? reinterpret_cast<const T *>(p.z) + b * p.z_batch_stride + d * p.z_d_stride : nullptr;
    const T *outp = p.z ? reinterpret_cast<const T *>(p.out) + b * p.out_batch_stride + d * p.out_d_stride : nullptr;
    const T *gop = reinterpret_cast<const T *>(p.dout) + b * p.dout_batch_stride + d * p.dout_d_stride;
    T *dup = reinterpret_cast<T *>(p.du) + b * p.du_batch_stride + d * p.du_d_stride;
    T *ddp = reinterpret_cast<T *>(p.ddelta) + b * p.ddelta_batch_stride + d * p.ddelta_d_stride;
    T *dzp = p.z ? reinterpret_cast<T *>(p.dz) + b * p.dz_batch_stride + d * p.dz_d_stride : nullptr;
    T *ozp = (p.z && p.out_z) ? reinterpret_cast<T *>(p.out_z) + b * p.out_z_batch_stride + d * p.out_z_d_stride : nullptr;
    const T *Bg = reinterpret_cast<const T *>(p.B) + b * p.B_batch_stride + g * p.B_group_stride;
    const T *Cg = reinterpret_cast<const T *>(p.C) + b * p.C_batch_stride + g * p.C_group_stride;

    // The R sums over a channel's states (Q h and P^T lam) are one transposed reduction over its 8
    // lanes (lane_sums), which wants the lane's rows of Q and columns of P in its order: position t
    // holds rank t ^ ro. Every rank-indexed quantity of the lane (q, P^T lam, dP, dQ) is kept in that
    // order. The forward's 8-lane layout forms Q h the same way, so pass 1 reproduces its tile states
    // bit for bit.
    static_assert(R <= LPR, "one transposed reduction per sum set");
    const int ro = lane_rank_offset<LPR, R>(k);
    float An[S], A2[S], Pr[S][R], Qr[R][S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int n = k * S + s;
        const bool on = n < N;
        An[s] = on ? p.A[d * p.A_d_stride + n * p.A_dstate_stride] : 0.f;
        A2[s] = An[s] * kLog2e;
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const int r = t ^ ro;
            const bool use = on && r < rank;
            Pr[s][t] = use ? p.P[d * p.P_d_stride + n * p.P_dstate_stride + r * p.P_r_stride] : 0.f;
            Qr[t][s] = use ? p.Q[d * p.Q_d_stride + r * p.Q_r_stride + n * p.Q_dstate_stride] : 0.f;
        }
    }
    // Q h over the channel's states, rank t ^ ro in q[t].
    auto qh = [&](const float *h, float (&q)[R]) {
#pragma unroll
        for (int t = 0; t < R; ++t) {
            q[t] = Qr[t][0] * h[0];
#pragma unroll
            for (int s = 1; s < S; ++s) q[t] = __builtin_fmaf(Qr[t][s], h[s], q[t]);
        }
        lane_sums<LPR, R>(q);
    };
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    // Checkpoints [tile][batch][dim][16] (states past dstate stay 0).
    const int64_t ck_tile = p.batch * p.dim * 16;
    float *const ckp = ck + (b * p.dim + d) * 16 + k * S;

    // B/C staging of one tile (32 rows (tensor, state) of kT steps): NT / 32 lanes per row, SPL
    // consecutive steps each.
    constexpr int SPL = kT / (NT / 32);    // steps per staging lane (NT / 32 lanes per row)
    const int st_row = tid / (NT / 32);    // 0 .. 31: tensor st_row / 16, state st_row % 16
    const int st_t0 = SPL * (tid % (NT / 32));
    const int st_n = st_row % 16;
    const bool st_on = st_n < N;
    const T *stp = (st_row < 16 ? Bg + int64_t(st_on ? st_n : 0) * p.B_dstate_stride
                                : Cg + int64_t(st_on ? st_n : 0) * p.C_dstate_stride);

    // A tile's global inputs, loaded one tile ahead of their use (raw, converted at commit):
    // delta, u, dout, z, out of this lane's E elements, its SPL staged B or C values and the
    // checkpoint. Addresses past L are clamped to the row's last element (their steps are padding).
    struct TileIn {
        T d[E], u[E], go[E], z[E], o[E], bc[SPL];
        float hck[S];
    };
    auto fetch = [&](int64_t j, bool full, bool with_ck) {
        TileIn r;
        const int64_t t0 = j * kT;
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const int64_t t = t0 + es + i;
            const int64_t tc = t < L ? t : L - 1;
            r.d[i] = dp[tc];
            r.u[i] = up[tc];
            if (full) {
                r.go[i] = gop[tc];
                if (zp) {
                    r.z[i] = zp[tc];
                    r.o[i] = outp[tc];
                }
            }
        }
        if (full || st_row < 16) {
#pragma unroll
            for (int i = 0; i < SPL; ++i) {
                const int64_t t = t0 + st_t0 + i;
                r.bc[i] = stp[t < L ? t : L - 1];
            }
        }
        if (with_ck) {
#pragma unroll
            for (int s = 0; s < S; ++s) r.hck[s] = ckp[j * ck_tile + s];
        }
        return r;
    };

    // Tile j's per-step values into LDS (with B, and C when `full`); this lane's elements kept in
    // registers; dz and out_z written. Steps past L are padding (dt' = g = 0, B = C = 0: inert).
    float e_raw[E], e_dt[E], e_u[E], e_g[E];
    auto commit = [&](int64_t j, bool full, const TileIn &r) {
        const int64_t t0 = j * kT;
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const int64_t t = t0 + es + i;
            const bool ev = t < L;
            const float dd = to_f32(r.d[i]);
            const float uu = to_f32(r.u[i]);
            float go = 0.f;
            if (full) {
                go = to_f32(r.go[i]);
                if (zp) {
                    const float zz = to_f32(r.z[i]);
                    const float oo = to_f32(r.o[i]);
                    const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-zz * kLog2e));
                    if (ev) {
                        dzp[t] = from_f32<T>(go * oo * sg * (1.f + zz * (1.f - sg)));
                        if (ozp) ozp[t] = from_f32<T>(oo * zz * sg);
                    }
                    go *= zz * sg;
                }
            }
            e_raw[i] = dd + bias;
            e_dt[i] = ev ? (p.delta_softplus ? softplus_fast(e_raw[i]) : e_raw[i]) : 0.f;
            e_u[i] = uu;
            e_g[i] = ev ? go : 0.f;
            sX[cw * kXS + es + i] = make_float4(e_dt[i], e_dt[i] * uu, uu, e_g[i]);
        }
        if (full || st_row < 16) {
#pragma unroll
            for (int i = 0; i < SPL; ++i) {
                const int64_t t = t0 + st_t0 + i;
                const bool on = st_on && t < L;
                sBC[(st_t0 + i) * kBCS + st_row] = on ? to_f32(r.bc[i]) : 0.f;
            }
        }
    };

    // ---- Pass 1: the states before every tile (skipped when the forward wrote them) ----
    if (!p.tile_states) {
        float h[S];
#pragma unroll
        for (int s = 0; s < S; ++s) h[s] = 0.f;
        TileIn in = fetch(0, false, false);
        for (int64_t j = 0; j < n_tiles; ++j) {
#pragma unroll
            for (int s = 0; s < S; ++s) ckp[j * ck_tile + s] = h[s];
            commit(j, false, in);
            if (j + 1 < n_tiles) in = fetch(j + 1, false, false);   // in flight during this tile
            __syncthreads();
#pragma unroll
            for (int t = 0; t < kT; ++t) {
                const float4 x = sX[cw * kXS + t];
                float q[R];
                qh(h, q);
#pragma unroll
                for (int r = 0; r < R; ++r) q[r] *= x.x;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    float w = x.y * sBC[t * kBCS + k * S + s];
#pragma unroll
                    for (int r = 0; r < R; ++r) w = __builtin_fmaf(Pr[s][r], q[r], w);
                    h[s] = __builtin_fmaf(decay_exp2(x.x, A2[s]), h[s], w);
                }
            }
            __syncthreads();
        }
    }

    // ---- Pass 2: tiles in reverse order ----
    float carry[S], dA[S], dP[S][R], dQ[R][S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        carry[s] = 0.f;
        dA[s] = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            dP[s][r] = 0.f;
            dQ[r][s] = 0.f;
        }
    }
    float dD_acc = 0.f, dbias_acc = 0.f;
    TileIn in = fetch(n_tiles - 1, true, true);
    for (int64_t j = n_tiles - 1; j >= 0; --j) {
        const int64_t t0 = j * kT;
        float hck[S];
#pragma unroll
        for (int s = 0; s < S; ++s) hck[s] = in.hck[s];
        commit(j, true, in);
        if (j > 0) in = fetch(j - 1, true, true);                  // in flight during this tile
        __syncthreads();
        // Recompute the tile's states from its checkpoint into sHS (read back by this lane only).
        {
            float h[S];
#pragma unroll
            for (int s = 0; s < S; ++s) h[s] = hck[s];
#pragma unroll 2
            for (int t = 0; t < kT; ++t) {
                const float4 x = sX[cw * kXS + t];
                float q[R];
                qh(h, q);
                // Q h_{t-1} in rank order, read by the whole channel: lane 0 of the channel (rank
                // offset 0) holds it in order.
                if (k == 0) {
#pragma unroll
                    for (int r = 0; r < R; r += 2)
                        *reinterpret_cast<float2 *>(&sQ[(t * 16 + cw) * R + r]) = make_float2(q[r], q[r + 1]);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) q[r] *= x.x;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    float w = x.y * sBC[t * kBCS + k * S + s];
#pragma unroll
                    for (int r = 0; r < R; ++r) w = __builtin_fmaf(Pr[s][r], q[r], w);
                    h[s] = __builtin_fmaf(decay_exp2(x.x, A2[s]), h[s], w);
                    sHS[(t * 16 + cw) * 16 + k * S + s] = h[s];
                }
            }
        }
        __syncthreads();                             // sQ is read by every lane of the channel
        float hc[S];                                 // h_t of the step being walked
#pragma unroll
        for (int s = 0; s < S; ++s) hc[s] = sHS[((kT - 1) * 16 + cw) * 16 + k * S + s];
        for (int tg = kT - kH; tg >= 0; tg -= kH) {
#pragma unroll 2
        for (int ti = kH - 1; ti >= 0; --ti) {
            const int t = tg + ti;
            const int sh = ti;
            const float4 x = sX[cw * kXS + t];       // dt', dt'u, u, g
            float Bv[S], Cv[S], lam[S], hp[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                Bv[s] = sBC[t * kBCS + k * S + s];
                Cv[s] = sBC[t * kBCS + 16 + k * S + s];
                lam[s] = __builtin_fmaf(Cv[s], x.w, carry[s]);
                hp[s] = t > 0 ? sHS[((t - 1) * 16 + cw) * 16 + k * S + s] : hck[s];   // h_{t-1}
            }
            // Q h_{t-1} and P^T lam_t, rank t ^ ro at position t (as Pr, Qr, dP and dQ).
            float q[R], sv[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                q[r] = sQ[(t * 16 + cw) * R + (r ^ ro)];
                sv[r] = Pr[0][r] * lam[0];
#pragma unroll
                for (int s = 1; s < S; ++s) sv[r] = __builtin_fmaf(Pr[s][r], lam[s], sv[r]);
            }
            lane_sums<LPR, R>(sv);
            float pdd = 0.f, pgb = 0.f;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float a = decay_exp2(x.x, A2[s]);
                const float ah = a * hp[s];
                float pq = 0.f, qs = 0.f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    pq = __builtin_fmaf(Pr[s][r], q[r], pq);
                    qs = __builtin_fmaf(Qr[r][s], sv[r], qs);
                }
                // dt' term: A a h_{t-1} + P q + u B
                pdd = __builtin_fmaf(lam[s], __builtin_fmaf(An[s], ah, __builtin_fmaf(x.z, Bv[s], pq)), pdd);
                pgb = __builtin_fmaf(lam[s], Bv[s], pgb);
                const float ld = lam[s] * x.x;
                dA[s] = __builtin_fmaf(ld, ah, dA[s]);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    dP[s][r] = __builtin_fmaf(ld, q[r], dP[s][r]);
                    dQ[r][s] = __builtin_fmaf(x.x * sv[r], hp[s], dQ[r][s]);
                }
                sRed[((0 * kH + sh) * 16 + k * S + s) * kRow + cw] = lam[s] * x.y;   // dB contribution
                sRed[((1 * kH + sh) * 16 + k * S + s) * kRow + cw] = x.w * hc[s];    // dC contribution
                carry[s] = __builtin_fmaf(a, lam[s], x.x * qs);                      // into step t - 1
                hc[s] = hp[s];
            }
            const float dd_t = group_sum<LPR>(pdd), gb_t = group_sum<LPR>(pgb);
            if (t / E == k) {                 // this lane owns step t of its channel (and reads it back)
                sOwn[(0 * 16 + cw) * kT + t] = gb_t;
                sOwn[(1 * 16 + cw) * kT + t] = dd_t;
            }
            if (sh == 0) {
                __syncthreads();
                // dB / dC of the last kH steps summed over the block's 16 channels, in channel order,
                // written as this block's partials: 2 x kH x 16 rows (tensor, step, state).
#pragma unroll
                for (int rr = 0; rr < (2 * kH * 16) / NT; ++rr) {
                    const int row = tid + NT * rr;
                    const int tz = row / (kH * 16), th = (row / 16) % kH, tn = row % 16;
                    const float4 *rv = reinterpret_cast<const float4 *>(&sRed[((tz * kH + th) * 16 + tn) * kRow]);
                    float q4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float4 v = rv[i];
                        q4[i] = (v.x + v.y) + (v.z + v.w);
                    }
                    const float acc = (q4[0] + q4[1]) + (q4[2] + q4[3]);
                    const int64_t ts = t0 + t + th;
                    if (ts < L && tn < N)
                        (tz == 0 ? partB : partC)[(((blk * p.batch + b) * p.n_groups + g) * 16 + tn) * L + ts] = acc;
                }
                __syncthreads();
            }
        }
        }
        // du / ddelta of this lane's steps.
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const int64_t te = t0 + es + i;
            if (te < L) {
                const float gb = sOwn[(0 * 16 + cw) * kT + es + i], ddt = sOwn[(1 * 16 + cw) * kT + es + i];
                const float du = __builtin_fmaf(Dv, e_g[i], e_dt[i] * gb);
                const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-e_raw[i] * kLog2e));
                const float ddl = (p.delta_softplus && e_raw[i] <= 20.f) ? ddt * sg : ddt;
                dup[te] = from_f32<T>(du);
                ddp[te] = from_f32<T>(ddl);
                dD_acc = __builtin_fmaf(e_g[i], e_u[i], dD_acc);
                dbias_acc += ddl;
            }
        }
    }
    // dP[s][t] and dQ[t][s] hold rank t ^ ro.
    const bool shared_pq = p.dP_d_stride == 0 && p.dQ_d_stride == 0;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int n = k * S + s;
        if (n >= N) continue;
        atomicAdd(p.dA + d * p.dA_d_stride + n * p.dA_dstate_stride, dA[s]);
        if (shared_pq) continue;
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const int r = t ^ ro;
            if (r >= rank) continue;
            atomicAdd(p.dP + d * p.dP_d_stride + n * p.dP_dstate_stride + r * p.dP_r_stride, dP[s][t]);
            atomicAdd(p.dQ + d * p.dQ_d_stride + r * p.dQ_r_stride + n * p.dQ_dstate_stride, dQ[t][s]);
        }
    }
    if (p.dD) atomicAdd(p.dD + d, dD_acc);
    if (p.ddelta_bias) atomicAdd(p.ddelta_bias + d, dbias_acc);
    if (shared_pq) {
        // One dP / dQ shared by every channel: the block's 16 channels are summed in LDS first
        // (sHS is free now), so that each element takes one atomic per block, not one per lane.
        static_assert(2 * 16 * R * 16 <= kT * 16 * 16, "the shared-P/Q sums fit sHS");
        __syncthreads();
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int t = 0; t < R; ++t) {
                const int r = t ^ ro;
                sHS[((0 * 16 + k * S + s) * R + r) * 16 + cw] = dP[s][t];
                sHS[((1 * 16 + k * S + s) * R + r) * 16 + cw] = dQ[t][s];
            }
        }
        __syncthreads();
        for (int e = tid; e < 2 * 16 * R; e += NT) {
            const int which = e / (16 * R), n = (e / R) % 16, r = e % R;
            if (n >= N || r >= rank) continue;
            const float4 *v = reinterpret_cast<const float4 *>(&sHS[e * 16]);
            float q4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q4[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
            const float acc = (q4[0] + q4[1]) + (q4[2] + q4[3]);
            if (which == 0) atomicAdd(p.dP + n * p.dP_dstate_stride + r * p.dP_r_stride, acc);
            else atomicAdd(p.dQ + r * p.dQ_r_stride + n * p.dQ_dstate_stride, acc);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// scan_bwd_pq_general<T, NP, R>: the P/Q backward for the shapes scan_bwd_pq16 does not take --
// dstate 17 .. 256 (the reference's dense kernel takes dstate <= 256, rank <= 8: the Motif module's
// "small" and "base" presets use dstate 32 and 64, mamba_simplemotif.py:33-35), constant B or C,
// lengths that are not multiples of 8 and channel counts that are not multiples of 16. One lane per
// state: a 256-lane workgroup holds 256 / NP rows (batch, channel), NP the next power of two
// >= max(dstate, 16). The two sums over a row's states that feed the recurrences -- q_t = Q h_{t-1}
// in the forward recompute and P^T lam_t in the reverse walk -- are taken every step as butterflies
// inside a wave (DPP and lane swaps; bit-identical totals in every lane), rows wider than a wave
// adding their waves' totals through LDS; the sums that only give du and ddelta are per-lane partials in
// LDS, added by one lane per step after each 16-step tile. Checkpoints every 16 steps in the
// workspace ([tile][row][NP]). The variable dB/dC terms of a tile are summed over the workgroup's
// rows of one (batch, group) in LDS before their float32 atomics (one per run of such rows, state
// and step); dA, dP, dQ, dD and ddelta_bias are float32 atomics once per lane.
constexpr int kGT = 256;   // lanes per workgroup
constexpr int kGBT = 16;   // steps per checkpoint tile

// Sum of v over the NP lanes of each row, in every lane. sx: (kGT / 64) * R floats of LDS, used
// only when a row spans several waves (then every lane of the workgroup must call this).
template <int NP, int R>
__device__ __forceinline__ void row_allreduce(float (&v)[R], float *sx, int tid) {
    // 16 lanes with DPP (group_sum), then the 16-lane rows of a wave pairwise with
    // v_permlane16_swap and its halves with v_permlane32_swap: every stage adds two equal-valued
    // pairs, so all lanes keep bit-identical totals.
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float x = group_sum<16>(v[r]);
        if constexpr (NP >= 32) {
            const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
            x = __uint_as_float(q[0]) + __uint_as_float(q[1]);
        }
        if constexpr (NP >= 64) {
            const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
            x = __uint_as_float(q[0]) + __uint_as_float(q[1]);
        }
        v[r] = x;
    }
    if constexpr (NP > 64) {
        constexpr int WPR = NP / 64;   // waves per row
        const int wave = tid >> 6;
        __syncthreads();               // the previous call's reads of sx are done
        if ((tid & 63) == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) sx[wave * R + r] = v[r];
        }
        __syncthreads();
        const int w0 = wave - wave % WPR;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float acc = sx[w0 * R + r];
            for (int w = 1; w < WPR; ++w) acc += sx[(w0 + w) * R + r];
            v[r] = acc;
        }
    }
}

template <typename T, int NP, int R>
__global__ void __launch_bounds__(kGT)
scan_bwd_pq_general(const mm_scan_bwd_params p, const int64_t ratio, float *const ck, float *const partB,
                    float *const partC) {
    constexpr int RPW = kGT / NP;                        // rows per workgroup
    __shared__ float sDu[kGBT * kGT];                    // [step][lane]: lam B
    __shared__ float sDdt[kGBT * kGT];                   // [step][lane]: the delta' derivative's term
    __shared__ float sQ[RPW * kGBT * R];                 // [row][step][r]: q_t of the tile
    __shared__ float sB[kGBT * kGT];                     // [step][lane]: dB terms of the tile
    __shared__ float sC[kGBT * kGT];                     // [step][lane]: dC terms of the tile
    __shared__ float sX[(NP > 64 ? kGT / 64 : 1) * R];   // waves' totals of the wider rows
    const int tid = threadIdx.x;
    const int slot = tid / NP;
    const int n = tid % NP;
    const int N = int(p.dstate);
    const int rank = int(p.pq_rank);
    const int64_t rows = p.batch * p.dim;
    const int64_t r_ = int64_t(blockIdx.x) * RPW + slot;
    const bool row_ok = r_ < rows;
    const int64_t rr = row_ok ? r_ : rows - 1;           // clamped for loads; stores are predicated
    const int64_t b = rr / p.dim;
    const int64_t d = rr - b * p.dim;
    const int64_t g = d / ratio;
    const bool on = row_ok && n < N;
    const int nn = n < N ? n : N - 1;
    const int64_t L = p.seqlen;
    const int64_t n_tiles = (L + kGBT - 1) / kGBT;

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
    const float Bc = p.is_variable_B ? 0.f : reinterpret_cast<const float *>(p.B)[d * p.B_d_stride + nn * p.B_dstate_stride];
    const float Cc = p.is_variable_C ? 0.f : reinterpret_cast<const float *>(p.C)[d * p.C_d_stride + nn * p.C_dstate_stride];
    // Lanes past dstate hold zero A, B, C, P and Q: their state and adjoint stay zero and they add
    // nothing to any sum.
    const float An = on ? p.A[d * p.A_d_stride + nn * p.A_dstate_stride] : 0.f;
    const float A2 = An * kLog2e;
    float Pn[R], Qn[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const bool use = on && r < rank;
        Pn[r] = use ? p.P[d * p.P_d_stride + nn * p.P_dstate_stride + r * p.P_r_stride] : 0.f;
        Qn[r] = use ? p.Q[d * p.Q_d_stride + r * p.Q_r_stride + nn * p.Q_dstate_stride] : 0.f;
    }
    const float Dv = p.D ? p.D[d] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
    const int64_t ck_tile = rows * NP;
    float *const ckr = ck + rr * NP + n;

    auto dt_at = [&](int64_t t, float &raw) {
        raw = to_f32(dp[t]) + bias;
        return p.delta_softplus ? softplus_fast(raw) : raw;
    };
    auto b_at = [&](int64_t t) { return on ? (Bv ? to_f32(Bv[t]) : Bc) : 0.f; };
    auto c_at = [&](int64_t t) { return on ? (Cv ? to_f32(Cv[t]) : Cc) : 0.f; };
    // g_t = dout_t silu(z_t) (or dout_t); `writer` also writes dz_t (and out_z_t).
    auto g_at = [&](int64_t t, bool writer) {
        float go = to_f32(gop[t]);
        if (zp) {
            const float zz = to_f32(zp[t]);
            const float sg = 1.f / (1.f + expf(-zz));
            if (writer) {
                const float o = to_f32(outp[t]);
                dzp[t] = from_f32<T>(go * o * sg * (1.f + zz * (1.f - sg)));
                if (ozp) ozp[t] = from_f32<T>(o * zz * sg);
            }
            go *= zz * sg;
        }
        return go;
    };

    // Pass 1: the states at every tile start.
    float h = 0.f;
    for (int64_t t = 0; t < L; ++t) {
        if (t % kGBT == 0 && row_ok) ckr[(t / kGBT) * ck_tile] = h;
        float raw;
        const float dt = dt_at(t, raw);
        float q[R];
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = Qn[r] * h;
        row_allreduce<NP, R>(q, sX, tid);
        float pq = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) pq = __builtin_fmaf(Pn[r], q[r], pq);
        h = __builtin_fmaf(decay_exp2(dt, A2), h, dt * __builtin_fmaf(to_f32(up[t]), b_at(t), pq));
    }
    __syncthreads();

    // Pass 2: tiles in reverse order. lam is the state adjoint, pl = P^T lam of the step after.
    float lam = 0.f, a_next = 0.f, dt_next = 0.f, pl[R];
    float dA_acc = 0.f, dBc = 0.f, dCc = 0.f, dD_acc = 0.f, dbias_acc = 0.f, dP_acc[R], dQ_acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pl[r] = dP_acc[r] = dQ_acc[r] = 0.f;
    for (int64_t j = n_tiles - 1; j >= 0; --j) {
        const int64_t t0 = j * kGBT;
        const int cnt = int(L - t0 < kGBT ? L - t0 : kGBT);   // the same in every lane
        float hp[kGBT], hs[kGBT], as[kGBT], dts[kGBT], us[kGBT];
        float hh = row_ok ? ckr[j * ck_tile] : 0.f;
#pragma unroll
        for (int s = 0; s < kGBT; ++s) {
            if (s < cnt) {
                const int64_t t = t0 + s;
                float raw;
                dts[s] = dt_at(t, raw);
                us[s] = to_f32(up[t]);
                as[s] = decay_exp2(dts[s], A2);
                hp[s] = hh;
                float q[R];
#pragma unroll
                for (int r = 0; r < R; ++r) q[r] = Qn[r] * hh;
                row_allreduce<NP, R>(q, sX, tid);
                float pq = 0.f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    pq = __builtin_fmaf(Pn[r], q[r], pq);
                    if (n == r) sQ[(slot * kGBT + s) * R + r] = q[r];
                }
                hh = __builtin_fmaf(as[s], hh, dts[s] * __builtin_fmaf(us[s], b_at(t), pq));
                hs[s] = hh;
            }
        }
        __syncthreads();   // sQ of the tile
        float dA_tile = 0.f, dB_tile = 0.f, dC_tile = 0.f;
#pragma unroll
        for (int s = kGBT - 1; s >= 0; --s) {
            if (s < cnt) {
                const int64_t t = t0 + s;
                const float gt = g_at(t, row_ok && n == 0);
                const float bn = b_at(t);
                // lam_t = C_t g_t + a_{t+1} lam_{t+1} + dt'_{t+1} Q^T (P^T lam_{t+1})
                float qpl = 0.f;
#pragma unroll
                for (int r = 0; r < R; ++r) qpl = __builtin_fmaf(Qn[r], pl[r], qpl);
                lam = __builtin_fmaf(c_at(t), gt, __builtin_fmaf(a_next, lam, dt_next * qpl));
#pragma unroll
                for (int r = 0; r < R; ++r) pl[r] = Pn[r] * lam;
                row_allreduce<NP, R>(pl, sX, tid);
                float pq = 0.f;
                const float ldt = lam * dts[s];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float q = sQ[(slot * kGBT + s) * R + r];
                    pq = __builtin_fmaf(Pn[r], q, pq);
                    dP_acc[r] = __builtin_fmaf(ldt, q, dP_acc[r]);
                    dQ_acc[r] = __builtin_fmaf(dts[s] * pl[r], hp[s], dQ_acc[r]);
                }
                const float ah = as[s] * hp[s];            // a_t h_{t-1}
                const float dcv = gt * hs[s];
                const float dbv = ldt * us[s];
                sB[s * kGT + tid] = dbv;
                sC[s * kGT + tid] = dcv;
                dC_tile += dcv;
                dB_tile += dbv;
                dA_tile = __builtin_fmaf(ldt, ah, dA_tile);
                sDu[s * kGT + tid] = lam * bn;
                sDdt[s * kGT + tid] = lam * __builtin_fmaf(An, ah, __builtin_fmaf(us[s], bn, pq));
                a_next = as[s];
                dt_next = dts[s];
            }
        }
        dA_acc += dA_tile;
        dBc += dB_tile;
        dCc += dC_tile;
        __syncthreads();
        // The variable dB / dC of the tile: per (step, state), the terms of consecutive rows of one
        // (batch, group) added in row order -- into this workgroup's slab when there is one (its
        // rows are then all of one (batch, group)), else one atomic per such run.
        if (partB || partC) {
            const int64_t row0 = int64_t(blockIdx.x) * RPW;
            const int64_t b0 = row0 / p.dim, d0 = row0 - b0 * p.dim, g0 = d0 / ratio;
            const int64_t blk = (d0 - g0 * ratio) / RPW;
            float *const slabB = partB ? partB + ((blk * p.batch + b0) * p.n_groups + g0) * N * L : nullptr;
            float *const slabC = partC ? partC + ((blk * p.batch + b0) * p.n_groups + g0) * N * L : nullptr;
            for (int e = tid; e < kGBT * NP; e += kGT) {
                const int se = e / NP, ne = e % NP;
                if (se >= cnt || ne >= N) continue;
                float accB = 0.f, accC = 0.f;
                for (int sl = 0; sl < RPW; ++sl) {
                    accB += sB[se * kGT + sl * NP + ne];
                    accC += sC[se * kGT + sl * NP + ne];
                }
                if (slabB) slabB[ne * L + t0 + se] = accB;
                if (slabC) slabC[ne * L + t0 + se] = accC;
            }
        } else if (p.is_variable_B || p.is_variable_C) {
            const int64_t row0 = int64_t(blockIdx.x) * RPW;
            for (int e = tid; e < kGBT * NP; e += kGT) {
                const int se = e / NP, ne = e % NP;
                if (se >= cnt || ne >= N) continue;
                const int64_t t = t0 + se;
                float accB = 0.f, accC = 0.f;
                int64_t key = -1, kb = 0, kg = 0;
                for (int sl = 0; sl < RPW; ++sl) {
                    const int64_t rw = row0 + sl;
                    if (rw >= rows) break;
                    const int64_t bw = rw / p.dim, gw = (rw - bw * p.dim) / ratio;
                    const int64_t kw = bw * p.n_groups + gw;
                    if (kw != key) {
                        if (key >= 0) {
                            if (p.is_variable_B)
                                atomicAdd(p.dB + kb * p.dB_batch_stride + kg * p.dB_group_stride + ne * p.dB_dstate_stride + t, accB);
                            if (p.is_variable_C)
                                atomicAdd(p.dC + kb * p.dC_batch_stride + kg * p.dC_group_stride + ne * p.dC_dstate_stride + t, accC);
                        }
                        key = kw; kb = bw; kg = gw; accB = 0.f; accC = 0.f;
                    }
                    accB += sB[se * kGT + sl * NP + ne];
                    accC += sC[se * kGT + sl * NP + ne];
                }
                if (key >= 0) {
                    if (p.is_variable_B)
                        atomicAdd(p.dB + kb * p.dB_batch_stride + kg * p.dB_group_stride + ne * p.dB_dstate_stride + t, accB);
                    if (p.is_variable_C)
                        atomicAdd(p.dC + kb * p.dC_batch_stride + kg * p.dC_group_stride + ne * p.dC_dstate_stride + t, accC);
                }
            }
        }
        // Per step: the sums over the row's states; the lane of state s finishes step s (NP >= 16).
        if (n < cnt && row_ok) {
            const int s = n;
            float su = 0.f, sd = 0.f;
            for (int k = 0; k < N; ++k) {
                su += sDu[s * kGT + slot * NP + k];
                sd += sDdt[s * kGT + slot * NP + k];
            }
            const int64_t t = t0 + s;
            float raw;
            const float dt = dt_at(t, raw);
            const float gt = g_at(t, false);
            const float uu = to_f32(up[t]);
            const float dd = (p.delta_softplus && raw <= 20.f) ? sd / (1.f + expf(-raw)) : sd;
            dup[t] = from_f32<T>(__builtin_fmaf(Dv, gt, dt * su));
            ddp[t] = from_f32<T>(dd);
            dD_acc = __builtin_fmaf(gt, uu, dD_acc);
            dbias_acc += dd;
        }
        __syncthreads();   // sDu, sDdt and sQ are rewritten by the next tile
    }
    if (on) {
        atomicAdd(p.dA + d * p.dA_d_stride + n * p.dA_dstate_stride, dA_acc);
        if (!p.is_variable_B) atomicAdd(p.dB + d * p.dB_d_stride + n * p.dB_dstate_stride, dBc);
        if (!p.is_variable_C) atomicAdd(p.dC + d * p.dC_d_stride + n * p.dC_dstate_stride, dCc);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r < rank) {
                atomicAdd(p.dP + d * p.dP_d_stride + n * p.dP_dstate_stride + r * p.dP_r_stride, dP_acc[r]);
                atomicAdd(p.dQ + d * p.dQ_d_stride + r * p.dQ_r_stride + n * p.dQ_dstate_stride, dQ_acc[r]);
            }
        }
    }
    // dD and ddelta_bias: the per-lane sums of the steps each lane finished (lanes 0 .. 15).
    if (row_ok && n < kGBT) {
        if (p.dD) atomicAdd(p.dD + d, dD_acc);
        if (p.ddelta_bias) atomicAdd(p.ddelta_bias + d, dbias_acc);
    }
}

}  // namespace pqbwd

// The P/Q backward's shape conditions: variable B/C, dstate <= 16, rank 1..8, 16-channel blocks
// inside one group, L a multiple of 8.
bool pq_bwd_ok(const mm_scan_bwd_params &p) {
    return p.is_variable_B && p.is_variable_C && p.dstate >= 1 && p.dstate <= 16 && p.pq_rank >= 1 &&
           p.pq_rank <= 8 && p.dim % 16 == 0 && (p.dim / p.n_groups) % 16 == 0 && p.seqlen >= 8 &&
           p.seqlen % 8 == 0 && p.batch <= 65535;
}

template <typename T, int S>
static int launch_pq_bwd_s(const mm_scan_bwd_params &p, hipStream_t s, float *ck, float *partB, float *partC) {
    const int64_t ratio = p.dim / p.n_groups;
    dim3 grid(unsigned(p.dim / 16), unsigned(p.batch));
    dim3 block(16 * (16 / S));
    if (p.pq_rank <= 2)
        hipLaunchKernelGGL((pqbwd::scan_bwd_pq16<T, S, 2>), grid, block, 0, s, p, ratio, ck, partB, partC);
    else if (p.pq_rank <= 4)
        hipLaunchKernelGGL((pqbwd::scan_bwd_pq16<T, S, 4>), grid, block, 0, s, p, ratio, ck, partB, partC);
    else
        hipLaunchKernelGGL((pqbwd::scan_bwd_pq16<T, S, 8>), grid, block, 0, s, p, ratio, ck, partB, partC);
    return launch_status("scan_bwd_pq16");
}

// Two states per lane: 135-157 registers (two or three waves per SIMD); four states per lane would
// need 187-227 (one wave per SIMD) for fewer butterfly steps.
template <typename T>
int launch_pq_bwd(const mm_scan_bwd_params &p, hipStream_t s, float *ck, float *partB, float *partC) {
    return launch_pq_bwd_s<T, 2>(p, s, ck, partB, partC);
}

int pq_general_np(const mm_scan_bwd_params &p) {   // lanes per row of the general kernel
    int np = 16;
    while (np < p.dstate) np *= 2;
    return np;
}

int64_t pq_general_ck_floats(const mm_scan_bwd_params &p) {
    return ((p.seqlen + pqbwd::kGBT - 1) / pqbwd::kGBT) * p.batch * p.dim * pq_general_np(p);
}

int pq_general_rows_per_block(const mm_scan_bwd_params &p) { return pqbwd::kGT / pq_general_np(p); }

template <typename T, int NP>
static int launch_pq_general_np(const mm_scan_bwd_params &p, hipStream_t s, float *ck, float *partB, float *partC) {
    const int64_t rows = p.batch * p.dim;
    const int64_t blocks = (rows + pqbwd::kGT / NP - 1) / (pqbwd::kGT / NP);
    if (blocks >= (int64_t(1) << 32) / pqbwd::kGT)   // gridDim.x * blockDim.x must stay below 2^32
        return set_error(MM_ERR_UNSUPPORTED, "mm_scan_bwd: batch * dim too large for one launch of the P/Q backward");
    const int64_t ratio = p.dim / p.n_groups;
    if (p.pq_rank <= 2)
        hipLaunchKernelGGL((pqbwd::scan_bwd_pq_general<T, NP, 2>), dim3(unsigned(blocks)), dim3(pqbwd::kGT), 0, s, p,
                           ratio, ck, partB, partC);
    else
        hipLaunchKernelGGL((pqbwd::scan_bwd_pq_general<T, NP, 8>), dim3(unsigned(blocks)), dim3(pqbwd::kGT), 0, s, p,
                           ratio, ck, partB, partC);
    return launch_status("scan_bwd_pq_general");
}

template <typename T>
int launch_pq_general(const mm_scan_bwd_params &p, hipStream_t s, float *ck, float *partB, float *partC) {
    switch (pq_general_np(p)) {
    case 16: return launch_pq_general_np<T, 16>(p, s, ck, partB, partC);
    case 32: return launch_pq_general_np<T, 32>(p, s, ck, partB, partC);
    case 64: return launch_pq_general_np<T, 64>(p, s, ck, partB, partC);
    case 128: return launch_pq_general_np<T, 128>(p, s, ck, partB, partC);
    default: return launch_pq_general_np<T, 256>(p, s, ck, partB, partC);
    }
}

template int launch_pq_general<float>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);
template int launch_pq_general<f16_t>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);
template int launch_pq_general<bf16_t>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);

template int launch_pq_bwd<float>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);
template int launch_pq_bwd<f16_t>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);
template int launch_pq_bwd<bf16_t>(const mm_scan_bwd_params &, hipStream_t, float *, float *, float *);

}  // namespace mm
