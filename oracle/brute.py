"""Pure-Python float64 restatement of the selective scan for tiny shapes -- TEST INFRASTRUCTURE.

Independent of the recurrence form used everywhere else: the state is evaluated as the closed
sum  h_t[n] = sum_{k<=t} (prod_{k<j<=t} a_j[n]) * b_k[n]  with a_j = exp(delta'_j A[d, n]) and
b_k = delta'_k u_k B[.., n, k]  (the solution of the recurrence in ssi.py:422-433), which is
O(L^2) and therefore only used for L of a few tens. Group mapping g(d) = d // (dim / G)
(ssi.py:395-400), softplus with threshold 20 (torch F.softplus), silu(z) = z / (1 + e^-z).
Inputs are nested Python lists (or anything indexable) of floats.

``scan_pq_brute`` does the same for the MotifMamba low-rank coupled scan (ssi.py:320-341) with
explicit N x N transition matrices diag(exp(dt A)) + dt P Q multiplied out step by step;
``scan_pq_bwd_brute`` is its reverse-mode adjoint through the transposed dense matrices.
"""
from __future__ import annotations

import math

from .ssm_ref import softplus_f64


def _b_at(B, b, d, n, t, dim, var_kind):
    if var_kind == "const":
        return B[d][n]
    if var_kind == "3d":
        return B[b][n][t]
    G = len(B[b])
    return B[b][d // (dim // G)][n][t]


def scan_brute(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
               b_kind="3d", c_kind="3d"):
    """Returns (out_pre_gate, out_gated_or_None, last_state) as nested lists of float64.
    b_kind / c_kind: "const" (dim, N), "3d" (batch, N, L) or "4d" (batch, G, N, L)."""
    batch = len(u)
    dim = len(u[0])
    L = len(u[0][0])
    N = len(A[0])
    out = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    outz = [[[0.0] * L for _ in range(dim)] for _ in range(batch)] if z is not None else None
    last = [[[0.0] * N for _ in range(dim)] for _ in range(batch)]
    for b in range(batch):
        for d in range(dim):
            dts = []
            for t in range(L):
                x = float(delta[b][d][t]) + (float(delta_bias[d]) if delta_bias is not None else 0.0)
                dts.append(softplus_f64(x) if delta_softplus else x)
            for t in range(L):
                y = 0.0
                for n in range(N):
                    h = 0.0
                    for k in range(t + 1):
                        w = 1.0
                        for j in range(k + 1, t + 1):
                            w *= math.exp(dts[j] * float(A[d][n]))
                        h += w * dts[k] * float(u[b][d][k]) * float(_b_at(B, b, d, n, k, dim, b_kind))
                    y += h * float(_b_at(C, b, d, n, t, dim, c_kind))
                    if t == L - 1:
                        last[b][d][n] = h
                if D is not None:
                    y += float(D[d]) * float(u[b][d][t])
                out[b][d][t] = y
                if z is not None:
                    zz = float(z[b][d][t])
                    outz[b][d][t] = y * zz / (1.0 + math.exp(-zz))
    return out, outz, last


def _matmul(X, Y):
    return [[sum(X[i][k] * Y[k][j] for k in range(len(Y))) for j in range(len(Y[0]))] for i in range(len(X))]


def scan_pq_brute(u, delta, A, B, C, P, Q, D=None, z=None, delta_bias=None, delta_softplus=False,
                  b_kind="3d", c_kind="3d"):
    """Float64 closed sum of the low-rank coupled scan (the recurrence of ssi.py:320-341,
    x_t = exp(dt_t A) * x_{t-1} + dt_t P (Q x_{t-1}) + dt_t u_t B_t), evaluated with explicit
    transition matrices instead of the recurrence:  h_t = sum_{k<=t} (M_t M_{t-1} ... M_{k+1}) b_k,
    M_j = diag(exp(dt_j A[d, :])) + dt_j W_d with the dense N x N product W_d = P_d Q_d, and
    b_k = dt_k u_k B_k. P is (N, R) shared or (dim, N, R) per channel, Q (R, N) or (dim, R, N).
    Returns (out_pre_gate, out_gated_or_None, last_state) as nested lists of float64."""
    batch = len(u)
    dim = len(u[0])
    L = len(u[0][0])
    N = len(A[0])
    per_dim = isinstance(P[0][0], (list, tuple))
    out = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    outz = [[[0.0] * L for _ in range(dim)] for _ in range(batch)] if z is not None else None
    last = [[[0.0] * N for _ in range(dim)] for _ in range(batch)]
    for d in range(dim):
        Pd = P[d] if per_dim else P
        Qd = Q[d] if per_dim else Q
        W = _matmul([[float(v) for v in row] for row in Pd], [[float(v) for v in row] for row in Qd])
        for b in range(batch):
            dts = []
            for t in range(L):
                x = float(delta[b][d][t]) + (float(delta_bias[d]) if delta_bias is not None else 0.0)
                dts.append(softplus_f64(x) if delta_softplus else x)
            Ms = [[[(math.exp(dts[j] * float(A[d][i])) if i == k else 0.0) + dts[j] * W[i][k]
                    for k in range(N)] for i in range(N)] for j in range(L)]
            for t in range(L):
                h = [0.0] * N
                for k in range(t + 1):
                    vec = [[dts[k] * float(u[b][d][k]) * float(_b_at(B, b, d, n, k, dim, b_kind))] for n in range(N)]
                    for j in range(k + 1, t + 1):
                        vec = _matmul(Ms[j], vec)
                    for n in range(N):
                        h[n] += vec[n][0]
                y = sum(h[n] * float(_b_at(C, b, d, n, t, dim, c_kind)) for n in range(N))
                if D is not None:
                    y += float(D[d]) * float(u[b][d][t])
                out[b][d][t] = y
                if z is not None:
                    zz = float(z[b][d][t])
                    outz[b][d][t] = y * zz / (1.0 + math.exp(-zz))
                if t == L - 1:
                    last[b][d] = h
    return out, outz, last


def scan_bwd_brute(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
                   b_kind="3d", c_kind="3d"):
    """Float64 reverse-mode adjoint of the selective scan written out as recurrences (the
    computation of selective_scan_bwd_kernel.cuh:405-880), independent of autograd:

      g_t  = dout_t * silu(z_t)                (z given; dz_t = dout_t * out_t * silu'(z_t))
      gh_t = C_t g_t + a_{t+1} gh_{t+1},  gh_L = 0              (reverse scan, per state)
      dC_t += g_t h_t ; dB_t += gh_t dt_t u_t ; du_t = D g_t + dt_t sum_n gh_t B_t
      ddt_t = sum_n gh_t (u_t B_t + A (a_t h_{t-1})) ; dA += gh_t dt_t a_t h_{t-1}
      ddelta_t = ddt_t * sigmoid(delta_t + bias) (softplus; 1 past the threshold 20)
      dD += g_t u_t ; ddelta_bias += ddelta_t

    Returns a dict of nested lists (du, ddelta, dA, dB, dC, dD, ddelta_bias, dz)."""
    batch, dim, L, N = len(u), len(u[0]), len(u[0][0]), len(A[0])

    def zeros_like_bc(X, kind):
        if kind == "const":
            return [[0.0] * N for _ in range(dim)]
        if kind == "3d":
            return [[[0.0] * L for _ in range(N)] for _ in range(batch)]
        G = len(X[0])
        return [[[[0.0] * L for _ in range(N)] for _ in range(G)] for _ in range(batch)]

    def add_bc(acc, kind, b, d, n, t, v):
        if kind == "const":
            acc[d][n] += v
        elif kind == "3d":
            acc[b][n][t] += v
        else:
            G = len(acc[b])
            acc[b][d // (dim // G)][n][t] += v

    du = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    ddelta = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    dz = [[[0.0] * L for _ in range(dim)] for _ in range(batch)] if z is not None else None
    dA = [[0.0] * N for _ in range(dim)]
    dB = zeros_like_bc(B, b_kind)
    dC = zeros_like_bc(C, c_kind)
    dD = [0.0] * dim if D is not None else None
    dbias = [0.0] * dim if delta_bias is not None else None
    for b in range(batch):
        for d in range(dim):
            raw = [float(delta[b][d][t]) + (float(delta_bias[d]) if delta_bias is not None else 0.0) for t in range(L)]
            dts = [softplus_f64(x) if delta_softplus else x for x in raw]
            uu = [float(u[b][d][t]) for t in range(L)]
            a = [[math.exp(dts[t] * float(A[d][n])) for n in range(N)] for t in range(L)]
            Bv = [[float(_b_at(B, b, d, n, t, dim, b_kind)) for n in range(N)] for t in range(L)]
            Cv = [[float(_b_at(C, b, d, n, t, dim, c_kind)) for n in range(N)] for t in range(L)]
            h = [[0.0] * N for _ in range(L)]
            prev = [0.0] * N
            for t in range(L):
                for n in range(N):
                    h[t][n] = a[t][n] * prev[n] + dts[t] * uu[t] * Bv[t][n]
                prev = h[t]
            g = []
            for t in range(L):
                go = float(dout[b][d][t])
                if z is not None:
                    zz = float(z[b][d][t])
                    sg = 1.0 / (1.0 + math.exp(-zz))
                    y = sum(h[t][n] * Cv[t][n] for n in range(N)) + (float(D[d]) * uu[t] if D is not None else 0.0)
                    dz[b][d][t] = go * y * sg * (1.0 + zz * (1.0 - sg))
                    go = go * zz * sg
                g.append(go)
            gh = [0.0] * N
            for t in range(L - 1, -1, -1):
                for n in range(N):
                    gh[n] = Cv[t][n] * g[t] + (a[t + 1][n] * gh[n] if t + 1 < L else 0.0)
                hprev = h[t - 1] if t > 0 else [0.0] * N
                ddt = 0.0
                s_du = 0.0
                for n in range(N):
                    ah = a[t][n] * hprev[n]
                    add_bc(dC, c_kind, b, d, n, t, g[t] * h[t][n])
                    add_bc(dB, b_kind, b, d, n, t, gh[n] * dts[t] * uu[t])
                    s_du += gh[n] * Bv[t][n]
                    ddt += gh[n] * (uu[t] * Bv[t][n] + float(A[d][n]) * ah)
                    dA[d][n] += gh[n] * dts[t] * ah
                du[b][d][t] = dts[t] * s_du + (float(D[d]) * g[t] if D is not None else 0.0)
                if delta_softplus and raw[t] <= 20.0:
                    ddt *= 1.0 / (1.0 + math.exp(-raw[t]))
                ddelta[b][d][t] = ddt
                if D is not None:
                    dD[d] += g[t] * uu[t]
                if dbias is not None:
                    dbias[d] += ddt
    return {"du": du, "ddelta": ddelta, "dA": dA, "dB": dB, "dC": dC, "dD": dD, "ddelta_bias": dbias, "dz": dz}


def scan_pq_bwd_brute(u, delta, A, B, C, P, Q, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
                      b_kind="3d", c_kind="3d"):
    """Float64 reverse-mode adjoint of the low-rank coupled scan (ssi.py:320-341) written out with
    the dense transition matrices M_t = diag(a_t) + dt_t W, W = P Q (N x N), independent of
    autograd and of the rank-R factorisation:

      h_t  = M_t h_{t-1} + dt_t u_t B_t                          (forward, h_{-1} = 0)
      g_t  = dout_t * silu(z_t)                                  (z given; dz as in scan_bwd_brute)
      lam_t = C_t g_t + M_{t+1}^T lam_{t+1},  lam_L = 0          (reverse scan through M^T)
      dC_t += g_t h_t ; dB_t += lam_t dt_t u_t ; du_t = D g_t + dt_t sum_n lam_t B_t
      ddt_t = sum_n lam_t[n] (A_n a_t[n] h_{t-1}[n] + (W h_{t-1})[n] + u_t B_t[n])
      dA_n += lam_t[n] dt_t a_t[n] h_{t-1}[n] ;  dW += dt_t lam_t h_{t-1}^T
      dP = dW Q^T, dQ = P^T dW (summed over channels when P/Q are shared)
      ddelta_t = ddt_t * sigmoid(delta_t + bias) (softplus; 1 past the threshold 20)

    Returns a dict of nested lists (du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, dP, dQ)."""
    batch, dim, L, N = len(u), len(u[0]), len(u[0][0]), len(A[0])
    per_dim = isinstance(P[0][0], (list, tuple))
    R = len(Q[0]) if per_dim else len(Q)

    def zeros_bc(X, kind):
        if kind == "const":
            return [[0.0] * N for _ in range(dim)]
        if kind == "3d":
            return [[[0.0] * L for _ in range(N)] for _ in range(batch)]
        return [[[[0.0] * L for _ in range(N)] for _ in range(len(X[0]))] for _ in range(batch)]

    def add_bc(acc, kind, b, d, n, t, v):
        if kind == "const":
            acc[d][n] += v
        elif kind == "3d":
            acc[b][n][t] += v
        else:
            acc[b][d // (dim // len(acc[b]))][n][t] += v

    du = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    ddelta = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    dz = [[[0.0] * L for _ in range(dim)] for _ in range(batch)] if z is not None else None
    dA = [[0.0] * N for _ in range(dim)]
    dB = zeros_bc(B, b_kind)
    dC = zeros_bc(C, c_kind)
    dD = [0.0] * dim if D is not None else None
    dbias = [0.0] * dim if delta_bias is not None else None
    dWs = [[[0.0] * N for _ in range(N)] for _ in range(dim)]
    for d in range(dim):
        Pd = [[float(v) for v in row] for row in (P[d] if per_dim else P)]
        Qd = [[float(v) for v in row] for row in (Q[d] if per_dim else Q)]
        W = _matmul(Pd, Qd)
        for b in range(batch):
            raw = [float(delta[b][d][t]) + (float(delta_bias[d]) if delta_bias is not None else 0.0) for t in range(L)]
            dts = [softplus_f64(x) if delta_softplus else x for x in raw]
            uu = [float(u[b][d][t]) for t in range(L)]
            a = [[math.exp(dts[t] * float(A[d][n])) for n in range(N)] for t in range(L)]
            Bv = [[float(_b_at(B, b, d, n, t, dim, b_kind)) for n in range(N)] for t in range(L)]
            Cv = [[float(_b_at(C, b, d, n, t, dim, c_kind)) for n in range(N)] for t in range(L)]
            h = []
            prev = [0.0] * N
            for t in range(L):
                Wh = [sum(W[i][k] * prev[k] for k in range(N)) for i in range(N)]
                cur = [a[t][n] * prev[n] + dts[t] * Wh[n] + dts[t] * uu[t] * Bv[t][n] for n in range(N)]
                h.append(cur)
                prev = cur
            g = []
            for t in range(L):
                go = float(dout[b][d][t])
                if z is not None:
                    zz = float(z[b][d][t])
                    sg = 1.0 / (1.0 + math.exp(-zz))
                    y = sum(h[t][n] * Cv[t][n] for n in range(N)) + (float(D[d]) * uu[t] if D is not None else 0.0)
                    dz[b][d][t] = go * y * sg * (1.0 + zz * (1.0 - sg))
                    go = go * zz * sg
                g.append(go)
            lam = [0.0] * N
            for t in range(L - 1, -1, -1):
                if t + 1 < L:
                    # M_{t+1}^T lam_{t+1}: column i of M_{t+1} dotted with lam
                    nxt = [a[t + 1][i] * lam[i] + dts[t + 1] * sum(W[k][i] * lam[k] for k in range(N))
                           for i in range(N)]
                else:
                    nxt = [0.0] * N
                lam = [Cv[t][n] * g[t] + nxt[n] for n in range(N)]
                hprev = h[t - 1] if t > 0 else [0.0] * N
                Wh = [sum(W[i][k] * hprev[k] for k in range(N)) for i in range(N)]
                ddt = 0.0
                s_du = 0.0
                for n in range(N):
                    ah = a[t][n] * hprev[n]
                    add_bc(dC, c_kind, b, d, n, t, g[t] * h[t][n])
                    add_bc(dB, b_kind, b, d, n, t, lam[n] * dts[t] * uu[t])
                    s_du += lam[n] * Bv[t][n]
                    ddt += lam[n] * (float(A[d][n]) * ah + Wh[n] + uu[t] * Bv[t][n])
                    dA[d][n] += lam[n] * dts[t] * ah
                    for k in range(N):
                        dWs[d][n][k] += dts[t] * lam[n] * hprev[k]
                du[b][d][t] = dts[t] * s_du + (float(D[d]) * g[t] if D is not None else 0.0)
                if delta_softplus and raw[t] <= 20.0:
                    ddt *= 1.0 / (1.0 + math.exp(-raw[t]))
                ddelta[b][d][t] = ddt
                if D is not None:
                    dD[d] += g[t] * uu[t]
                if dbias is not None:
                    dbias[d] += ddt
    dPs, dQs = [], []
    for d in range(dim):
        Pd = [[float(v) for v in row] for row in (P[d] if per_dim else P)]
        Qd = [[float(v) for v in row] for row in (Q[d] if per_dim else Q)]
        QdT = [[Qd[r][n] for r in range(R)] for n in range(N)]
        PdT = [[Pd[n][r] for n in range(N)] for r in range(R)]
        dPs.append(_matmul(dWs[d], QdT))
        dQs.append(_matmul(PdT, dWs[d]))
    if per_dim:
        dP, dQ = dPs, dQs
    else:
        dP = [[sum(dPs[d][n][r] for d in range(dim)) for r in range(R)] for n in range(N)]
        dQ = [[sum(dQs[d][r][n] for d in range(dim)) for n in range(N)] for r in range(R)]
    return {"du": du, "ddelta": ddelta, "dA": dA, "dB": dB, "dC": dC, "dD": dD, "ddelta_bias": dbias, "dz": dz,
            "dP": dP, "dQ": dQ}
