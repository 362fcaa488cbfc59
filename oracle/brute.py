"""Pure-Python float64 restatement of the selective scan for tiny shapes -- TEST INFRASTRUCTURE.

Independent of the recurrence form used everywhere else: the state is evaluated as the closed
sum  h_t[n] = sum_{k<=t} (prod_{k<j<=t} a_j[n]) * b_k[n]  with a_j = exp(delta'_j A[d, n]) and
b_k = delta'_k u_k B[.., n, k]  (the solution of the recurrence in ssi.py:422-433), which is
O(L^2) and therefore only used for L of a few tens. Group mapping g(d) = d // (dim / G)
(ssi.py:395-400), softplus with threshold 20 (torch F.softplus), silu(z) = z / (1 + e^-z).
Inputs are nested Python lists (or anything indexable) of floats.

``scan_pq_brute`` does the same for the MotifMamba low-rank coupled scan (ssi.py:320-341) with
explicit N x N transition matrices diag(exp(dt A)) + dt P Q multiplied out step by step.
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
