"""ctypes wrapper of scan_f64.c -- TEST INFRASTRUCTURE ONLY.

``build()`` compiles ``scan_f64.c`` with gcc (OpenMP) into ``oracle/_build/libscan_f64.so``;
``scan_rows`` evaluates selected (batch, dim) rows of a selective scan in float64 on the host.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "scan_f64.c")
_LIB = os.path.join(_HERE, "_build", "libscan_f64.so")
_lib = None


def build(force: bool = True) -> str:
    """Compile the float64 oracle (gcc -O2 -fopenmp). Returns the library path."""
    os.makedirs(os.path.dirname(_LIB), exist_ok=True)
    if force or not os.path.exists(_LIB):
        tmp = _LIB + ".tmp"
        subprocess.check_call(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-std=c11",
                               _SRC, "-o", tmp, "-lm"])
        os.replace(tmp, _LIB)
    return _LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build(force=False)
        lib = ctypes.CDLL(_LIB)
        f = lib.mm_oracle_scan_rows_f64
        i64, dp = ctypes.c_int64, ctypes.c_void_p
        f.argtypes = [i64, i64, i64, dp, dp, dp, dp,
                      dp, i64, i64, i64, dp, i64, i64, i64,
                      dp, dp, ctypes.c_int, dp, dp, dp, i64, dp]
        f.restype = None
        h = lib.mm_oracle_scan_bwd_rows_f64
        h.argtypes = [i64, i64, i64, dp, dp, dp, dp, dp, i64, i64, dp, i64, i64,
                      dp, dp, ctypes.c_int, dp, dp, dp, dp, dp, dp, dp, dp, dp]
        h.restype = None
        g = lib.mm_oracle_scan_pq_rows_f64
        g.argtypes = [i64, i64, i64, i64, dp, dp, dp, dp,
                      dp, i64, i64, i64, dp, i64, i64, i64,
                      dp, i64, dp, i64,
                      dp, dp, ctypes.c_int, dp, dp, dp, i64, dp]
        g.restype = None
        _lib = lib
    return _lib


def torch_index(i):
    import torch
    return torch.from_numpy(i)


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def scan_rows(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
              rows=None, chunk=0, P=None, Q=None):
    """Float64 scan of the rows ``rows`` (list of (b, d) pairs; all rows if None).

    With P and Q (2-D (N, R) / (R, N) shared, or 3-D (dim, N, R) / (dim, R, N) per channel) the
    low-rank coupled scan ``mm_oracle_scan_pq_rows_f64`` is evaluated instead.

    Tensors are torch CPU tensors or numpy arrays in the reference layouts (u/delta/z
    (batch, dim, L); A (dim, N); B/C (dim, N), (batch, N, L) or (batch, G, N, L)).
    Returns dict with 'out' (R, L), 'out_z' (R, L) or None, 'last_state' (R, N) and, when
    ``chunk`` > 0, 'h_chunks' (R, n_chunks, N) -- all float64 numpy arrays.
    """
    def npf(x):
        if x is None:
            return None
        if hasattr(x, "detach"):
            x = x.detach().cpu().float().numpy()
        return np.asarray(x, dtype=np.float64)

    batch, dim, L = u.shape
    N = A.shape[1]
    if rows is None:
        rows = [(b, d) for b in range(batch) for d in range(dim)]
    bi = np.array([r[0] for r in rows], dtype=np.int64)
    di = np.array([r[1] for r in rows], dtype=np.int64)
    R = len(rows)

    def take(x, idx):  # gather rows before converting, so full-size tensors are never copied
        if x is None:
            return None
        if hasattr(x, "detach"):
            return npf(x[tuple(torch_index(i) for i in idx)])
        return npf(np.asarray(x)[idx])

    def gather_bc(X):
        nd = X.dim() if hasattr(X, "dim") else np.ndim(X)
        if nd == 2:  # constant (dim, N): broadcast over l with l_stride 0
            return np.ascontiguousarray(take(X, (di,))), N, 1, 0
        if nd == 3:  # (batch, N, L): one group
            rowsX = take(X, (bi,))
        else:        # (batch, G, N, L): channel d reads group d // (dim / G)
            rowsX = take(X, (bi, di // (dim // X.shape[1])))
        return np.ascontiguousarray(rowsX), N * L, L, 1

    ur = np.ascontiguousarray(take(u, (bi, di)))
    dr = np.ascontiguousarray(take(delta, (bi, di)))
    zr = np.ascontiguousarray(take(z, (bi, di))) if z is not None else None
    Ar = np.ascontiguousarray(take(A, (di,)))
    Dr = np.ascontiguousarray(take(D, (di,))) if D is not None else None
    br = np.ascontiguousarray(take(delta_bias, (di,))) if delta_bias is not None else None
    Bs, bR, bN, bL = gather_bc(B)
    Cs, cR, cN, cL = gather_bc(C)
    out = np.zeros((R, L))
    outz = np.zeros((R, L)) if zr is not None else None
    last = np.zeros((R, N))
    n_chunks = (L + chunk - 1) // chunk if chunk > 0 else 0
    hch = np.zeros((R, n_chunks, N)) if chunk > 0 else None
    if P is not None:
        K = P.shape[-1]
        if P.dim() == 2:
            Ps, pR = np.ascontiguousarray(npf(P)), 0
            Qs, qR = np.ascontiguousarray(npf(Q)), 0
        else:
            Ps, pR = np.ascontiguousarray(take(P, (di,))), N * K
            Qs, qR = np.ascontiguousarray(take(Q, (di,))), K * N
        _load().mm_oracle_scan_pq_rows_f64(R, L, N, K, _p(ur), _p(dr), _p(zr), _p(Ar),
                                           _p(Bs), bR, bN, bL, _p(Cs), cR, cN, cL,
                                           _p(Ps), pR, _p(Qs), qR,
                                           _p(Dr), _p(br), int(bool(delta_softplus)),
                                           _p(out), _p(outz), _p(last), int(chunk), _p(hch))
        return {"out": out, "out_z": outz, "last_state": last, "h_chunks": hch}
    _load().mm_oracle_scan_rows_f64(R, L, N, _p(ur), _p(dr), _p(zr), _p(Ar),
                                    _p(Bs), bR, bN, bL, _p(Cs), cR, cN, cL,
                                    _p(Dr), _p(br), int(bool(delta_softplus)),
                                    _p(out), _p(outz), _p(last), int(chunk), _p(hch))
    return {"out": out, "out_z": outz, "last_state": last, "h_chunks": hch}


def scan_all_rows(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False, batches=None,
                  P=None, Q=None):
    """Float64 scan of every (batch, dim) row of a variable-B/C selective scan, for full-size
    checks: the rows of one (batch, group) share their B/C slice, so each (batch, group) is one
    call with a B/C row stride of 0 (no per-row copies of B/C). B/C are (batch, N, L) or
    (batch, G, N, L). With P and Q (shared (N, R) / (R, N) or per channel (dim, N, R) / (dim, R, N))
    the low-rank coupled scan is evaluated. Returns float64 numpy arrays out_z (or out, without z)
    of shape (len(batches), dim, L) and last_state (len(batches), dim, N) for ``batches`` (all by
    default).
    """
    batch, dim, L = u.shape
    N = A.shape[1]
    G = B.shape[1] if B.dim() == 4 else 1
    gsz = dim // G
    batches = list(range(batch)) if batches is None else list(batches)
    ys = np.zeros((len(batches), dim, L))
    last = np.zeros((len(batches), dim, N))

    def f64(x):
        return np.ascontiguousarray(x.detach().cpu().double().numpy())

    Ad = f64(A)
    Dd = f64(D) if D is not None else None
    bd = f64(delta_bias) if delta_bias is not None else None
    for i, b in enumerate(batches):
        for g in range(G):
            sl = slice(g * gsz, (g + 1) * gsz)
            ur, dr = f64(u[b, sl]), f64(delta[b, sl])
            zr = f64(z[b, sl]) if z is not None else None
            Bg = f64(B[b, g] if B.dim() == 4 else B[b])
            Cg = f64(C[b, g] if C.dim() == 4 else C[b])
            out = np.zeros((gsz, L))
            outz = np.zeros((gsz, L)) if zr is not None else None
            lst = np.zeros((gsz, N))
            Dg = np.ascontiguousarray(Dd[sl]) if Dd is not None else None
            bg = np.ascontiguousarray(bd[sl]) if bd is not None else None
            if P is not None:
                K = P.shape[-1]
                if P.dim() == 2:
                    Ps, pR, Qs, qR = f64(P), 0, f64(Q), 0
                else:
                    Ps, pR, Qs, qR = f64(P[sl]), N * K, f64(Q[sl]), K * N
                _load().mm_oracle_scan_pq_rows_f64(gsz, L, N, K, _p(ur), _p(dr), _p(zr),
                                                   _p(np.ascontiguousarray(Ad[sl])), _p(Bg), 0, L, 1,
                                                   _p(Cg), 0, L, 1, _p(Ps), pR, _p(Qs), qR, _p(Dg), _p(bg),
                                                   int(bool(delta_softplus)), _p(out), _p(outz), _p(lst), 0, None)
            else:
                _load().mm_oracle_scan_rows_f64(gsz, L, N, _p(ur), _p(dr), _p(zr), _p(np.ascontiguousarray(Ad[sl])),
                                                _p(Bg), 0, L, 1, _p(Cg), 0, L, 1, _p(Dg), _p(bg),
                                                int(bool(delta_softplus)), _p(out), _p(outz), _p(lst), 0, None)
            ys[i, sl] = outz if outz is not None else out
            last[i, sl] = lst
    return ys, last


def scan_bwd_all_rows(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False):
    """Float64 gradients of a variable-B/C selective scan (``mm_oracle_scan_bwd_rows_f64``, the
    adjoint recurrences of brute.scan_bwd_brute), one call per (batch, group) whose rows share the
    group's B/C slice. B/C are (batch, N, L) or (batch, G, N, L); dB/dC come back in B's/C's shape.
    Returns a dict of float64 numpy arrays du, ddelta, dz (None without z), dA, dB, dC, dD,
    ddelta_bias (None when D / delta_bias are None)."""
    batch, dim, L = u.shape
    N = A.shape[1]
    G = B.shape[1] if B.dim() == 4 else 1
    gsz = dim // G
    if N > 256:
        raise ValueError("dstate <= 256")

    def f64(x):
        return np.ascontiguousarray(x.detach().cpu().double().numpy())

    Ad = f64(A)
    Dd = f64(D) if D is not None else None
    bd = f64(delta_bias) if delta_bias is not None else None
    res = {"du": np.zeros((batch, dim, L)), "ddelta": np.zeros((batch, dim, L)),
           "dz": np.zeros((batch, dim, L)) if z is not None else None, "dA": np.zeros((dim, N)),
           "dB": np.zeros(tuple(B.shape)), "dC": np.zeros(tuple(C.shape)),
           "dD": np.zeros(dim) if D is not None else None,
           "ddelta_bias": np.zeros(dim) if delta_bias is not None else None}
    for b in range(batch):
        for g in range(G):
            sl = slice(g * gsz, (g + 1) * gsz)
            ur, dr, gr = f64(u[b, sl]), f64(delta[b, sl]), f64(dout[b, sl])
            zr = f64(z[b, sl]) if z is not None else None
            Bg = f64(B[b, g] if B.dim() == 4 else B[b])
            Cg = f64(C[b, g] if C.dim() == 4 else C[b])
            du, dd = np.zeros((gsz, L)), np.zeros((gsz, L))
            dz = np.zeros((gsz, L)) if zr is not None else None
            dA, dD, db = np.zeros((gsz, N)), np.zeros(gsz), np.zeros(gsz)
            dB, dC = np.zeros((N, L)), np.zeros((N, L))
            _load().mm_oracle_scan_bwd_rows_f64(
                gsz, L, N, _p(ur), _p(dr), _p(zr), _p(np.ascontiguousarray(Ad[sl])), _p(Bg), L, 1, _p(Cg), L, 1,
                _p(np.ascontiguousarray(Dd[sl]) if Dd is not None else None),
                _p(np.ascontiguousarray(bd[sl]) if bd is not None else None), int(bool(delta_softplus)), _p(gr),
                _p(du), _p(dd), _p(dz), _p(dA), _p(dD), _p(db), _p(dB), _p(dC))
            res["du"][b, sl], res["ddelta"][b, sl] = du, dd
            if dz is not None:
                res["dz"][b, sl] = dz
            res["dA"][sl] += dA
            if res["dD"] is not None:
                res["dD"][sl] += dD
            if res["ddelta_bias"] is not None:
                res["ddelta_bias"][sl] += db
            if B.dim() == 4:
                res["dB"][b, g] += dB
            else:
                res["dB"][b] += dB
            if C.dim() == 4:
                res["dC"][b, g] += dC
            else:
                res["dC"][b] += dC
    return res
