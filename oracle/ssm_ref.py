"""Torch (CPU) restatement of the reference selective-scan algorithms -- TEST INFRASTRUCTURE ONLY.

``selective_scan_ref`` follows ``selective_scan_ref`` of the reference,
``mamba_ssm/ops/selective_scan_interface.py:353-451``, for real A without P/Q/gamma, keeping its
op sequence so that the rounding behaviour is that of the reference on the same torch build:

* u and delta upcast to float32, ``delta += delta_bias[..., None]``, ``F.softplus`` (threshold 20)
  (ssi.py:367-374);
* ``deltaA = exp(einsum('bdl,dn->bdln'))`` and the three-operand ``deltaB_u`` einsum; 4-D B/C
  are repeated ``B G N L -> B (G H) N L`` so channel d reads group ``d // (D/G)``
  (ssi.py:388-400);
* a per-timestep loop ``x = deltaA[..., t] * x + deltaB_u[..., t]`` and ``y = einsum(x, C_t)``
  (ssi.py:422-445);
* ``out = y + u * D``; ``out *= F.silu(z)`` with z in its *original* dtype; cast to the input
  dtype; ``last_state`` is the float32 state after the last step (ssi.py:441-451).

``selective_state_update_ref`` restates the single-token decode update. The reference calls the
un-vendored upstream ``selective_state_update`` (mamba_simplemotif.py:397-399) whose in-tree
restatement is the torch fallback ``mamba_simplemotif.py:369-376``. The fallback runs the
discretisation in the activation dtype; the upstream kernel and this restatement run it in
float32 (dt + dt_bias promotes to float32), which is the behaviour the kernel must match. A state
of a 16-bit dtype (the module allocates it in dt_proj.weight.dtype, mamba_simplemotif.py:410-414)
is widened, updated in float32 and rounded back to its dtype; the output reads the float32 state.

``selective_scan_pq_ref`` restates the MotifMamba low-rank coupled scan
``selective_scan_full_matrix_cuda`` (ssi.py:262-350): h_t = exp(delta' A) h_{t-1} + delta' P (Q h_{t-1})
+ delta' u B_t, the path ``selective_scan_fn`` takes for P/Q (ssi.py:243-258). Pinned against the
transition-matrix brute force of ``brute.scan_pq_brute``, the C float64 restatement
``mm_oracle_scan_pq_rows_f64``, its P = 0 reduction to ``selective_scan_ref``, a scalar closed form
and the P -> P M, Q -> M^-1 Q invariance (tests/test_oracle_pq.py).

Pins (see tests/test_oracle.py): float64 brute-force sum on tiny shapes, a hand-worked
known-answer case, closed forms (L=1, delta=0, memoryless decay, N=1 geometric filter against
numpy.convolve, z-gate composition), invariants (linearity in u, group split, decode/scan
consistency) and the C float64 restatement ``scan_f64.c``.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from einops import rearrange, repeat


def _softplus_f32(x: torch.Tensor) -> torch.Tensor:
    return F.softplus(x)


def selective_scan_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                       return_last_state=False, compute_dtype=torch.float32):
    """CPU restatement of ssi.py:353-451 (real A, no P/Q). Shapes as in the reference:
    u, delta, z: (batch, dim, L); A: (dim, N); B, C: (dim, N) | (batch, N, L) | (batch, G, N, L).
    The reference upcasts to float32 (``.float()``); ``compute_dtype=torch.float64`` evaluates the
    same op sequence in float64 (used for exact gradients in precision checks).
    """
    if A.is_complex():
        raise NotImplementedError("complex A is out of scope")
    in_dtype = u.dtype
    u32 = u.to(compute_dtype)
    dt = delta.to(compute_dtype)
    if delta_bias is not None:
        dt = dt + delta_bias[..., None].to(compute_dtype)
    if delta_softplus:
        dt = _softplus_f32(dt)
    A = A.to(compute_dtype)
    nbatch, ndim, nstate = u.shape[0], A.shape[0], A.shape[1]
    var_B = B.dim() >= 3
    var_C = C.dim() >= 3
    Bf = B.to(compute_dtype)
    Cf = C.to(compute_dtype)
    decay = torch.exp(torch.einsum("bdl,dn->bdln", dt, A))
    if not var_B:
        drive = torch.einsum("bdl,dn,bdl->bdln", dt, Bf, u32)
    elif Bf.dim() == 3:
        drive = torch.einsum("bdl,bnl,bdl->bdln", dt, Bf, u32)
    else:
        Bf = repeat(Bf, "B G N L -> B (G H) N L", H=ndim // Bf.shape[1])
        drive = torch.einsum("bdl,bdnl,bdl->bdln", dt, Bf, u32)
    if var_C and Cf.dim() == 4:
        Cf = repeat(Cf, "B G N L -> B (G H) N L", H=ndim // Cf.shape[1])
    state = A.new_zeros((nbatch, ndim, nstate))
    ys = []
    for t in range(u.shape[2]):
        state = decay[:, :, t] * state + drive[:, :, t]
        if not var_C:
            ys.append(torch.einsum("bdn,dn->bd", state, Cf))
        elif Cf.dim() == 3:
            ys.append(torch.einsum("bdn,bn->bd", state, Cf[:, :, t]))
        else:
            ys.append(torch.einsum("bdn,bdn->bd", state, Cf[:, :, :, t]))
    y = torch.stack(ys, dim=2)
    out = y if D is None else y + u32 * rearrange(D.to(compute_dtype), "d -> d 1")
    if z is not None:
        out = out * F.silu(z)
    out = out.to(dtype=in_dtype)
    return out if not return_last_state else (out, state)


def selective_scan_ref_chunked(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                               delta_softplus=False, return_last_state=False, chunk=512):
    """Same arithmetic as ``selective_scan_ref`` but materialising the (B, D, chunk, N)
    intermediates one sequence chunk at a time, carrying the state between chunks. Used only
    as the CPU baseline when the full (B, D, L, N) intermediates do not fit the host's RAM;
    every per-element operation and its order are those of ``selective_scan_ref``."""
    in_dtype = u.dtype
    L = u.shape[2]
    nbatch, ndim, nstate = u.shape[0], A.shape[0], A.shape[1]
    state = A.new_zeros((nbatch, ndim, nstate))
    outs = []
    for s in range(0, L, chunk):
        e = min(L, s + chunk)
        sl = slice(s, e)
        u32 = u[:, :, sl].float()
        dt = delta[:, :, sl].float()
        if delta_bias is not None:
            dt = dt + delta_bias[..., None].float()
        if delta_softplus:
            dt = _softplus_f32(dt)
        Bs = B[..., sl].float() if B.dim() >= 3 else B.float()
        Cs = C[..., sl].float() if C.dim() >= 3 else C.float()
        decay = torch.exp(torch.einsum("bdl,dn->bdln", dt, A))
        if B.dim() < 3:
            drive = torch.einsum("bdl,dn,bdl->bdln", dt, Bs, u32)
        elif B.dim() == 3:
            drive = torch.einsum("bdl,bnl,bdl->bdln", dt, Bs, u32)
        else:
            Bs = repeat(Bs, "B G N L -> B (G H) N L", H=ndim // Bs.shape[1])
            drive = torch.einsum("bdl,bdnl,bdl->bdln", dt, Bs, u32)
        if C.dim() == 4:
            Cs = repeat(Cs, "B G N L -> B (G H) N L", H=ndim // Cs.shape[1])
        ys = []
        for t in range(e - s):
            state = decay[:, :, t] * state + drive[:, :, t]
            if C.dim() < 3:
                ys.append(torch.einsum("bdn,dn->bd", state, Cs))
            elif C.dim() == 3:
                ys.append(torch.einsum("bdn,bn->bd", state, Cs[:, :, t]))
            else:
                ys.append(torch.einsum("bdn,bdn->bd", state, Cs[:, :, :, t]))
        y = torch.stack(ys, dim=2)
        out = y if D is None else y + u32 * rearrange(D, "d -> d 1")
        if z is not None:
            out = out * F.silu(z[:, :, sl])
        outs.append(out.to(dtype=in_dtype))
    out = torch.cat(outs, dim=2)
    return out if not return_last_state else (out, state)


def chunk_states_ref(delta, A, delta_bias=None, delta_softplus=False, last_states=None,
                     chunk=2048):
    """Expected prod-a component of the reference's chunk-state tensor ``x``
    (selective_scan_fwd_kernel.cuh:476-495): for chunk c, prod over t < min(L, 2048(c+1)) of
    exp(delta'_t A[d, n]) = exp(A[d, n] * sum_t delta'_t). Returned as (B, D, n_chunks, N)
    float64 (the h component is the state at the chunk end, checked separately)."""
    dt = delta.double()
    if delta_bias is not None:
        dt = dt + delta_bias[..., None].double()
    if delta_softplus:
        dt = F.softplus(dt)
    L = dt.shape[-1]
    n_chunks = (L + chunk - 1) // chunk
    ends = [min(L, chunk * (c + 1)) for c in range(n_chunks)]
    cums = torch.stack([dt[:, :, :e].sum(-1) for e in ends], dim=2)  # (B, D, n_chunks)
    return torch.exp(cums[..., None] * A.double()[None, :, None, :])


def selective_state_update_ref(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                               dt_softplus=False):
    """One decode step, in place on ``state`` (float32, (batch, dim, dstate)).

    x, dt, z: (batch, dim); A: (dim, dstate); B, C: (batch, dstate) or (batch, G, dstate);
    D, dt_bias: (dim,). Discretisation and readout in float32 (dt + dt_bias promotes to
    float32 as in the upstream kernel); output cast to x.dtype.
    """
    batch, dim, nstate = state.shape
    dtf = dt.float()
    if dt_bias is not None:
        dtf = dtf + dt_bias.float()
    if dt_softplus:
        dtf = F.softplus(dtf)
    Bf = B.float()
    Cf = C.float()
    if Bf.dim() == 2:
        Bf = Bf[:, None, :]
    if Cf.dim() == 2:
        Cf = Cf[:, None, :]
    Bf = repeat(Bf, "b g n -> b (g h) n", h=dim // Bf.shape[1])
    Cf = repeat(Cf, "b g n -> b (g h) n", h=dim // Cf.shape[1])
    dA = torch.exp(dtf[:, :, None] * A.float()[None])
    dB = dtf[:, :, None] * Bf
    new_state = state.float() * dA + dB * x.float()[:, :, None]
    state.copy_(new_state.to(state.dtype))
    out = torch.einsum("bdn,bdn->bd", new_state, Cf)
    if D is not None:
        out = out + x.float() * D.float()
    if z is not None:
        out = out * F.silu(z.float())
    return out.to(x.dtype)


def softplus_f64(x: float) -> float:
    """float64 softplus with torch's threshold of 20 (used by the brute-force restatement)."""
    return x if x > 20.0 else math.log1p(math.exp(x))


def selective_scan_pq_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                          return_last_state=False, P=None, Q=None, gamma=None, compute_dtype=torch.float32):
    """CPU restatement of the MotifMamba low-rank coupled scan ``selective_scan_full_matrix_cuda``
    (reference ``mamba_ssm/ops/selective_scan_interface.py:262-350``), op for op:

    * argument checks and their ValueError / NotImplementedError (ssi.py:266-271, 306-318);
    * float32 upcasts, ``delta += delta_bias``, ``F.softplus`` (ssi.py:273-280);
    * 3-D B/C broadcast over channels, 4-D B/C repeated ``B G N L -> B (G H) N L``, 2-D B/C constant
      (ssi.py:287-301); 2-D P (N, R) / Q (R, N) expanded to every channel, 3-D used per channel
      (ssi.py:303-316);
    * per step: ``A_diag = exp(dt * A)``, ``input_term = (dt * u) * B_t``, ``q = einsum('drn,bdn->bdr')``,
      ``pq = einsum('dnr,bdr->bdn')``, ``x = A_diag * x + dt * pq + input_term``, ``y_t = sum(x * C_t)``
      (ssi.py:320-341);
    * ``out = y + u * D``, ``out *= silu(z.to(compute_dtype))``, cast to the input dtype; returns ``(out, x)``
      with x the float32 state after the last step (ssi.py:343-350).

    gamma is accepted and ignored, as in the reference (neither forward path reads it).
    The reference requires CUDA tensors (ssi.py:270-271); this restatement runs on CPU tensors.
    ``compute_dtype=torch.float64`` evaluates the same op sequence in float64 (exact gradients for
    precision checks); the default is the reference's float32.
    """
    if P is None or Q is None:
        raise ValueError("P and Q must both be provided for full-matrix path")
    if A.is_complex():
        raise NotImplementedError("Full-matrix P/Q path currently supports real A only")
    dtype_in = u.dtype
    u_f = u.to(compute_dtype)
    delta_f = delta.to(compute_dtype)
    A_f = A.to(compute_dtype)
    if delta_bias is not None:
        delta_f = delta_f + delta_bias[..., None].to(compute_dtype)
    if delta_softplus:
        delta_f = F.softplus(delta_f)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    var_B = B.dim() >= 3
    var_C = C.dim() >= 3
    B_f = B.to(compute_dtype)
    C_f = C.to(compute_dtype)
    if var_B:
        B_full = (B_f.unsqueeze(1).expand(-1, dim, -1, -1) if B_f.dim() == 3
                  else repeat(B_f, "B G N L -> B (G H) N L", H=dim // B_f.shape[1]))
    if var_C:
        C_full = (C_f.unsqueeze(1).expand(-1, dim, -1, -1) if C_f.dim() == 3
                  else repeat(C_f, "B G N L -> B (G H) N L", H=dim // C_f.shape[1]))
    if P.dim() == 2 and Q.dim() == 2:
        if P.shape[0] != dstate or Q.shape[1] != dstate or P.shape[1] != Q.shape[0]:
            raise ValueError("Expected P(n, r), Q(r, n) with n=dstate")
        P_d = P.to(compute_dtype).unsqueeze(0).expand(dim, -1, -1)
        Q_d = Q.to(compute_dtype).unsqueeze(0).expand(dim, -1, -1)
    elif P.dim() == 3 and Q.dim() == 3:
        if P.shape[0] != dim or Q.shape[0] != dim:
            raise ValueError("Expected P(dim, n, r), Q(dim, r, n)")
        if P.shape[1] != dstate or Q.shape[2] != dstate or P.shape[2] != Q.shape[1]:
            raise ValueError("Expected P(dim, n, r), Q(dim, r, n)")
        P_d = P.to(compute_dtype)
        Q_d = Q.to(compute_dtype)
    else:
        raise ValueError("P and Q must both be 2D or both be 3D")
    x = A_f.new_zeros((batch, dim, dstate))
    ys = []
    A_expand = A_f.unsqueeze(0)
    for t in range(seqlen):
        dt = delta_f[:, :, t]
        A_diag = torch.exp(dt.unsqueeze(-1) * A_expand)
        B_t = B_full[:, :, :, t] if var_B else B_f.unsqueeze(0).expand(batch, -1, -1)
        input_term = (dt * u_f[:, :, t]).unsqueeze(-1) * B_t
        q = torch.einsum("drn,bdn->bdr", Q_d, x)
        pq_term = torch.einsum("dnr,bdr->bdn", P_d, q)
        x = A_diag * x + dt.unsqueeze(-1) * pq_term + input_term
        if var_C:
            ys.append((x * C_full[:, :, :, t]).sum(dim=-1))
        else:
            ys.append((x * C_f.unsqueeze(0)).sum(dim=-1))
    y = torch.stack(ys, dim=2)
    out = y if D is None else y + u_f * D.to(compute_dtype).view(1, -1, 1)
    if z is not None:
        out = out * F.silu(z.to(compute_dtype))
    out = out.to(dtype=dtype_in)
    return out if not return_last_state else (out, x)


def selective_scan_bwd_ref(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
                           dtype=None):
    """Gradients of ``selective_scan_ref`` (the restatement of ssi.py:353-451) with respect to every
    input, by torch autograd -- the function the reference's ``selective_scan_cuda.bwd``
    (csrc/selective_scan/selective_scan.cpp:415-612, kernel selective_scan_bwd_kernel.cuh:405-880)
    computes, returned in its output order and shapes: du, ddelta (input dtype), dA, dB, dC
    (float32, cast to B's / C's dtype as selective_scan.cpp:609 does), dD, ddelta_bias (float32 or
    None) and dz (input dtype or None). ``dout`` is the gradient of the returned output (out_z when
    z is given, else out).

    ``dtype`` (default: float32) is the precision of the differentiated computation; float64
    gives the exact gradient of the same function for precision checks."""
    wt = torch.float32 if dtype is None else dtype
    leaves = {}

    def leaf(name, t, cast=True):
        if t is None:
            return None
        v = t.detach().to(wt) if cast else t.detach().clone()
        v.requires_grad_(True)
        leaves[name] = v
        return v

    # float32: the leaves keep the caller's dtypes (the forward upcasts as the reference does);
    # float64: every leaf is float64 and so is the computation.
    cast = dtype is not None
    uu = leaf("u", u, cast)
    dd = leaf("delta", delta, cast)
    AA = leaf("A", A, cast)
    BB = leaf("B", B, cast)
    CC = leaf("C", C, cast)
    DD = leaf("D", D, cast)
    zz = leaf("z", z, cast)
    bb = leaf("delta_bias", delta_bias, cast)
    out = selective_scan_ref(uu, dd, AA, BB, CC, DD, zz, bb, delta_softplus, compute_dtype=wt)
    out.backward(dout.to(out.dtype))
    g = {k: v.grad for k, v in leaves.items()}
    res = {
        "du": g["u"].to(u.dtype) if dtype is None else g["u"],
        "ddelta": g["delta"].to(delta.dtype) if dtype is None else g["delta"],
        "dA": g["A"],
        "dB": g["B"].to(B.dtype) if dtype is None else g["B"],
        "dC": g["C"].to(C.dtype) if dtype is None else g["C"],
        "dD": g.get("D"),
        "ddelta_bias": g.get("delta_bias"),
        "dz": (g["z"].to(z.dtype) if dtype is None else g["z"]) if z is not None else None,
    }
    return res


def selective_scan_pq_bwd_ref(u, delta, A, B, C, P, Q, dout, D=None, z=None, delta_bias=None,
                              delta_softplus=False, dtype=torch.float64):
    """Gradients of the low-rank coupled scan ``selective_scan_pq_ref`` (the restatement of
    ssi.py:262-350) with respect to every input, P and Q included, by torch autograd. This is what
    the reference returns in its default gradient mode (``MOTIFMAMBA_PQ_GRAD_MODE`` "exact",
    ssi.py:152-205): dP and dQ by autograd through ``selective_scan_full_matrix_cuda``, the other
    gradients from its dense CUDA backward (selective_scan_bwd_kernel.cuh:166-345, the adjoint of
    the same recurrence) for z-less calls, or from the same autograd for calls with z.

    ``dtype`` (default float64: the exact gradient) is the precision of the differentiated
    computation. Returns a dict with du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, dP, dQ (None for
    absent inputs), all in ``dtype``."""
    leaves = {}

    def leaf(name, t):
        if t is None:
            return None
        v = t.detach().to(dtype)
        v.requires_grad_(True)
        leaves[name] = v
        return v

    args = {n: leaf(n, t) for n, t in (("u", u), ("delta", delta), ("A", A), ("B", B), ("C", C), ("D", D),
                                       ("z", z), ("delta_bias", delta_bias), ("P", P), ("Q", Q))}
    out = selective_scan_pq_ref(**args, delta_softplus=delta_softplus, compute_dtype=dtype)
    out.backward(dout.to(out.dtype))
    return {"d" + n: (leaves[n].grad if n in leaves else None)
            for n in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias", "P", "Q")}
