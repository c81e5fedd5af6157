"""Float64 brute force of the S6 scan and its analytic gradients -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and the other checker legs named in ``oracle/selective_scan_ref.py``)
may import this.  It restates the mathematics of the reference recurrence
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:107-156)
in float64 NumPy, written independently of torch so that a mistake in the torch
restatement (a dropped term, a transposed operand) shows up as a disagreement:

    Delta_t   = softplus(delta_t + bias)              (or delta_t + bias)
    abar_t,n  = exp(Delta_t * A_n)
    h_t,n     = abar_t,n * h_{t-1},n + Delta_t * u_t * B_t,n      (h_{-1} = 0)
    y_t       = sum_n C_t,n h_t,n + D * u_t
    out_t     = y_t * silu(z_t)                        (if z is given)

Varlen (``cu_seqlens``): h_{s-1} is taken as 0 at every sequence start s.

The backward is derived by hand (lambda_t = dL/dh_t, a reverse recurrence), not by autograd:

    dy_t      = dout_t * silu(z_t)                     (dout_t without z)
    lambda_t  = C_t dy_t + abar_{t+1} lambda_{t+1}     (flow cut at sequence starts)
    q_t       = lambda_t * abar_t * h_{t-1}            (= dL/d(Delta_t A_n))
    dA_n     += q_t Delta_t ;  dDelta_t += sum_n q_t A_n + lambda_t u_t B_t,n
    du_t      = sum_n lambda_t Delta_t B_t,n + D dy_t ; dB_t,n += lambda_t Delta_t u_t
    dC_t,n   += dy_t h_t,n ;  dD += dy_t u_t ;  dz_t = dout_t y_t silu'(z_t)
    ddelta_t  = dDelta_t * sigmoid(delta_t + bias)     (softplus, below threshold 20)

It is checked against ``torch.autograd.gradcheck`` and autograd of the torch restatement
in ``tests/test_oracle.py``.
"""
import numpy as np


def _softplus(x):
    return np.where(x <= 20.0, np.log1p(np.exp(np.minimum(x, 20.0))), x)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _bc4(M, batch, dim):
    """[B,N,L] -> [B,G=1,N,L]; then expand groups to one row per channel [B,D,N,L]."""
    M = np.asarray(M, dtype=np.float64)
    if M.ndim == 3:
        M = M[:, None]
    G = M.shape[1]
    return np.repeat(M, dim // G, axis=1), G


def _starts(L, cu_seqlens):
    s = np.zeros(L, dtype=bool)
    s[0] = True
    if cu_seqlens is not None:
        for v in np.asarray(cu_seqlens)[:-1]:
            if int(v) < L:
                s[int(v)] = True
    return s


def scan_fwd64(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
               cu_seqlens=None):
    """Returns dict(out, y, h, last_state, Delta, abar).  h is [B, D, L, N]."""
    u = np.asarray(u, np.float64)
    dr = np.asarray(delta, np.float64)
    A = np.asarray(A, np.float64)
    batch, dim, L = u.shape
    N = A.shape[1]
    Bf, _ = _bc4(B, batch, dim)
    Cf, _ = _bc4(C, batch, dim)
    pre = dr + (0.0 if delta_bias is None else np.asarray(delta_bias, np.float64)[None, :, None])
    Delta = _softplus(pre) if delta_softplus else pre
    abar = np.exp(Delta[..., None] * A[None, :, None, :])          # [B, D, L, N]
    starts = _starts(L, cu_seqlens)
    h = np.zeros((batch, dim, L, N))
    cur = np.zeros((batch, dim, N))
    for t in range(L):
        if starts[t]:
            cur = np.zeros_like(cur)
        cur = abar[:, :, t] * cur + (Delta[:, :, t] * u[:, :, t])[..., None] * Bf[:, :, :, t]
        h[:, :, t] = cur
    y = np.einsum('bdln,bdnl->bdl', h, Cf)
    if D is not None:
        y = y + u * np.asarray(D, np.float64)[None, :, None]
    out = y
    if z is not None:
        zz = np.asarray(z, np.float64)
        out = y * zz * _sigmoid(zz)
    if cu_seqlens is None:
        last = h[:, :, -1]
    else:
        cu = np.asarray(cu_seqlens)
        last = np.stack([h[0, :, int(e) - 1] if int(e) > int(s) else np.zeros((dim, N))
                         for s, e in zip(cu[:-1], cu[1:])], axis=0)
    return dict(out=out, y=y, h=h, last_state=last, Delta=Delta, abar=abar, pre=pre)


def scan_bwd64(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
               cu_seqlens=None):
    """Hand-derived gradients of sum(out * dout).  dB/dC come back in B/C's own shape."""
    f = scan_fwd64(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                   delta_softplus=delta_softplus, cu_seqlens=cu_seqlens)
    u = np.asarray(u, np.float64)
    A = np.asarray(A, np.float64)
    dout = np.asarray(dout, np.float64)
    batch, dim, L = u.shape
    N = A.shape[1]
    Bf, GB = _bc4(B, batch, dim)
    Cf, GC = _bc4(C, batch, dim)
    Delta, abar, h, pre = f['Delta'], f['abar'], f['h'], f['pre']
    starts = _starts(L, cu_seqlens)
    dz = None
    if z is not None:
        zz = np.asarray(z, np.float64)
        sg = _sigmoid(zz)
        dy = dout * zz * sg
        dz = dout * f['y'] * sg * (1.0 + zz * (1.0 - sg))
    else:
        dy = dout
    lam_next = np.zeros((batch, dim, N))     # abar_{t+1} * lambda_{t+1}
    dA = np.zeros_like(A)
    dDelta = np.zeros((batch, dim, L))
    du = np.zeros((batch, dim, L))
    dBf = np.zeros_like(Bf)
    dCf = np.zeros_like(Cf)
    for t in range(L - 1, -1, -1):
        lam = Cf[:, :, :, t] * dy[:, :, t, None] + lam_next
        hprev = h[:, :, t - 1] if (t > 0 and not starts[t]) else np.zeros((batch, dim, N))
        q = lam * abar[:, :, t] * hprev
        dA += np.einsum('bdn,bd->dn', q, Delta[:, :, t])
        dDelta[:, :, t] = (q * A[None]).sum(-1) + (lam * Bf[:, :, :, t]).sum(-1) * u[:, :, t]
        du[:, :, t] = (lam * Bf[:, :, :, t]).sum(-1) * Delta[:, :, t]
        dBf[:, :, :, t] = lam * (Delta[:, :, t] * u[:, :, t])[..., None]
        dCf[:, :, :, t] = h[:, :, t] * dy[:, :, t, None]
        lam_next = np.zeros_like(lam) if starts[t] else abar[:, :, t] * lam
    dD = None
    if D is not None:
        du = du + dy * np.asarray(D, np.float64)[None, :, None]
        dD = (dy * u).sum(axis=(0, 2))
    if delta_softplus:
        ddelta = dDelta * np.where(pre <= 20.0, _sigmoid(pre), 1.0)
    else:
        ddelta = dDelta
    ddelta_bias = ddelta.sum(axis=(0, 2)) if delta_bias is not None else None

    def fold(M, G, orig):
        s = M.reshape(batch, G, dim // G, N, L).sum(2)
        return s[:, 0] if np.asarray(orig).ndim == 3 else s
    return dict(du=du, ddelta=ddelta, dA=dA, dB=fold(dBf, GB, B), dC=fold(dCf, GC, C), dD=dD,
                dz=dz, ddelta_bias=ddelta_bias, out=f['out'])
