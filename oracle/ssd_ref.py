"""CPU restatements of the Mamba-2 SSD scan -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and the other checker legs named in ``oracle/selective_scan_ref.py``)
may import this module, as the checker of ``s6scan.ssd_combined``.

``ssd_chunked_ref`` restates the reference's chunked forward
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/ssd_combined.py:281-332)
step by step, with the semantics of each Triton kernel it calls:

* dt' = clamp(softplus(dt + dt_bias)), zero past the sequence end; S = cumsum(dt' A) within
  each chunk                                                (ssd_chunk_state.py:34-84)
* chunk states st_c = sum_l x_l (dt'_l e^{S_last - S_l}) B_l^T over the positions whose
  seq_idx equals the chunk's last one                       (ssd_chunk_state.py:177-266)
* state passing H_{c+1} = e^{S_last} H_c + st_c, the carried part dropped when the chunk's
  last seq_idx differs from the previous chunk's (the previous one starts as 0)
                                                            (ssd_state_passing.py:28-91)
* CB = C B^T within each chunk, zero where seq_idx differs  (ssd_bmm.py:35-106)
* y_l = e^{S_l} C_l H_c^T [seq_idx_l == seq_idx at the step before the chunk (0 for the
  first chunk)] + sum_{s<=l} CB[l,s] e^{S_l - S_s} dt'_s x_s + D x_l; out = y silu(z)
                                                            (ssd_chunk_scan.py:43-185)

``ssd_varlen_states_ref`` restates the per-sequence final states of a packed batch-1 input
(chunk_state_varlen); tests pin it against the brute force on each sequence's prefix.

``ssd_brute64`` is an independent float64 NumPy loop over the recurrence itself (state reset
where seq_idx changes, the initial state belonging to seq_idx 0).  Tests
(``tests/test_oracle_ssd.py``) pin the chunked restatement against it, and the brute force
against the S6 brute force ``brute64.scan_fwd64`` through the head expansion the reference
itself uses to express SSD as a selective scan (ssd_combined.py:663-711).
"""
import math

import numpy as np
import torch
import torch.nn.functional as F


def _dt_process(dt, dt_bias, dt_softplus, dt_limit):
    if dt_bias is not None:
        dt = dt + dt_bias
    if dt_softplus:
        dt = F.softplus(dt)
    return dt.clamp(min=dt_limit[0], max=dt_limit[1])


def _chunked_states(x, dt, A, B, chunk_size, dt_bias, initial_states, seq_idx, dt_softplus,
                    dt_limit, cd):
    """The chunk quantities shared by the forward and the varlen states: processed dt, the
    per-chunk cumsum S, the chunk states and the states entering each chunk."""
    batch, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    Q = chunk_size
    K = math.ceil(L / Q)
    pad = K * Q - L
    f = lambda t: None if t is None else t.to(cd)
    x, dt, B = f(x), f(dt), f(B)
    dtp = _dt_process(dt, f(dt_bias), dt_softplus, dt_limit)            # (b, L, h)
    padL = lambda t: F.pad(t, (0, 0) * (t.dim() - 2) + (0, pad)) if pad else t
    dtp = padL(dtp)                                                      # zero past the end
    xc = padL(x).reshape(batch, K, Q, H, P)
    Bh = padL(B).repeat_interleave(hpg, dim=2).reshape(batch, K, Q, H, N)
    dtc = dtp.reshape(batch, K, Q, H)
    S = torch.cumsum(dtc * f(A), dim=2)                                  # (b, K, Q, h)
    if seq_idx is not None:
        seqp = F.pad(seq_idx.long(), (0, pad), value=-1).reshape(batch, K, Q)
        lims = [min(Q, L - c * Q) for c in range(K)]
        seq_last = torch.stack([seqp[:, c, lims[c] - 1] for c in range(K)], dim=1)   # (b, K)
    # chunk states
    w = dtc * torch.exp(S[:, :, -1:, :] - S)                             # (b, K, Q, h)
    if seq_idx is not None:
        w = w * (seqp == seq_last[:, :, None])[..., None].to(cd)
    st = torch.einsum("bclhp,bclh,bclhn->bchpn", xc, w, Bh)
    # state passing
    Hc = (f(initial_states) if initial_states is not None
          else torch.zeros(batch, H, P, N, dtype=cd))
    prev = torch.zeros(batch, dtype=torch.long)
    Hs = []
    for c in range(K):
        Hs.append(Hc)
        scale = torch.exp(S[:, c, -1, :])                                # (b, h)
        if seq_idx is not None:
            scale = scale * (seq_last[:, c] == prev).to(cd)[:, None]
            prev = seq_last[:, c]
        Hc = scale[:, :, None, None] * Hc + st[:, c]
    final = Hc
    Hs = torch.stack(Hs, dim=1)                                          # (b, K, h, p, n)
    return dict(x=x, dtp=dtp, xc=xc, Bh=Bh, dtc=dtc, S=S, Hs=Hs, final=final,
                seqp=seqp if seq_idx is not None else None, K=K, Q=Q, pad=pad, hpg=hpg)


def ssd_chunked_ref(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                    initial_states=None, seq_idx=None, dt_softplus=False,
                    dt_limit=(0.0, float("inf")), compute_dtype=torch.float32):
    """Returns (out, out_x, final_states); out_x is y before the z gate (None without z)."""
    cd = compute_dtype
    f = lambda t: None if t is None else t.to(cd)
    q = _chunked_states(x, dt, A, B, chunk_size, dt_bias, initial_states, seq_idx, dt_softplus,
                        dt_limit, cd)
    x, xc, Bh, dtc, S, Hs, final = q["x"], q["xc"], q["Bh"], q["dtc"], q["S"], q["Hs"], q["final"]
    K, Q, pad, hpg = q["K"], q["Q"], q["pad"], q["hpg"]
    seqp = q["seqp"]
    batch, L, H, P = x.shape
    N = B.shape[3]
    padL = lambda t: F.pad(t, (0, 0) * (t.dim() - 2) + (0, pad)) if pad else t
    Ch = padL(f(C)).repeat_interleave(hpg, dim=2).reshape(batch, K, Q, H, N)
    z = f(z)
    # C B^T within chunks, decay, causal mask
    CB = torch.einsum("bclhn,bcshn->bchls", Ch, Bh)
    if seq_idx is not None:
        CB = CB * (seqp[:, :, :, None] == seqp[:, :, None, :])[:, :, None].to(cd)
    Sl = S.permute(0, 1, 3, 2)                                           # (b, K, h, Q)
    diff = Sl[..., :, None] - Sl[..., None, :]
    causal = torch.ones(Q, Q, dtype=torch.bool).tril()
    decay = torch.exp(torch.where(causal, diff, torch.full_like(diff, -math.inf)))
    M = CB * decay * dtc.permute(0, 1, 3, 2)[:, :, :, None, :]
    y = torch.einsum("bchls,bcshp->bclhp", M, xc)
    inter = torch.einsum("bclhn,bchpn->bclhp", Ch, Hs) * torch.exp(S)[..., None]
    if seq_idx is not None:
        sprev = torch.zeros(batch, K, dtype=torch.long)  # seq_idx at the step before chunk c
        for c in range(1, K):
            sprev[:, c] = seq_idx[:, c * Q - 1].long()
        inter = inter * (seqp == sprev[:, :, None])[..., None, None].to(cd)
    y = (y + inter).reshape(batch, K * Q, H, P)[:, :L]
    if D is not None:
        Df = f(D)
        y = y + x * (Df if Df.dim() == 2 else Df[:, None])
    out_x = None
    if z is not None:
        out_x = y
        y = y * F.silu(z)
    return y, out_x, final


def ssd_varlen_states_ref(x, dt, A, B, chunk_size, cu_seqlens, dt_bias=None,
                          initial_states=None, seq_idx=None, dt_softplus=False,
                          dt_limit=(0.0, float("inf")), compute_dtype=torch.float32):
    """The state at the end of each sequence of a packed batch-1 input, as the reference's
    chunk_state_varlen computes it (ssd_chunk_state.py:589-660, called at
    ssd_combined.py:329-331): for the sequence [s0, s1) and c the chunk of step s1 - 1,
    the chunk-state sum over the rows of chunk c from max(s0, c Q) to s1 - 1 with the decay
    to step s1 - 1, plus e^{S(s1 - 1)} times the state entering chunk c when s0 < c Q.
    Returns [nseq, nheads, headdim, dstate]."""
    q = _chunked_states(x, dt, A, B, chunk_size, dt_bias, initial_states, seq_idx, dt_softplus,
                        dt_limit, compute_dtype)
    xc, Bh, dtc, S, Hs, Q = q["xc"], q["Bh"], q["dtc"], q["S"], q["Hs"], q["Q"]
    cu = [int(v) for v in cu_seqlens]
    out = []
    for s0, s1 in zip(cu[:-1], cu[1:]):
        c = (s1 - 1) // Q
        e = s1 - 1 - c * Q
        r0 = max(s0 - c * Q, 0)
        w = dtc[0, c, r0:e + 1] * torch.exp(S[0, c, e][None] - S[0, c, r0:e + 1])   # (rows, h)
        st = torch.einsum("lhp,lh,lhn->hpn", xc[0, c, r0:e + 1], w, Bh[0, c, r0:e + 1])
        if s0 < c * Q:
            st = st + torch.exp(S[0, c, e])[:, None, None] * Hs[0, c]
        out.append(st)
    return torch.stack(out)


def ssd_brute64(x, dt, A, B, C, D=None, z=None, dt_bias=None, initial_states=None,
                seq_idx=None, dt_softplus=False, dt_limit=(0.0, float("inf"))):
    """Float64 loop over the recurrence.  NumPy or torch inputs; returns (out, final)."""
    a = lambda t: None if t is None else np.asarray(t.detach().cpu() if torch.is_tensor(t) else t,
                                                   np.float64)
    x, dt, A, B, C, D, z, bias = a(x), a(dt), a(A), a(B), a(C), a(D), a(z), a(dt_bias)
    init = a(initial_states)
    batch, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    seq = None if seq_idx is None else np.asarray(seq_idx.cpu() if torch.is_tensor(seq_idx) else seq_idx)
    out = np.zeros((batch, L, H, P))
    final = np.zeros((batch, H, P, N))
    for b in range(batch):
        h = np.zeros((H, P, N)) if init is None else init[b].copy()
        if seq is not None and seq[b, 0] != 0:
            h[:] = 0.0
        for t in range(L):
            if seq is not None and t > 0 and seq[b, t] != seq[b, t - 1]:
                h[:] = 0.0
            d = dt[b, t] + (0.0 if bias is None else bias)
            if dt_softplus:
                d = np.where(d <= 20.0, np.log1p(np.exp(np.minimum(d, 20.0))), d)
            d = np.clip(d, dt_limit[0], dt_limit[1])                     # (H,)
            for hh in range(H):
                g = hh // hpg
                h[hh] = np.exp(A[hh] * d[hh]) * h[hh] + d[hh] * np.outer(x[b, t, hh], B[b, t, g])
                y = h[hh] @ C[b, t, g]
                if D is not None:
                    y = y + (D[hh] if D.ndim == 2 else D[hh]) * x[b, t, hh]
                if z is not None:
                    zz = z[b, t, hh]
                    y = y * zz / (1.0 + np.exp(-zz))
                out[b, t, hh] = y
        final[b] = h
    return out, final
