"""Fused Mamba block (``MambaInnerFn`` / ``mamba_inner_fn``) on the gfx950 kernels.

Same signature, argument meaning and gradients as the reference's ``MambaInnerFn``
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:160-308):

    mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                   out_proj_weight, out_proj_bias, A, B=None, C=None, D=None,
                   delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                   delta_softplus=True) -> [batch, seqlen, d_model]

Forward: causal conv1d + SiLU on the x half of ``xz`` (HIP), ``x_dbl = x_proj(conv)``,
``delta = dt_proj.weight @ x_dbl[:, :dt_rank]`` and B / C slices of ``x_dbl`` (hipBLASLt
GEMMs through torch), the selective scan with the z gate, delta bias and softplus fused
(HIP), ``out_proj``.  Backward (``checkpoint_lvl`` 1 recomputes the conv output and delta,
as the reference): ``out_proj`` GEMMs, the scan backward writing dz straight into ``dxz``
and recomputing ``out_z`` (HIP), the projection GEMMs, and the conv backward writing dx
into ``dxz`` (HIP).

Layout.  Every activation is kept channel-last (``[batch, seqlen, channels]`` storage seen
as ``[batch, channels, seqlen]`` views): the kernels want channels contiguous and the GEMMs
then read and write their operands in place, so none of the reference's ``rearrange``
calls costs a copy.  ``xz`` may come in either layout; an ``xz`` whose channel stride is
not 1 (the reference's ``in_proj.weight @ hidden.T`` layout) is copied to channel-last once
and ``dxz`` is returned channel-last.

``mamba_forward(m, hidden_states)`` runs the fast path of the reference's zoology ``Mamba``
(mamba.py:120-153) for a module with its attribute names, with ``xz = in_proj(hidden)``
produced channel-last directly.
"""
import torch
import torch.nn.functional as F

from .causal_conv1d import causal_conv1d_bwd, causal_conv1d_fwd
from .selective_scan_interface import selective_scan_backward, selective_scan_forward


# Measurement hook: a pair of already-recorded torch.cuda.Events, re-recorded by the library
# around the backward scan kernel of every MambaInnerFn.backward while it is set (None: off).
KERNEL_EVENTS = None


def _channel_last(t):
    """[batch, C, L] -> the same values with stride(1) == 1 (no copy when already so)."""
    return t if t.stride(1) == 1 else t.mT.contiguous().mT


def _as_bcl(flat, batch, seqlen):
    """[(batch seqlen), C] -> [batch, C, seqlen] view."""
    return flat.view(batch, seqlen, flat.shape[-1]).mT


def _wgrad(a, b):
    """``a.t() @ b`` for token-major ``a`` [T, M] and ``b`` [T, N]: the weight gradients of
    the block's projections, T = batch * seqlen.  As one GEMM the output is small and T long,
    so the product runs on few workgroups.  T is split into S slices, one batched product with
    fp32 partials, summed in a fixed order and rounded once to the product's dtype (autocast's
    when it is on, as the reference's ``@`` under autocast) -- the rounding point of the
    single product."""
    dev = a.device.type
    dt = (torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev)
          else torch.promote_types(a.dtype, b.dtype))
    T, M = a.shape
    N = b.shape[1]
    tiles = -(-M // 64) * -(-N // 64)
    S = 1
    while S < 32 and S * tiles < 2048 and T % (2 * S) == 0 and T // (2 * S) >= 1024:
        S *= 2
    with torch.autocast(dev, enabled=False):
        a, b = a.to(dt), b.to(dt).contiguous()
        if S == 1:
            return a.t() @ b
        a3 = a.reshape(S, T // S, M).transpose(1, 2)
        b3 = b.view(S, T // S, N)  # the right operand stays contiguous
        part = (torch.bmm(a3, b3, out_dtype=torch.float32) if dt != torch.float32
                else torch.bmm(a3, b3))
        return part.sum(0).to(dt)


def _flat(bcl):
    """[batch, C, seqlen] channel-last view -> [(batch seqlen), C] view."""
    batch, c, seqlen = bcl.shape
    return bcl.mT.reshape(batch * seqlen, c)


class MambaInnerFn(torch.autograd.Function):

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                B_proj_bias=None, C_proj_bias=None, delta_softplus=True, checkpoint_lvl=1):
        """xz: (batch, 2 * d_inner, seqlen).  Returns (batch, seqlen, d_model)."""
        if checkpoint_lvl not in (0, 1):
            raise ValueError("checkpoint_lvl must be 0 or 1")
        if A.is_complex():
            raise NotImplementedError("mamba_inner_fn: complex A is not supported")
        batch, _, L = xz.shape
        delta_rank = delta_proj_weight.shape[1]
        d_state = A.shape[-1]
        if torch.is_autocast_enabled("cuda"):
            dt = torch.get_autocast_dtype("cuda")
            x_proj_weight = x_proj_weight.to(dtype=dt)
            delta_proj_weight = delta_proj_weight.to(dtype=dt)
            out_proj_weight = out_proj_weight.to(dtype=dt)
            out_proj_bias = out_proj_bias.to(dtype=dt) if out_proj_bias is not None else None
        xz = _channel_last(xz)
        conv1d_weight = conv1d_weight.flatten(1) if conv1d_weight.dim() == 3 else conv1d_weight
        x, z = xz.chunk(2, dim=1)
        conv1d_out = causal_conv1d_fwd(x, conv1d_weight, conv1d_bias, silu_activation=True)
        x_dbl = F.linear(_flat(conv1d_out), x_proj_weight)  # (bl, dt_rank + 2 d_state)
        delta = _as_bcl(F.linear(x_dbl[:, :delta_rank], delta_proj_weight), batch, L)
        ctx.is_variable_B = B is None
        ctx.is_variable_C = C is None
        ctx.B_proj_bias_is_None = B_proj_bias is None
        ctx.C_proj_bias_is_None = C_proj_bias is None
        if B is None:
            B = x_dbl[:, delta_rank:delta_rank + d_state]
            if B_proj_bias is not None:
                B = B + B_proj_bias.to(dtype=B.dtype)
            B = _as_bcl(B, batch, L).unsqueeze(1)  # (batch, 1, d_state, seqlen) view
        if C is None:
            C = x_dbl[:, -d_state:]
            if C_proj_bias is not None:
                C = C + C_proj_bias.to(dtype=C.dtype)
            C = _as_bcl(C, batch, L).unsqueeze(1)
        if delta.dtype != conv1d_out.dtype:
            delta = delta.to(conv1d_out.dtype)
        out, out_z, x_ckpt, _ = selective_scan_forward(
            conv1d_out, delta, A, B, C, D, z, delta_bias, delta_softplus, want_ckpt=True)
        ctx.delta_softplus = delta_softplus
        ctx.out_proj_bias_is_None = out_proj_bias is None
        ctx.checkpoint_lvl = checkpoint_lvl
        if checkpoint_lvl >= 1:  # recomputed in the backward
            conv1d_out, delta = None, None
        ctx.save_for_backward(xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight,
                              delta_proj_weight, out_proj_weight, conv1d_out, delta,
                              A, B, C, D, delta_bias, x_ckpt, out)
        return F.linear(out_z.mT, out_proj_weight, out_proj_bias)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        (xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight, delta_proj_weight,
         out_proj_weight, conv1d_out, delta, A, B, C, D, delta_bias, x_ckpt,
         out) = ctx.saved_tensors
        batch, _, L = xz.shape
        delta_rank = delta_proj_weight.shape[1]
        d_state = A.shape[-1]
        x, z = xz.chunk(2, dim=1)
        if ctx.checkpoint_lvl == 1:
            conv1d_out = causal_conv1d_fwd(x, conv1d_weight, conv1d_bias, silu_activation=True)
            delta = _as_bcl(F.linear(x_dbl[:, :delta_rank], delta_proj_weight), batch, L)
            if delta.dtype != conv1d_out.dtype:
                delta = delta.to(conv1d_out.dtype)
        dxz = torch.empty_like(xz)
        dx, dz = dxz.chunk(2, dim=1)
        dout = dout.reshape(batch * L, dout.shape[-1])
        dout_y = _as_bcl(dout @ out_proj_weight, batch, L)  # (batch, d_inner, seqlen)
        (dconv1d_out, ddelta, dA, dB, dC, dD, _, ddelta_bias, out_z) = selective_scan_backward(
            conv1d_out, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, dout_y, x_ckpt,
            out=out, dz_out=dz, recompute_out_z=True, kernel_events=KERNEL_EVENTS)
        dout_proj_weight = _wgrad(dout, _flat(out_z))
        dout_proj_bias = dout.sum(dim=0) if not ctx.out_proj_bias_is_None else None
        dD = dD if D is not None else None
        dx_dbl = torch.empty_like(x_dbl)
        dB_proj_bias = None
        if ctx.is_variable_B:
            dB = _flat(dB.squeeze(1))  # (bl, d_state)
            dB_proj_bias = dB.sum(0) if not ctx.B_proj_bias_is_None else None
            dx_dbl[:, delta_rank:delta_rank + d_state] = dB
            dB = None
        dC_proj_bias = None
        if ctx.is_variable_C:
            dC = _flat(dC.squeeze(1))
            dC_proj_bias = dC.sum(0) if not ctx.C_proj_bias_is_None else None
            dx_dbl[:, -d_state:] = dC
            dC = None
        ddelta = _flat(ddelta)  # (bl, d_inner)
        ddelta_proj_weight = _wgrad(ddelta, x_dbl[:, :delta_rank])
        dx_dbl[:, :delta_rank] = ddelta @ delta_proj_weight
        dconv = _flat(dconv1d_out)  # (bl, d_inner) view of dconv1d_out
        dx_proj_weight = _wgrad(dx_dbl, _flat(conv1d_out))
        torch.addmm(dconv, dx_dbl, x_proj_weight, out=dconv)
        _, dconv1d_weight, dconv1d_bias, _ = causal_conv1d_bwd(
            x, conv1d_weight, conv1d_bias, dconv1d_out, dx=dx, silu_activation=True)
        dconv1d_bias = dconv1d_bias if conv1d_bias is not None else None
        dconv1d_weight = dconv1d_weight.unsqueeze(1)  # "d w -> d 1 w"
        return (dxz, dconv1d_weight, dconv1d_bias, dx_proj_weight, ddelta_proj_weight,
                dout_proj_weight, dout_proj_bias, dA, dB, dC, dD,
                ddelta_bias if delta_bias is not None else None,
                dB_proj_bias, dC_proj_bias, None, None)


def mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                   out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                   B_proj_bias=None, C_proj_bias=None, delta_softplus=True):
    return MambaInnerFn.apply(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                              out_proj_weight, out_proj_bias, A, B, C, D, delta_bias,
                              B_proj_bias, C_proj_bias, delta_softplus)


class InProjFn(torch.autograd.Function):
    """``F.linear(hidden, weight, bias)`` over the tokens of a block's in_proj, with the same
    forward and gradients as autograd's, except that the weight gradient is computed split
    over tokens (``_wgrad``): one GEMM over batch * seqlen tokens into a small weight runs on
    few workgroups.  Under autocast the products run in the autocast dtype and the weight
    and bias gradients come back in the parameters' dtypes, as autograd's cast would."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, h2d, weight, bias):
        ctx.save_for_backward(h2d, weight)
        ctx.bias_dtype = None if bias is None else bias.dtype
        return F.linear(h2d, weight, bias)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        h2d, weight = ctx.saved_tensors
        dh = (dy @ weight).to(h2d.dtype) if ctx.needs_input_grad[0] else None
        dw = _wgrad(dy, h2d).to(weight.dtype)
        db = dy.sum(0).to(ctx.bias_dtype) if ctx.bias_dtype is not None else None
        return dh, dw, db


def mamba_forward(m, hidden_states):
    """Fast-path forward of a zoology-``Mamba``-shaped module ``m`` (mamba.py:120-153):
    in_proj, then ``mamba_inner_fn`` with input-dependent B / C, ``D``, the dt_proj bias as
    delta bias and softplus.  hidden_states: (batch, seqlen, d_model)."""
    batch, seqlen, d_model = hidden_states.shape
    xz = InProjFn.apply(hidden_states.reshape(batch * seqlen, d_model), m.in_proj.weight,
                        m.in_proj.bias).view(batch, seqlen, -1).mT  # channel-last
    A = -torch.exp(m.A_log.float())
    return mamba_inner_fn(xz, m.conv1d.weight, m.conv1d.bias, m.x_proj.weight,
                          m.dt_proj.weight, m.out_proj.weight, m.out_proj.bias, A, None, None,
                          m.D.float(), delta_bias=m.dt_proj.bias.float(), delta_softplus=True)
