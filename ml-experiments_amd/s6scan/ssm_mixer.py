"""SSMMixer integration: the reference mixer's S6 core on the HIP scan.

The reference's ``SSMMixer`` (/root/reference/src/heuristic_secrets/models/backbone.py:
1100-1246) computes its scan with an inline per-step Python loop over ``[B, L, I, N]``
tensors (steps 4-6 of its forward, 1207-1242).  ``ssm_mixer_scan`` replaces those steps with
one ``selective_scan_fn`` call on channel-last views:

* ``dt = softplus(dt_proj(dt))`` becomes ``delta_softplus=True`` on the raw ``dt_proj``
  output, so the softplus runs inside the scan kernel;
* ``+ x_conv * D`` and ``* silu(z)`` are the kernel's fused D skip and z gate;
* x_conv, dt, z ``[B, L, I]`` and B, C ``[B, L, N]`` (slices of the ``x_proj`` output) are
  passed as ``.mT`` views: nothing is copied, and the result comes back as a ``[B, L, I]``
  view of a channel-last buffer.

The state is fp32 (the reference's loop keeps it in ``x.dtype``).

``mixer_forward`` runs a whole mixer forward with the module's own projections, conv,
norm and SE block, and ``patch_ssm_mixer`` installs it on a mixer instance; both address
the submodules by the reference's attribute names, so any module shaped like the
reference's ``SSMMixer`` works.
"""
import types

import torch

from .selective_scan_interface import selective_scan_fn


def ssm_mixer_scan(x_conv, dt_lin, A_log, B_param, C_param, D, z):
    """Steps 4-6 of SSMMixer.forward (backbone.py:1207-1242) on the HIP scan.

    x_conv, dt_lin, z: [B, L, I] with dt_lin the ``dt_proj`` output before softplus;
    A_log: [I, N]; B_param, C_param: [B, L, N]; D: [I].  Returns ``(y + x_conv * D) *
    silu(z)`` as [B, L, I] in x_conv's dtype.  Differentiable in every tensor argument."""
    A = -torch.exp(A_log.float())
    if dt_lin.dtype != x_conv.dtype:
        dt_lin = dt_lin.to(x_conv.dtype)
    if z.dtype != x_conv.dtype:
        z = z.to(x_conv.dtype)
    out = selective_scan_fn(x_conv.mT, dt_lin.mT, A, B_param.mT, C_param.mT, D=D.float(),
                            z=z.mT, delta_softplus=True)
    return out.mT


def mixer_forward(m, x, mask=None, scan=ssm_mixer_scan):
    """Forward of a reference-shaped SSMMixer ``m`` (backbone.py:1173-1246) with ``scan``
    for its S6 core.  x: [B, L, width]; mask: [B, L] (True = masked) or None."""
    xz = m.in_proj(x)
    x_branch, z = xz.chunk(2, dim=-1)
    if mask is not None:
        x_branch = x_branch.masked_fill(mask.unsqueeze(-1), 0.0)
    x_conv = m.conv(x_branch)
    x_conv = m.conv_norm(x_conv)
    x_conv = m.se(x_conv, mask)
    x_conv = m.conv_act(x_conv)
    if mask is not None:
        x_conv = x_conv.masked_fill(mask.unsqueeze(-1), 0.0)
    ssm_params = m.x_proj(x_conv)
    dt, B_param, C_param = ssm_params.split([m.dt_rank, m.state_size, m.state_size], dim=-1)
    dt_lin = m.dt_proj(dt)
    y = scan(x_conv, dt_lin, m.A_log, B_param, C_param, m.D, z)
    return m.dropout(m.out_proj(y))


def patch_ssm_mixer(m):
    """Make ``m.forward`` run ``mixer_forward`` (the HIP scan); returns ``m``."""
    m.forward = types.MethodType(lambda self, x, mask=None: mixer_forward(self, x, mask), m)
    return m
