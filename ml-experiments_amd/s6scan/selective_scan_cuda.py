"""The reference's native-module contract on the gfx950 kernels: ``fwd`` / ``bwd`` with the
argument lists and return lists of the un-vendored ``selective_scan_cuda`` pybind module, as
the reference calls it (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/
selective_scan_interface.py:42, 67-70 in SelectiveScanFn; :225-227, 263-267 in MambaInnerFn).
A maintainer who keeps the reference's own Python autograd code swaps only the import:

    from s6scan import selective_scan_cuda      # was: import selective_scan_cuda

* ``fwd(u, delta, A, B, C, D, z, delta_bias, delta_softplus) -> [out, x]`` or
  ``[out, x, out_z]`` with z.  B and C are the 4-D [batch, ngroups, dstate, seqlen] the
  reference passes (:36-41, 205-217).
* ``x`` is the saved state the backward takes back.  Its shape is
  [batch, dim, nck, 2 * dstate] fp32, nck = ceil(seqlen / 8), a permuted view of
  [batch, nck, dim, 2 * dstate] storage.  ``x[:, :, k, :dstate]`` is the state after the
  k-th 8-step segment, contiguous as the kernels store and load it.  The final state is
  also copied to the odd slots of the last segment, ``x[:, :, -1, 1::2]``, which is where
  the reference reads it (:45); that overwrites part of the last segment's first half,
  which the backward never reads (it starts each segment from the state before it).
* ``bwd(u, delta, A, B, C, D, z, delta_bias, dout, x, out, dz, delta_softplus,
  recompute_out_z) -> [du, ddelta, dA, dB, dC, dD, ddelta_bias]``, plus ``dz`` with z and then
  ``out_z`` with recompute_out_z.  A preallocated ``dz`` is written in place, as the
  reference's kernel does (:263-267).  dB / dC are 4-D fp32.
"""
import math

import torch

from .selective_scan_interface import selective_scan_backward, selective_scan_forward

_SEG = 8  # steps between saved states (S6_CKPT_INTERVAL)


def _x_view(x):
    """The kernels' [batch, nck, dim, dstate] view of the first half of x's last axis."""
    return x[..., :x.shape[-1] // 2].permute(0, 2, 1, 3)


def fwd(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    batch, dim, seqlen = u.shape
    dstate = A.shape[-1]
    nck = math.ceil(seqlen / _SEG)
    x = torch.empty(batch, nck, dim, 2 * dstate, dtype=torch.float32,
                    device=u.device).permute(0, 2, 1, 3)
    out, out_z, _, _ = selective_scan_forward(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                                              delta_softplus=delta_softplus,
                                              x_ckpt_out=_x_view(x))
    x[:, :, -1, 1::2] = x[:, :, -1, :dstate].clone()
    return [out, x] if z is None else [out, x, out_z]


def bwd(u, delta, A, B, C, D, z, delta_bias, dout, x, out, dz, delta_softplus, recompute_out_z):
    res = selective_scan_backward(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout,
                                  _x_view(x), out=out, dz_out=dz,
                                  recompute_out_z=bool(recompute_out_z) and z is not None)
    du, ddelta, dA, dB, dC, dD, dzr, ddelta_bias = res[:8]
    ret = [du, ddelta, dA, dB, dC, dD, ddelta_bias]
    if z is not None:
        ret.append(dzr)
        if recompute_out_z:
            ret.append(res[8])
    return ret
