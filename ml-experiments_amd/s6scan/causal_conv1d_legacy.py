"""The older ``causal_conv1d`` native-module API, on the same gfx950 kernels as
``s6scan.causal_conv1d``.

The reference ships two copies of the Mamba interface file.  The one zoology's ``Mamba``
actually imports (/root/reference/zoology/zoology/mixers/mamba_ssm/
selective_scan_interface.py, imported at zoology/mixers/mamba.py:16) was written against the
earlier package release, whose module calls have shorter argument lists:

* ``causal_conv1d_fwd(x, weight, bias, seq_idx, silu_activation) -> out``
  (selective_scan_interface.py:181, 243);
* ``causal_conv1d_bwd(x, weight, bias, dout, seq_idx, dx, silu_activation)
  -> (dx, dweight, dbias)``, three values (selective_scan_interface.py:288-290);
* ``causal_conv1d_fn(x, weight, bias, activation)`` with the activation in the fourth
  positional slot (selective_scan_interface.py:321).

Swapping this module in for that file's ``causal_conv1d_cuda`` (and its ``causal_conv1d_fn``)
keeps the file's calls unchanged; ``s6scan.causal_conv1d`` serves the newer argument lists of
the other copy (mamba_ssm/ops/selective_scan_interface.py:187-189, 299-301).  ``seq_idx``
must be None, as every reference call passes it.
"""
from . import causal_conv1d as _conv


def causal_conv1d_fwd(x, weight, bias, seq_idx, silu_activation):
    """out = act(causal depthwise conv of x with weight, plus bias); x [batch, dim, seqlen]."""
    return _conv.causal_conv1d_fwd(x, weight, bias, seq_idx, None, None, silu_activation)


def causal_conv1d_bwd(x, weight, bias, dout, seq_idx, dx, silu_activation):
    """Gradients of causal_conv1d_fwd: ``(dx, dweight, dbias)``; ``dx`` may be a preallocated
    output of x's shape and dtype (or None); dbias is None without bias."""
    gx, gw, gb, _ = _conv.causal_conv1d_bwd(x, weight, bias, dout, seq_idx, None, None, dx,
                                            False, silu_activation)
    return gx, gw, gb


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, activation=None):
    """Differentiable conv.  Accepts the activation either by keyword or, as the earlier
    release's ``(x, weight, bias, activation)`` order has it, as the fourth positional
    argument (a string there cannot be a ``seq_idx`` tensor)."""
    if isinstance(seq_idx, str):
        if activation is not None:
            raise TypeError("causal_conv1d_fn: activation given twice")
        seq_idx, activation = None, seq_idx
    return _conv.causal_conv1d_fn(x, weight, bias, seq_idx, activation)
