"""CPU restatement of the S6 scan inside the reference's SSMMixer -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker for ``s6scan.ssm_mixer``.

``ssm_mixer_scan_ref`` restates steps 4-6 of ``SSMMixer.forward``
(/root/reference/src/heuristic_secrets/models/backbone.py:1207-1242) op for op, in the
mixer's channel-last ``[B, L, *]`` layout:

* ``dt = F.softplus(dt_proj(dt))``                                              (1208-1209)
* ``A = -exp(A_log)``                                                           (1212)
* ``dA = exp(A[None, None] * dt[..., None])``  ``[B, L, I, N]``                 (1217-1219)
* ``dB_x = dt[..., None] * B[:, :, None, :] * x_conv[..., None]``               (1220-1225)
* ``state = dA[:, i] * state + dB_x[:, i]``; ``y[:, i] = einsum('bis,bs->bi')`` (1227-1238)
* ``y = y + x_conv * D``; ``y = y * silu(z)``                                   (1241-1242)

One deliberate departure from the reference's text: backbone.py:1220-1222 forms
``dB = dt[:, :, :, None] * B_param[:, None, :, :]``, i.e. ``[B, L, I, 1] * [B, 1, L, N]``.
That broadcast fails unless ``I == L``, and when ``I == L`` it pairs channel i with the B row
of *time step* i, which is not the S6 recurrence the mixer documents (dB = dt * B,
``[B, L, I, N]``, backbone.py:1214-1216) nor what ``selective_scan_ref`` computes
(selective_scan_interface.py:130-134).  This restatement uses ``B_param[:, :, None, :]``
(``[B, L, 1, N]``), the broadcast that yields the documented ``[B, L, I, N]`` shape; with
it the two restatements agree (``tests/test_oracle.py``).

The reference keeps the state in ``x.dtype``; ``state_dtype`` selects it (None = the input
dtype, as the reference; torch.float32 = the fp32 state the HIP kernel keeps).  Pinned by
``tests/test_oracle.py`` against ``selective_scan_ref`` (itself pinned by the float64 brute
force): the two restatements describe the same recurrence in two layouts.
"""
import torch
import torch.nn.functional as F


def ssm_mixer_scan_ref(x_conv, dt_lin, A_log, B_param, C_param, D, z, state_dtype=None):
    """x_conv, dt_lin, z: [B, L, I] (dt_lin = dt_proj output before softplus);
    A_log: [I, N]; B_param, C_param: [B, L, N]; D: [I].  Returns [B, L, I]."""
    dtype = x_conv.dtype if state_dtype is None else state_dtype
    x_conv, dt_lin, z = x_conv.to(dtype), dt_lin.to(dtype), z.to(dtype)
    B_param, C_param = B_param.to(dtype), C_param.to(dtype)
    dt = F.softplus(dt_lin)
    A = -torch.exp(A_log.to(dtype))
    dA = torch.exp(A[None, None, :, :] * dt[:, :, :, None])
    dB = dt[:, :, :, None] * B_param[:, :, None, :]
    dB_x = dB * x_conv[:, :, :, None]
    Bsz, L, I = x_conv.shape
    state = torch.zeros(Bsz, I, A.shape[1], dtype=dtype)
    y = torch.empty(Bsz, L, I, dtype=dtype)
    for i in range(L):
        state = dA[:, i] * state + dB_x[:, i]
        y[:, i] = torch.einsum("bis,bs->bi", state, C_param[:, i])
    y = y + x_conv * D.to(dtype)[None, None, :]
    return y * F.silu(z)
