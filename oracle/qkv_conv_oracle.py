"""CPU restatement of the fused Q/K/V short convolution -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product package never routes through it.

The function is the reference's ``delta_feedback::pkda_qkv_conv``
(``delta_feedback_experiment/fla_ops.py:134-170``) whose portable form is
``PreconditionedKDA._causal_conv`` followed by ``_l2norm`` on the query and key
slabs (``delta_feedback_experiment/pkda.py:197-220,290-316,37-44``): a
depthwise causal convolution of ``W`` taps with zero history, SiLU, and a
per-head L2 normalisation ``y * rsqrt(sum(y^2) + eps)`` of the channels below
``norm_channels``.  The fused CUDA path keeps the convolution, SiLU and
normalisation in FP32 and casts only the final Q/K/V
(``delta_feedback_experiment/pkda.py:231-233``); so does this restatement.

The convolution is written as explicit shifted sums
``a[t] = sum_w weight[w] x[t - (W - 1) + w]`` rather than through
``F.conv1d``, so that ``tests/test_conv_oracle.py`` can pin the tap order and
the causal offset against the reference's own ``F.conv1d`` formulation (the
history-padded grouped convolution of ``_causal_conv``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor


def causal_conv_silu(x: Tensor, weight: Tensor, dtype: torch.dtype = torch.float32,
                     history: Tensor | None = None) -> Tensor:
    """``silu(sum_w weight[c, w] x[b, t - (W - 1) + w, c])``.

    ``x`` is ``[B, T, C]``, ``weight`` ``[C, W]``; computed in ``dtype``.  The
    rows before ``t = 0`` are ``history [B, W - 1, C]`` (oldest first) or zero:
    a cached row's stored conv state prepended to its new projections
    (``delta_feedback_experiment/pkda.py:205-219,240-260``).
    """
    xf, wf = x.to(dtype), weight.to(dtype)
    B, T, C = xf.shape
    W = wf.shape[1]
    before = xf.new_zeros(B, W - 1, C) if history is None else history.to(dtype)
    padded = torch.cat((before, xf), dim=1)
    a = sum(wf[:, w] * padded[:, w:w + T] for w in range(W))
    return F.silu(a)


def history_after(x: Tensor, history: Tensor | None, conv_size: int) -> Tensor:
    """The conv state a cached row keeps: the last ``conv_size - 1`` rows of
    ``history ++ x`` (``combined[..., -history:]``, pkda.py:219 and 248-258),
    ``[B, conv_size - 1, C]`` in ``x.dtype``."""
    B, T, C = x.shape
    before = x.new_zeros(B, conv_size - 1, C) if history is None else history.to(x.dtype)
    return torch.cat((before, x), dim=1)[:, T:]


def qkv_conv_reference(x: Tensor, weight: Tensor, head_dim: int, norm_channels: int, eps: float = 1e-6,
                       dtype: torch.dtype = torch.float32, out_dtype: torch.dtype | None = None,
                       history: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``(q, k, v)`` slabs ``[B, T, C / 3]`` of the fused op (fla_ops.py:134-170).

    Differentiable (FP32 or FP64 autograd is the gradient oracle).  The outputs
    come in ``out_dtype`` (default: ``x.dtype``).  ``history`` as in
    :func:`causal_conv_silu`.
    """
    y = causal_conv_silu(x, weight, dtype, history)
    B, T, C = y.shape
    if norm_channels:
        yn = y[..., :norm_channels].reshape(B, T, norm_channels // head_dim, head_dim)
        yn = yn * torch.rsqrt(yn.square().sum(-1, keepdim=True) + eps)
        y = torch.cat((yn.reshape(B, T, norm_channels), y[..., norm_channels:]), dim=-1)
    width = C // 3
    out = out_dtype or x.dtype
    return tuple(part.to(out) for part in y.split(width, dim=-1))
