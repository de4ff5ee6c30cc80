"""Custom op over the gfx950 depthwise causal conv kernel: Q, K and V slabs
out of one pass, each through SiLU, Q and K unit-normalised per head.

Mirrors ``delta_feedback::pkda_qkv_conv`` and its backward op
(``delta_feedback_experiment/fla_ops.py:134-249``): same arguments
``(x, weight, head_dim, norm_channels, eps)``, same outputs (the Q, K and V
slabs ``[B, T, C / 3]`` in ``x.dtype``), gradients ``(dx, dw)`` in the dtypes
of ``x`` and ``weight``.  ``PreconditionedKDA._project`` calls it on the
concatenated projections with ``norm_channels = 2 * projection_size``
(``delta_feedback_experiment/pkda.py:223-288``).  The kernels index ``x`` by
dense strides, so the forward and the backward both take ``x.contiguous()``.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .pkda import _dtype_code, _ptr, _stream


def _args(x: Tensor, weight: Tensor, head_dim: int, norm_channels: int, eps: float) -> _lib.QkvConvArgs:
    if x.dim() != 3 or weight.dim() != 2 or x.shape[-1] != weight.shape[0] or x.shape[-1] % 3:
        raise ValueError(f"x [B, T, 3 * width] and weight [3 * width, conv_size] expected, got "
                         f"{tuple(x.shape)} and {tuple(weight.shape)}")
    if not x.is_cuda or not weight.is_cuda:
        raise RuntimeError("pkda_qkv_conv needs tensors on a HIP device; there is no CPU fallback")
    B, T, C = x.shape
    return _lib.QkvConvArgs(
        dtype=_dtype_code(x), w_dtype=_dtype_code(weight), batch=B, seqlen=T, width=C // 3,
        head_dim=int(head_dim), norm_channels=int(norm_channels), conv_size=weight.shape[1], eps=float(eps),
        x=_ptr(x), weight=_ptr(weight),
    )


@torch.library.custom_op("pkda_mi355x::pkda_qkv_conv", mutates_args=(), device_types="cuda")
def pkda_qkv_conv(x: Tensor, weight: Tensor, head_dim: int, norm_channels: int,
                  eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """One SiLU short convolution over concatenated Q/K/V with the per-head L2
    normalisation of the first ``norm_channels`` channels, written as three
    slabs (the reference's contract, fla_ops.py:134-170)."""
    x, weight = x.contiguous(), weight.contiguous()
    args = _args(x, weight, head_dim, norm_channels, eps)
    B, T, C = x.shape
    q, k, v = (torch.empty(B, T, C // 3, device=x.device, dtype=x.dtype) for _ in range(3))
    args.q, args.k, args.v = _ptr(q), _ptr(k), _ptr(v)
    with torch.cuda.device(x.device):
        _lib.call("pkda_qkv_conv_fwd", args, _stream(x.device))
    return q, k, v


@pkda_qkv_conv.register_fake
def _pkda_qkv_conv_fake(x, weight, head_dim, norm_channels, eps):
    B, T, C = x.shape
    return tuple(x.new_empty(B, T, C // 3) for _ in range(3))


@torch.library.custom_op("pkda_mi355x::pkda_qkv_conv_backward", mutates_args=(), device_types="cuda")
def pkda_qkv_conv_backward(x: Tensor, weight: Tensor, dq: Tensor, dk: Tensor, dv: Tensor, head_dim: int,
                           norm_channels: int, eps: float) -> tuple[Tensor, Tensor]:
    """``(dx, dw)`` of :func:`pkda_qkv_conv` (fla_ops.py:181-215).  ``dw`` is a
    fixed-order sum over token tiles: bitwise reproducible."""
    x, weight = x.contiguous(), weight.contiguous()
    dq, dk, dv = (t.to(x.dtype).contiguous() for t in (dq, dk, dv))
    args = _args(x, weight, head_dim, norm_channels, eps)
    B, T, C = x.shape
    dx = torch.empty_like(x)
    dw = torch.zeros_like(weight)
    ws = _lib.lib().pkda_qkv_conv_workspace(B, T, C // 3, weight.shape[1])
    part = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
    args.dq, args.dk, args.dv = _ptr(dq), _ptr(dk), _ptr(dv)
    args.dx, args.dw, args.dw_part = _ptr(dx), _ptr(dw), _ptr(part)
    with torch.cuda.device(x.device):
        _lib.call("pkda_qkv_conv_bwd", args, _stream(x.device))
    return dx, dw


@pkda_qkv_conv_backward.register_fake
def _pkda_qkv_conv_backward_fake(x, weight, dq, dk, dv, head_dim, norm_channels, eps):
    return torch.empty_like(x), torch.empty_like(weight)


def _setup_context(ctx, inputs, output) -> None:
    x, weight, head_dim, norm_channels, eps = inputs
    ctx.save_for_backward(x, weight)
    ctx.geometry = (head_dim, norm_channels, eps)


def _backward(ctx, dq, dk, dv):
    x, weight = ctx.saved_tensors
    head_dim, norm_channels, eps = ctx.geometry
    dx, dw = pkda_qkv_conv_backward(x, weight, dq, dk, dv, head_dim, norm_channels, eps)
    return dx, dw, None, None, None


pkda_qkv_conv.register_autograd(_backward, setup_context=_setup_context)
