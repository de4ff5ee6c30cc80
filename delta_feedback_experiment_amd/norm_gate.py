"""RMSNorm with a sigmoid output gate, as a custom op.

Mirrors ``delta_feedback::pkda_norm_gate`` and its backward op
(``delta_feedback_experiment/fla_ops.py:572-657``): ``(x, gate, weight, eps)
-> (y, rstd)`` with ``y = x rstd weight sigmoid(gate)`` over the last
dimension and ``rstd [rows]`` FP32 for the backward, which returns
``(dx, dgate, dweight)`` in the dtypes of ``x``, ``gate`` and ``weight``.
``PreconditionedKDA.forward`` applies it to the recurrence output
(``delta_feedback_experiment/pkda.py:536-547``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .pkda import _dtype_code, _ptr, _stream


def _args(x: Tensor, gate: Tensor, weight: Tensor, eps: float) -> _lib.NormGateArgs:
    if gate.shape != x.shape or weight.dim() != 1 or weight.numel() != x.shape[-1]:
        raise ValueError(f"x and gate of one shape [..., d] and weight [d] expected, got {tuple(x.shape)}, "
                         f"{tuple(gate.shape)}, {tuple(weight.shape)}")
    if not (x.is_cuda and gate.is_cuda and weight.is_cuda):
        raise RuntimeError("pkda_norm_gate needs tensors on a HIP device; there is no CPU fallback")
    return _lib.NormGateArgs(dtype=_dtype_code(x), w_dtype=_dtype_code(weight), dim=x.shape[-1],
                             rows=x.numel() // max(x.shape[-1], 1), eps=float(eps))


@torch.library.custom_op("pkda_mi355x::pkda_norm_gate", mutates_args=(), device_types="cuda")
def pkda_norm_gate(x: Tensor, gate: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """Fused RMSNorm with a sigmoid output gate; ``rstd`` feeds the backward
    (fla_ops.py:572-593)."""
    x, gate, weight = x.contiguous(), gate.to(x.dtype).contiguous(), weight.contiguous()
    args = _args(x, gate, weight, eps)
    y = torch.empty_like(x)
    rstd = torch.empty(args.rows, device=x.device, dtype=torch.float32)
    args.x, args.gate, args.weight, args.y, args.rstd = _ptr(x), _ptr(gate), _ptr(weight), _ptr(y), _ptr(rstd)
    with torch.cuda.device(x.device):
        _lib.call("pkda_norm_gate_fwd", args, _stream(x.device))
    return y, rstd


@pkda_norm_gate.register_fake
def _pkda_norm_gate_fake(x, gate, weight, eps):
    rows = x.numel() // x.shape[-1]
    return torch.empty_like(x), torch.empty((rows,), device=x.device, dtype=torch.float32)


@torch.library.custom_op("pkda_mi355x::pkda_norm_gate_backward", mutates_args=(), device_types="cuda")
def pkda_norm_gate_backward(x: Tensor, gate: Tensor, weight: Tensor, rstd: Tensor, dy: Tensor,
                            eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """``(dx, dgate, dweight)`` (fla_ops.py:610-637); ``dweight`` is a
    fixed-order sum over rows: bitwise reproducible."""
    gate_dtype = gate.dtype
    x, weight = x.contiguous(), weight.contiguous()
    gate, dy = gate.to(x.dtype).contiguous(), dy.to(x.dtype).contiguous()
    args = _args(x, gate, weight, eps)
    dx, dgate = torch.empty_like(x), torch.empty_like(x)
    dw = torch.zeros_like(weight)
    ws = _lib.lib().pkda_norm_gate_workspace(args.rows, args.dim)
    part = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
    args.x, args.gate, args.weight, args.rstd, args.dy = _ptr(x), _ptr(gate), _ptr(weight), _ptr(rstd), _ptr(dy)
    args.dx, args.dgate, args.dw, args.dw_part = _ptr(dx), _ptr(dgate), _ptr(dw), _ptr(part)
    with torch.cuda.device(x.device):
        _lib.call("pkda_norm_gate_bwd", args, _stream(x.device))
    return dx, dgate.to(gate_dtype), dw


@pkda_norm_gate_backward.register_fake
def _pkda_norm_gate_backward_fake(x, gate, weight, rstd, dy, eps):
    return torch.empty_like(x), torch.empty_like(gate), torch.empty_like(weight)


def _setup_context(ctx, inputs, output) -> None:
    x, gate, weight, eps = inputs
    _y, rstd = output
    ctx.save_for_backward(x, gate, weight, rstd)
    ctx.eps = eps
    ctx.mark_non_differentiable(rstd)


def _backward(ctx, dy, _drstd):
    x, gate, weight, rstd = ctx.saved_tensors
    dx, dgate, dw = pkda_norm_gate_backward(x, gate, weight, rstd, dy, ctx.eps)
    return dx, dgate, dw, None


pkda_norm_gate.register_autograd(_backward, setup_context=_setup_context)
