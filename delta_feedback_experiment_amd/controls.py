"""PKDA control activations and their packed gradient.

``PreconditionedKDA._controls`` (``delta_feedback_experiment/pkda.py:318-353``)
projects each token once to five control slices side by side,

    decay hidden [K] | beta logits [H] | precond decay logits [H] |
    precond beta logits [H] | output-gate hidden [K],

splits them (``_PackedControlSplit``, ``pkda.py:56-74``) and activates the
middle three.  Its backward assembles the five slice gradients into one
packed buffer (``pack_control_gradients``,
``delta_feedback_experiment/cuda_kernels.py:1081-1172``).

:func:`pkda_controls` is that split and activation with the reference's
outputs: the two hidden slices are views of ``packed`` (as the reference's
split returns them), ``beta`` and ``precond_beta`` come in ``packed.dtype``,
``precond_decay = -exp(A_log_p) softplus(logit + dt_bias_p)`` in FP32.  Its
backward is one kernel that writes the packed gradient with the sigmoid and
softplus derivatives already applied, plus the FP32 gradients of
``A_log_p`` and ``dt_bias_p`` (fixed-order sums).  The decay hidden is meant
for :func:`chunk_pkda`'s ``decay_up`` form, which expands it inside the gate
kernel instead of materialising the raw decay.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .pkda import _dtype_code, _f32, _ptr, _stream


def _rows(packed: Tensor, width: int) -> tuple[Tensor, int, int]:
    """``packed [..., >= width]`` as evenly strided rows: (tensor, rows, row_stride)."""
    rows = packed.numel() // packed.shape[-1] if packed.shape[-1] else 0
    flat = packed.reshape(rows, packed.shape[-1])
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    return flat, rows, flat.stride(0) if rows else width


def _args(packed: Tensor, A_log_p: Tensor, dt_bias_p: Tensor, rank: int, heads: int) -> tuple:
    if not (packed.is_cuda and A_log_p.is_cuda and dt_bias_p.is_cuda):
        raise RuntimeError("pkda_controls needs tensors on a HIP device; there is no CPU fallback")
    width = packed.shape[-1]
    gate_width = width - rank - 3 * heads
    if gate_width < 0 or A_log_p.shape != (heads,) or dt_bias_p.shape != (heads,):
        raise ValueError(f"packed [..., rank + 3 H + gate_width] with A_log_p, dt_bias_p [H] expected, got "
                         f"{tuple(packed.shape)}, rank {rank}, H {heads}")
    flat, rows, stride = _rows(packed, width)
    A32, dt32 = _f32(A_log_p), _f32(dt_bias_p)
    args = _lib.ControlsArgs(dtype=_dtype_code(packed), rows=rows, heads=heads, rank=rank, gate_width=gate_width,
                             row_stride=stride, packed=_ptr(flat), A_log_p=_ptr(A32), dt_bias_p=_ptr(dt32))
    return args, flat, A32, dt32, gate_width


@torch.library.custom_op("pkda_mi355x::pkda_controls_act", mutates_args=(), device_types="cuda")
def pkda_controls_act(packed: Tensor, A_log_p: Tensor, dt_bias_p: Tensor, rank: int,
                      heads: int) -> tuple[Tensor, Tensor, Tensor]:
    """``(beta, precond_decay, precond_beta)`` ``[..., H]`` of the packed controls."""
    args, flat, A32, dt32, _ = _args(packed, A_log_p, dt_bias_p, rank, heads)
    lead = packed.shape[:-1]
    beta = torch.empty(*lead, heads, device=packed.device, dtype=packed.dtype)
    pbeta = torch.empty_like(beta)
    pdecay = torch.empty(*lead, heads, device=packed.device, dtype=torch.float32)
    args.beta, args.precond_decay, args.precond_beta = _ptr(beta), _ptr(pdecay), _ptr(pbeta)
    with torch.cuda.device(packed.device):
        _lib.call("pkda_controls_fwd", args, _stream(packed.device))
    return beta, pdecay, pbeta


@pkda_controls_act.register_fake
def _pkda_controls_act_fake(packed, A_log_p, dt_bias_p, rank, heads):
    lead = packed.shape[:-1]
    beta = packed.new_empty(*lead, heads)
    return beta, packed.new_empty(*lead, heads, dtype=torch.float32), packed.new_empty(*lead, heads)


@torch.library.custom_op("pkda_mi355x::pkda_controls_backward", mutates_args=(), device_types="cuda")
def pkda_controls_backward(packed: Tensor, A_log_p: Tensor, dt_bias_p: Tensor, d_decay_hidden: Tensor | None,
                           dbeta: Tensor | None, dprecond_decay: Tensor | None, dprecond_beta: Tensor | None,
                           d_gate_hidden: Tensor | None, rank: int, heads: int) -> tuple[Tensor, Tensor, Tensor]:
    """``(dpacked [..., width] contiguous, dA_log_p [H], ddt_bias_p [H])``;
    a missing slice gradient counts as zero (pkda.py:65-73)."""
    args, flat, A32, dt32, gw = _args(packed, A_log_p, dt_bias_p, rank, heads)
    width = packed.shape[-1]
    lead = packed.shape[:-1]
    dev = packed.device

    def prep(t, cols, dtype):
        return None if t is None else t.to(dtype).reshape(args.rows, cols).contiguous()

    dh = prep(d_decay_hidden, rank, packed.dtype)
    db = prep(dbeta, heads, packed.dtype)
    dpd = prep(dprecond_decay, heads, torch.float32)
    dpb = prep(dprecond_beta, heads, packed.dtype)
    dg = prep(d_gate_hidden, gw, packed.dtype)
    dpacked = torch.empty(*lead, width, device=dev, dtype=packed.dtype)
    part = torch.empty(max(_lib.lib().pkda_controls_workspace(args.rows, heads), 1), device=dev, dtype=torch.float32)
    dA = torch.empty(heads, device=dev, dtype=torch.float32)
    ddt = torch.empty(heads, device=dev, dtype=torch.float32)
    args.d_decay_hidden, args.dbeta, args.dprecond_decay = _ptr(dh), _ptr(db), _ptr(dpd)
    args.dprecond_beta, args.d_gate_hidden = _ptr(dpb), _ptr(dg)
    args.dpacked, args.part, args.dA_log_p, args.ddt_bias_p = _ptr(dpacked), _ptr(part), _ptr(dA), _ptr(ddt)
    with torch.cuda.device(dev):
        _lib.call("pkda_controls_bwd", args, _stream(dev))
    return dpacked, dA.to(A_log_p.dtype), ddt.to(dt_bias_p.dtype)


@pkda_controls_backward.register_fake
def _pkda_controls_backward_fake(packed, A_log_p, dt_bias_p, d_decay_hidden, dbeta, dprecond_decay, dprecond_beta,
                                 d_gate_hidden, rank, heads):
    return packed.new_empty(packed.shape), torch.empty_like(A_log_p), torch.empty_like(dt_bias_p)


class _Controls(torch.autograd.Function):
    """Five control tensors whose backward writes one packed gradient buffer."""

    @staticmethod
    def forward(ctx, packed, A_log_p, dt_bias_p, rank, heads):
        beta, pdecay, pbeta = pkda_controls_act(packed, A_log_p, dt_bias_p, rank, heads)
        ctx.save_for_backward(packed, A_log_p, dt_bias_p)
        ctx.geometry = (rank, heads)
        return packed[..., :rank], beta, pdecay, pbeta, packed[..., rank + 3 * heads:]

    @staticmethod
    def backward(ctx, d_hidden, dbeta, dpdecay, dpbeta, d_gate):
        packed, A_log_p, dt_bias_p = ctx.saved_tensors
        rank, heads = ctx.geometry
        dpacked, dA, ddt = pkda_controls_backward(packed, A_log_p, dt_bias_p, d_hidden, dbeta, dpdecay, dpbeta,
                                                  d_gate, rank, heads)
        return dpacked, dA, ddt, None, None


def pkda_controls(packed: Tensor, A_log_precond: Tensor, dt_bias_precond: Tensor, head_dim: int,
                  num_heads: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """``(decay_hidden, beta, precond_decay, precond_beta, output_gate_hidden)``
    of the packed control projection ``[..., 2 head_dim + 3 num_heads]``
    (``control_splits = (d, H, H, H, d)``, pkda.py:158-165), as
    ``PreconditionedKDA._controls`` produces them before the decay expansion."""
    return _Controls.apply(packed, A_log_precond, dt_bias_precond, int(head_dim), int(num_heads))
