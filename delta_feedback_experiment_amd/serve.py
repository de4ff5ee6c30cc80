"""Slot-pool serving: cached prefill into decode slots, and the short-convolution
histories that travel with them.

The reference's decode cache keeps, per PKDA layer and sequence, the FP32
matrix state ``S [H, d, d]``, the preconditioner state ``A [H, d]`` and the
three raw-projection histories of the Q/K/V short convolutions
(``KVCache.pkda_states``, ``delta_feedback_experiment/model.py:391-471``).
Cached prefill is ``chunk_precond_kda(..., output_final_state=True)``
(``delta_feedback_experiment/pkda.py:450-475``), and the convolution prepends
the stored history to the new projections and keeps the last ``conv_size - 1``
rows (``delta_feedback_experiment/pkda.py:240-260``).

Here every one of those states lives in a slot pool indexed by an int32 slot
per sequence, the layout :func:`pkda_decode_step_` already updates in place:

* ``state [P, H, d, d]`` FP32 and ``a [P, H, d]`` FP32;
* ``conv [P, conv_size - 1, 3 * H * d]`` in the projection dtype: the raw
  Q/K/V projection rows of the last ``conv_size - 1`` positions, oldest first,
  side by side as :func:`pkda_qkv_conv` takes them.

:func:`pkda_prefill_` runs the chunked forward with each document's states
read from (``continue_state``) and written to its slot by the kernels
themselves; :func:`pkda_qkv_conv_cached_` runs the fused convolution with the
slot's history in front of the rows and leaves the new history in the slot.
A decode token is the same convolution call with one row per sequence,
followed by :func:`pkda_decode_step_`.  None of these record autograd history.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .chunk import ChunkPlan, _flat, chunk_forward, gate_forward, validate_cu_seqlens, wants_gcum_lo
from .pkda import (_check_common, _dtype_code, _f32, _ptr, _require_cuda, _require_device, _stream,
                   check_slot_indices, gate_form)


@dataclass
class DecodePool:
    """The decode states of one PKDA layer for ``slots`` sequences."""

    state: Tensor           # [P, H, d, d] FP32
    a: Tensor | None        # [P, H, d] FP32 (preconditioner), or None
    conv: Tensor | None     # [P, conv_size - 1, 3 * H * d] projection dtype, or None

    @staticmethod
    def zeros(slots: int, heads: int, head_dim: int, *, conv_size: int = 4, dtype: torch.dtype = torch.bfloat16,
              precond: bool = True, device: torch.device | str = "cuda") -> "DecodePool":
        f32 = dict(device=device, dtype=torch.float32)
        conv = None
        if conv_size > 1:
            conv = torch.zeros(slots, conv_size - 1, 3 * heads * head_dim, device=device, dtype=dtype)
        return DecodePool(
            state=torch.zeros(slots, heads, head_dim, head_dim, **f32),
            a=torch.zeros(slots, heads, head_dim, **f32) if precond else None,
            conv=conv,
        )


def _slots(slot_idx: Tensor, n: int, pool_size: int, check: bool) -> None:
    if slot_idx.dtype != torch.int32 or tuple(slot_idx.shape) != (n,):
        raise ValueError(f"slot_idx must be int32 [{n}]")
    if check:
        check_slot_indices(slot_idx, pool_size)


def pkda_prefill_(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    state_pool: Tensor,
    slot_idx: Tensor,
    *,
    a_pool: Tensor | None = None,
    continue_state: bool = False,
    cu_seqlens: Tensor | None = None,
    g_atk: Tensor | None = None,
    beta_atk: Tensor | None = None,
    log_atk_scale: Tensor | None = None,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
    use_gate_in_kernel: bool = False,
    scale: float | None = None,
    x: float = 1.0,
    eps: float = 1e-6,
    check_slots: bool = False,
    check_cu_seqlens: bool = False,
) -> Tensor:
    """Chunked prefill whose final states land in pool slots; returns ``o``.

    Arguments as :func:`chunk_pkda` (``q, k, v [B, T, H, d]``, or ``B = 1``
    with ``cu_seqlens`` for packed documents; ``g`` raw or log-decay, per head
    or per channel; the preconditioner when ``g_atk`` is given), plus
    ``state_pool [P, H, d, d]`` and, with the preconditioner, ``a_pool
    [P, H, d]`` (both contiguous FP32, updated in place) and ``slot_idx``
    (int32 ``[N]`` on the device, one unique slot per row or document).
    ``continue_state=False`` starts every sequence from zero states (a new
    prompt); ``True`` continues from the states in its slot (a prompt
    extended in pieces).  ``check_slots`` verifies range and uniqueness on the
    host first (synchronising); ``check_cu_seqlens`` likewise that
    ``cu_seqlens`` rises from 0 to the packed length (a malformed one is
    otherwise clamped on the device).
    """
    _check_common(q, k, v, beta)
    _require_device(q, k, v, g, beta, state_pool, slot_idx, a_pool, cu_seqlens, g_atk, beta_atk,
                    log_atk_scale, A_log, dt_bias)
    B, T, H, D = q.shape
    if state_pool.dtype != torch.float32 or not state_pool.is_contiguous() or tuple(state_pool.shape[1:]) != (H, D, D):
        raise ValueError(f"state_pool must be a contiguous float32 [P, {H}, {D}, {D}] tensor")
    P = state_pool.shape[0]
    if g_atk is not None:
        if beta_atk is None or log_atk_scale is None:
            raise ValueError("the preconditioner needs g_atk, beta_atk and log_atk_scale")
        if a_pool is None:
            raise ValueError("with the preconditioner the A states need a_pool")
    if a_pool is not None and (a_pool.dtype != torch.float32 or not a_pool.is_contiguous()
                               or tuple(a_pool.shape) != (P, H, D)):
        raise ValueError(f"a_pool must be a contiguous float32 [{P}, {H}, {D}] tensor")
    if cu_seqlens is not None and B != 1:
        raise ValueError("cu_seqlens requires batch size 1")
    if check_cu_seqlens and cu_seqlens is not None:
        validate_cu_seqlens(cu_seqlens, T)
    gate_form(g, q.shape[:-1], D, use_gate_in_kernel, A_log, dt_bias)  # shape check
    N = B if cu_seqlens is None else cu_seqlens.numel() - 1
    _slots(slot_idx, N, P, check_slots)
    if scale is None:
        scale = D ** -0.5
    o = torch.empty_like(v)
    prefill_op(q, k, v, g, beta, state_pool, slot_idx, a_pool, bool(continue_state), cu_seqlens, g_atk, beta_atk,
               log_atk_scale, A_log, dt_bias, bool(use_gate_in_kernel), float(scale), float(x), float(eps), o)
    return o


@torch.library.custom_op("pkda_mi355x::prefill_", mutates_args=("state_pool", "a_pool", "o"), device_types="cuda")
def prefill_op(
    q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state_pool: Tensor, slot_idx: Tensor,
    a_pool: Tensor | None, continue_state: bool, cu_seqlens: Tensor | None, g_atk: Tensor | None,
    beta_atk: Tensor | None, log_atk_scale: Tensor | None, A_log: Tensor | None, dt_bias: Tensor | None,
    use_gate_in_kernel: bool, scale: float, x: float, eps: float, o: Tensor,
) -> None:
    """The prefill's launches (arguments checked by :func:`pkda_prefill_`):
    writes ``o`` and the final S (and A) of every document into its slot."""
    device = _require_cuda(q, k, v, g, beta, state_pool, slot_idx, a_pool, cu_seqlens, g_atk, beta_atk,
                           log_atk_scale, A_log, dt_bias, o)
    H, D = q.shape[2], q.shape[3]
    idx = slot_idx.contiguous()
    from . import precond as pre

    with torch.no_grad(), torch.cuda.device(device):
        plan = ChunkPlan.make(q, cu_seqlens)
        kind, g_used = gate_form(g, q.shape[:-1], D, use_gate_in_kernel, A_log, dt_bias)
        g_used = g_used.contiguous()
        if g_used.dtype not in (torch.float32, torch.bfloat16):
            g_used = g_used.float()
        A_log32, dt32 = _f32(A_log), _f32(dt_bias)
        qf, kf, vf = (_flat(t.contiguous(), plan) for t in (q, k, v))
        beta32 = _f32(beta).reshape(plan.num_tokens, H)
        gcum_lo = None
        if wants_gcum_lo(kind, q.dtype):  # as chunk_pkda takes it
            gcum_lo = torch.empty(plan.num_tokens, H, D, device=device, dtype=torch.float32)
        gcum = gate_forward(plan, _flat(g_used, plan), kind, A_log32, dt32, gcum_lo=gcum_lo)
        kwf = kf
        if g_atk is not None:
            pstate = pre.precond_forward(plan, kf, g_atk, beta_atk, log_atk_scale, x, eps,
                                         a_pool if continue_state else None, slot_idx=idx, final_A=a_pool)
            kwf = pstate.kw
        chunk_forward(plan, qf, kf, kwf, vf, gcum, beta32, float(scale),
                      state_pool if continue_state else None, True, False,
                      slot_idx=idx, final_state=state_pool, out=_flat(o, plan), gcum_lo=gcum_lo)


@prefill_op.register_fake
def _prefill_fake(q, k, v, g, beta, state_pool, slot_idx, a_pool, continue_state, cu_seqlens, g_atk, beta_atk,
                  log_atk_scale, A_log, dt_bias, use_gate_in_kernel, scale, x, eps, o) -> None:
    return None


def pkda_qkv_conv_cached_(
    x: Tensor,
    weight: Tensor,
    head_dim: int,
    norm_channels: int,
    eps: float,
    conv_pool: Tensor,
    slot_idx: Tensor | None = None,
    *,
    continue_state: bool = True,
    check_slots: bool = False,
) -> tuple[Tensor, Tensor, Tensor]:
    """:func:`pkda_qkv_conv` on rows that continue a cached history.

    ``x [B, T, 3 * width]`` are the new raw projections of ``B`` sequences;
    ``conv_pool [P, conv_size - 1, 3 * width]`` (``x.dtype``, contiguous)
    holds each slot's history, oldest row first.  Row ``b`` reads the history
    of slot ``slot_idx[b]`` (``b`` when ``None``) -- or zeros when
    ``continue_state`` is false, a new prompt -- and that slot receives the
    last ``conv_size - 1`` rows of history ++ x.  ``T = 1`` is the decode
    token.  Returns ``(q, k, v)`` ``[B, T, width]`` as :func:`pkda_qkv_conv`.
    """
    _require_device(x, weight, conv_pool, slot_idx)
    if x.dim() != 3 or weight.dim() != 2 or x.shape[-1] != weight.shape[0] or x.shape[-1] % 3:
        raise ValueError(f"x [B, T, 3 * width] and weight [3 * width, conv_size] expected, got "
                         f"{tuple(x.shape)} and {tuple(weight.shape)}")
    B, T, Cx = x.shape
    W = weight.shape[1]
    if W < 2:
        raise ValueError("conv_size 1 keeps no history")
    if (conv_pool.dtype != x.dtype or not conv_pool.is_contiguous()
            or tuple(conv_pool.shape[1:]) != (W - 1, Cx)):
        raise ValueError(f"conv_pool must be a contiguous {x.dtype} [P, {W - 1}, {Cx}] tensor")
    P = conv_pool.shape[0]
    if slot_idx is not None:
        _slots(slot_idx, B, P, check_slots)
    elif B > P:
        raise ValueError("more rows than pool slots")
    return qkv_conv_cached_op(x, weight, int(head_dim), int(norm_channels), float(eps), conv_pool, slot_idx,
                              bool(continue_state))


@torch.library.custom_op("pkda_mi355x::qkv_conv_cached_", mutates_args=("conv_pool",), device_types="cuda")
def qkv_conv_cached_op(
    x: Tensor, weight: Tensor, head_dim: int, norm_channels: int, eps: float, conv_pool: Tensor,
    slot_idx: Tensor | None, continue_state: bool,
) -> tuple[Tensor, Tensor, Tensor]:
    """The cached convolution's launch (arguments checked by
    :func:`pkda_qkv_conv_cached_`): returns ``(q, k, v)`` and leaves each
    slot's new history in ``conv_pool``."""
    _require_cuda(x, weight, conv_pool, slot_idx)
    B, T, Cx = x.shape
    W = weight.shape[1]
    P = conv_pool.shape[0]
    idx = None if slot_idx is None else slot_idx.contiguous()
    x, weight = x.contiguous(), weight.contiguous()
    q, k, v = (torch.empty(B, T, Cx // 3, device=x.device, dtype=x.dtype) for _ in range(3))
    args = _lib.QkvConvArgs(
        dtype=_dtype_code(x), w_dtype=_dtype_code(weight), batch=B, seqlen=T, width=Cx // 3,
        head_dim=int(head_dim), norm_channels=int(norm_channels), conv_size=W, eps=float(eps),
        x=_ptr(x), weight=_ptr(weight), q=_ptr(q), k=_ptr(k), v=_ptr(v),
        slot_idx=_ptr(idx), history_in=_ptr(conv_pool) if continue_state else None,
        history_out=_ptr(conv_pool), pool_size=P,
    )
    with torch.no_grad(), torch.cuda.device(x.device):
        _lib.call("pkda_qkv_conv_fwd", args, _stream(x.device))
    return q, k, v


@qkv_conv_cached_op.register_fake
def _qkv_conv_cached_fake(x, weight, head_dim, norm_channels, eps, conv_pool, slot_idx, continue_state):
    B, T, Cx = x.shape
    return tuple(x.new_empty(B, T, Cx // 3) for _ in range(3))
