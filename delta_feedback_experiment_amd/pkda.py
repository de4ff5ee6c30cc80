"""Host-side PKDA operators over the gfx950 library.

This mirrors the call surface ``PreconditionedKDA._cuda_recurrence`` binds
(``delta_feedback_experiment/pkda.py:412-475``):

* :func:`fused_recurrent_pkda` -- FLA's ``fused_recurrent_precond_kda``
  (pkda.py:473-474): token-recurrent forward, cached decode/eval;
* :func:`chunk_pkda` -- FLA's ``chunk_precond_kda`` (pkda.py:475): stateful,
  differentiable chunked forward/backward (in :mod:`.chunk`);
* :func:`pkda_decode_step_` -- the in-place slot-pool decode step;
* ``pkda_recurrence`` -- the stateless training custom op of
  ``delta_feedback_experiment/fla_ops.py:252-569`` (in :mod:`.ops`).

Every operator requires CUDA (HIP) tensors and the built library; there is
no CPU fallback.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dtype_code(t: Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.PKDA_F32
    if t.dtype == torch.bfloat16:
        return _lib.PKDA_BF16
    raise ValueError(f"PKDA supports float32 and bfloat16 activations, not {t.dtype}")


def _require_cuda(*tensors: Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("PKDA operators need tensors on a HIP device; there is no CPU fallback")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    return device


def _f32(t: Tensor | None) -> Tensor | None:
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def gate_form(g: Tensor, lead_shape: tuple[int, ...], K: int, use_gate_in_kernel: bool,
              A_log, dt_bias) -> tuple[int, Tensor]:
    """Classify ``g``: raw per-channel gate, per-channel or per-head log-decay.

    ``lead_shape`` is the token tensors' shape without the channel axis; ``g``
    must be that shape (per head) or that shape plus ``K`` (per channel).
    """
    per_head = tuple(g.shape) == tuple(lead_shape)
    if not per_head and tuple(g.shape) != (*lead_shape, K):
        raise ValueError(f"g {tuple(g.shape)} must be {tuple(lead_shape)} or {(*lead_shape, K)}")
    if use_gate_in_kernel:
        if A_log is None or dt_bias is None:
            raise ValueError("use_gate_in_kernel=True needs A_log and dt_bias")
        if per_head:  # a per-head raw value broadcast over channels
            g = g.unsqueeze(-1).expand(*lead_shape, K)
        return _lib.GATE_RAW_CHANNEL, g
    return (_lib.GATE_LOG_HEAD if per_head else _lib.GATE_LOG_CHANNEL), g


def _check_common(q, k, v, beta):
    if q.shape != k.shape:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} differ")
    if q.shape[:-1] != v.shape[:-1] or q.shape[-1] != v.shape[-1]:
        raise ValueError("PKDA needs dk == dv and matching q/v leading dims")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share one dtype")
    if beta.shape != q.shape[:-1]:
        raise ValueError(f"beta {tuple(beta.shape)} must be {tuple(q.shape[:-1])}")


def fused_recurrent_pkda(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    *,
    g_atk: Tensor | None = None,
    beta_atk: Tensor | None = None,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
    use_gate_in_kernel: bool = False,
    scale: float | None = None,
    initial_state: Tensor | None = None,
    initial_A_state: Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: Tensor | None = None,
    x: float = 1.0,
    eps: float = 1e-6,
    log_atk_scale: Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    check_cu_seqlens: bool = False,
    **_ignored,
) -> tuple[Tensor, Tensor | None, Tensor | None]:
    """Token-recurrent PKDA forward (no autograd): ``(o, S_T, A_T)``.

    Shapes as FLA's operator: ``q, k, v [B,T,H,D]``, ``g [B,T,H,D]`` raw gate
    (``use_gate_in_kernel``) or log-decay ``[B,T,H]``/``[B,T,H,D]``, ``beta
    [B,T,H]``, ``g_atk, beta_atk [B,T,H]``, ``log_atk_scale [H]`` (the
    preconditioner's log-space center), states ``[N,H,D,D]`` / ``[N,H,D]``
    FP32 where ``N = B`` or ``len(cu_seqlens) - 1``.  ``check_cu_seqlens``
    verifies ``cu_seqlens`` on the host first (synchronising); without it a
    malformed array is clamped on the device.
    """
    if use_qk_l2norm_in_kernel:
        raise ValueError("q and k arrive L2-normalised (pkda.py:464-465); in-kernel norm is not provided")
    _check_common(q, k, v, beta)
    device = _require_cuda(q, k, v, g, beta, g_atk, beta_atk, initial_state, initial_A_state, cu_seqlens)
    B, T, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    gate_kind, g = gate_form(g, q.shape[:-1], D, use_gate_in_kernel, A_log, dt_bias)
    if g_atk is not None and (beta_atk is None or log_atk_scale is None):
        raise ValueError("the preconditioner needs g_atk, beta_atk and log_atk_scale")
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1")
        from .chunk import ChunkPlan, validate_cu_seqlens

        if check_cu_seqlens:
            validate_cu_seqlens(cu_seqlens, T)
        # the kernel reads document bounds from the chunk table's sanitised
        # copy: a malformed cu_seqlens cannot send it past the token tensors
        with torch.cuda.device(device):
            cu = ChunkPlan.make(q, cu_seqlens).sanitized_cu
        N = cu.numel() - 1
        seqlen = 0
    else:
        cu = None
        N = B
        seqlen = T
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g = g.contiguous()
    if g.dtype not in (torch.float32, torch.bfloat16):
        g = g.float()
    beta32 = _f32(beta)
    o = torch.empty_like(v)
    S_T = torch.empty(N, H, D, D, device=device, dtype=torch.float32) if output_final_state else None
    A_T = (
        torch.empty(N, H, D, device=device, dtype=torch.float32)
        if output_final_state and g_atk is not None
        else None
    )
    s0 = _f32(initial_state)
    a0 = _f32(initial_A_state)
    if s0 is not None and tuple(s0.shape) != (N, H, D, D):
        raise ValueError(f"initial_state must be {(N, H, D, D)}")
    if a0 is not None and tuple(a0.shape) != (N, H, D):
        raise ValueError(f"initial_A_state must be {(N, H, D)}")
    # Converted temporaries are bound to locals so they outlive the enqueue.
    A_log32, dt32, gatk32, batk32, center32 = map(_f32, (A_log, dt_bias, g_atk, beta_atk, log_atk_scale))
    args = _lib.RecurrentArgs(
        dtype=_dtype_code(q), num_seqs=N, seqlen=seqlen, heads=H, head_dim=D,
        cu_seqlens=_ptr(cu), q=_ptr(q), k=_ptr(k), v=_ptr(v), g=_ptr(g),
        gate_kind=gate_kind, g_dtype=_dtype_code(g),
        A_log=_ptr(A_log32), dt_bias=_ptr(dt32), beta=_ptr(beta32), scale=float(scale),
        g_atk=_ptr(gatk32), beta_atk=_ptr(batk32), center=_ptr(center32),
        squash_x=float(x), squash_eps=float(eps),
        initial_state=_ptr(s0), initial_A_state=_ptr(a0),
        final_state=_ptr(S_T), final_A_state=_ptr(A_T), o=_ptr(o),
    )
    with torch.cuda.device(device):
        _lib.call("pkda_recurrent_fwd", args, _stream(device))
    return o, S_T, A_T


def _require_device(*tensors: Tensor | None) -> torch.device:
    """Device of the given tensors for the in-place serving operators: a HIP
    device, or the fake device of a trace (``torch.compile`` and ``make_fx``
    run the custom ops' fake implementations there).  CPU tensors are
    refused: there is no CPU fallback."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not (t.is_cuda or t.is_meta):
            raise RuntimeError("PKDA operators need tensors on a HIP device; there is no CPU fallback")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    return device


def check_slot_indices(slot_idx: Tensor, pool_size: int) -> None:
    """Host-side range and uniqueness check of slot indices (synchronises):
    the pools are updated in place, so a repeated slot would race."""
    host = slot_idx.cpu().tolist()
    seen = set()
    for i, s in enumerate(host):
        if s < 0 or s >= pool_size:
            raise IndexError(f"slot_idx[{i}] = {s} is out of range [0, {pool_size})")
        if s in seen:
            raise ValueError(f"slot_idx[{i}] = {s} is repeated: the pool is updated in place")
        seen.add(s)


def pkda_decode_step_(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    state_pool: Tensor,
    slot_idx: Tensor | None,
    *,
    a_pool: Tensor | None = None,
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
    out: Tensor | None = None,
) -> Tensor:
    """One decode token per live sequence, updating ``state_pool`` in place.

    ``q, k, v [N,H,D]``; ``g [N,H]`` or ``[N,H,D]``; ``beta [N,H]``;
    ``state_pool [P,H,D,D]`` FP32 (contiguous); ``slot_idx [N]`` int32 on the
    device (``None`` = slots ``0..N-1``).  Slots must be unique: the update is
    in place.  ``check_slots`` copies the indices to the host and verifies
    range and uniqueness first (a synchronising debug check).

    The launch is the custom op ``pkda_mi355x::decode_step_``, which declares
    ``state_pool``, ``a_pool`` and the output buffer as mutated, so
    ``torch.compile`` and functionalization see the in-place update.
    """
    _check_common(q, k, v, beta)
    _require_device(q, k, v, g, beta, state_pool, slot_idx, a_pool)
    N, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    if state_pool.dtype != torch.float32 or not state_pool.is_contiguous():
        raise ValueError("state_pool must be a contiguous float32 tensor")
    if tuple(state_pool.shape[1:]) != (H, D, D):
        raise ValueError(f"state_pool must be [P, {H}, {D}, {D}]")
    if a_pool is not None and (a_pool.dtype != torch.float32 or not a_pool.is_contiguous()
                               or tuple(a_pool.shape) != (state_pool.shape[0], H, D)):
        raise ValueError("a_pool must be a contiguous float32 [P, H, D] tensor")
    gate_form(g, q.shape[:-1], D, use_gate_in_kernel, A_log, dt_bias)  # shape check
    if slot_idx is not None:
        if slot_idx.dtype != torch.int32 or slot_idx.shape != (N,):
            raise ValueError("slot_idx must be int32 [N]")
        if check_slots:
            check_slot_indices(slot_idx, state_pool.shape[0])
    elif N > state_pool.shape[0]:
        raise ValueError("more sequences than pool slots")
    o = out if out is not None else torch.empty_like(v)
    if o.shape != v.shape or o.dtype != v.dtype or not o.is_contiguous():
        raise ValueError(f"out must be a contiguous {v.dtype} {tuple(v.shape)} tensor")
    decode_step_op(q, k, v, g, beta, state_pool, slot_idx, a_pool, g_atk, beta_atk, log_atk_scale, A_log, dt_bias,
                   bool(use_gate_in_kernel), float(scale), float(x), float(eps), o)
    return o


@torch.library.custom_op("pkda_mi355x::decode_step_", mutates_args=("state_pool", "a_pool", "o"),
                         device_types="cuda")
def decode_step_op(
    q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state_pool: Tensor, slot_idx: Tensor | None,
    a_pool: Tensor | None, g_atk: Tensor | None, beta_atk: Tensor | None, log_atk_scale: Tensor | None,
    A_log: Tensor | None, dt_bias: Tensor | None, use_gate_in_kernel: bool, scale: float, x: float, eps: float,
    o: Tensor,
) -> None:
    """The decode step's launch (arguments checked by :func:`pkda_decode_step_`):
    writes ``o`` and the indexed slots of ``state_pool`` / ``a_pool``."""
    device = _require_cuda(q, k, v, g, beta, state_pool, slot_idx, a_pool, o)
    N, H, D = q.shape
    gate_kind, g = gate_form(g, q.shape[:-1], D, use_gate_in_kernel, A_log, dt_bias)
    idx = None if slot_idx is None else slot_idx.contiguous()
    q, k, v, g = q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous()
    if g.dtype not in (torch.float32, torch.bfloat16):
        g = g.float()
    beta32 = _f32(beta)
    A_log32, dt32, gatk32, batk32, center32 = map(_f32, (A_log, dt_bias, g_atk, beta_atk, log_atk_scale))
    args = _lib.RecurrentArgs(
        dtype=_dtype_code(q), num_seqs=N, seqlen=1, heads=H, head_dim=D,
        q=_ptr(q), k=_ptr(k), v=_ptr(v), g=_ptr(g), gate_kind=gate_kind, g_dtype=_dtype_code(g),
        A_log=_ptr(A_log32), dt_bias=_ptr(dt32), beta=_ptr(beta32), scale=float(scale),
        g_atk=_ptr(gatk32), beta_atk=_ptr(batk32), center=_ptr(center32),
        squash_x=float(x), squash_eps=float(eps),
        state_pool=_ptr(state_pool), a_pool=_ptr(a_pool), pool_size=state_pool.shape[0],
        slot_idx=_ptr(idx), o=_ptr(o),
    )
    with torch.cuda.device(device):
        _lib.call("pkda_decode_step", args, _stream(device))


@decode_step_op.register_fake
def _decode_step_fake(q, k, v, g, beta, state_pool, slot_idx, a_pool, g_atk, beta_atk, log_atk_scale, A_log,
                      dt_bias, use_gate_in_kernel, scale, x, eps, o) -> None:
    return None
