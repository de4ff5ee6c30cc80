"""Host side of the diagonal write-key preconditioner scans.

The forward turns the raw key into the write key
``kw = k * exp(-ln(x) r / (1 + |r|))``, ``r = log(A + eps) - center`` with
``A_t = exp(g_atk_t) A_{t-1} + beta_atk_t k_t^2``
(``delta_feedback_experiment/pkda.py:392-398``), checkpointing ``A`` at every
chunk start; the backward is its reverse scan.  Both run in
``libpkda_gfx950.so`` (``pkda_precond_fwd`` / ``pkda_precond_bwd``),
chunk-parallel: local chunk ends (and each chunk's decay, handed to the
scan in a small workspace), a scan over each document's chunks, then the
chunks again from their entering values.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .pkda import _dtype_code, _f32, _ptr, _stream


@dataclass
class PrecondState:
    kw: Tensor            # [N_tok, H, K], dtype of k
    a_chunk: Tensor       # [num_chunks, H, K] FP32, A entering each chunk
    final_A: Tensor | None  # [N, H, K] FP32
    initial_A: Tensor | None
    kw32: Tensor | None = None  # kw in FP32 as well (when k is narrower and it was asked for)


def _flat2(t: Tensor, plan) -> Tensor:
    return _f32(t).reshape(plan.num_tokens, plan.heads)


def precond_forward(plan, kf: Tensor, g_atk: Tensor, beta_atk: Tensor, center: Tensor, x: float, eps: float,
                    initial_A_state: Tensor | None, *, slot_idx: Tensor | None = None,
                    final_A: Tensor | None = None, want_kw32: bool = False,
                    handoff: bool = True) -> PrecondState:
    """Write keys for flat ``kf [N_tok, H, K]``; returns the scan's state.

    With ``slot_idx`` the A states are rows of a pool: ``initial_A_state``
    (zero when ``None``) and ``final_A`` are contiguous FP32 ``[P, H, K]``,
    used in place (no conversion copy), document ``n`` at row ``slot_idx[n]``.
    ``want_kw32`` also returns the write keys in FP32 when ``kf`` is narrower
    (the chunk backward with per-channel gates sums its in-block pairs from
    them).  ``handoff=False`` passes no chunk-decay workspace: the document
    scan then sums every chunk's g_atk itself (the same bits, more loads)."""
    dev = kf.device
    H, K, N = plan.heads, plan.head_dim, plan.num_seqs
    ga, ba, cen = _flat2(g_atk, plan), _flat2(beta_atk, plan), _f32(center)
    if cen.shape != (H,):
        raise ValueError(f"log_atk_scale must be [{H}]")
    if slot_idx is not None:
        a0 = initial_A_state
    else:
        a0 = _f32(initial_A_state)
        if a0 is not None and tuple(a0.shape) != (N, H, K):
            raise ValueError(f"initial_A_state must be {(N, H, K)}")
    kw = torch.empty_like(kf)
    kw32 = torch.empty(kf.shape, device=dev, dtype=torch.float32) if want_kw32 and kf.dtype != torch.float32 else None
    a_chunk = torch.empty(plan.num_chunks, H, K, device=dev, dtype=torch.float32)
    decay = torch.empty(plan.num_chunks, H, device=dev, dtype=torch.float32) if handoff else None
    if final_A is None:
        final_A = torch.empty(N, H, K, device=dev, dtype=torch.float32)
    args = _lib.PrecondArgs(
        dtype=_dtype_code(kf), num_seqs=N, seqlen=plan.seqlen, heads=H, head_dim=K,
        cu_seqlens=_ptr(plan.cu_seqlens), k=_ptr(kf), g_atk=_ptr(ga), beta_atk=_ptr(ba), center=_ptr(cen),
        squash_x=float(x), squash_eps=float(eps), initial_A_state=_ptr(a0), final_A_state=_ptr(final_A),
        kw=_ptr(kw), a_chunk=_ptr(a_chunk), num_chunks=plan.num_chunks, table=_ptr(plan.table),
        slot_idx=_ptr(slot_idx), pool_size=final_A.shape[0] if slot_idx is not None else 0, kw32=_ptr(kw32),
        chunk_decay=_ptr(decay),
    )
    _lib.call("pkda_precond_fwd", args, _stream(dev))
    return PrecondState(kw, a_chunk, final_A, a0, kw32)


def precond_backward(plan, kf: Tensor, g_atk: Tensor, beta_atk: Tensor, center: Tensor, x: float, eps: float,
                     state: PrecondState, dkw: Tensor, dk: Tensor, dA_T: Tensor | None, want_dA0: bool,
                     dk_final: Tensor | None = None, handoff: bool = True):
    """Reverse scan: adds the preconditioner's terms into ``dk`` (FP32, in
    place) -- or, with ``dk_final`` (``kf``'s shape and dtype), writes the
    sum there and leaves ``dk`` alone -- and returns ``(dg_atk [N_tok,H],
    dbeta_atk [N_tok,H], dcenter [H], dA0 [N,H,K] or None)``, all FP32.

    ``dkw`` and ``dk`` come in FP32, or both in ``kf``'s dtype (the chunk
    backward's key gradients as it rounds them once); the narrow form needs
    ``dk_final``.  ``handoff`` as in ``precond_forward``."""
    dev = kf.device
    H, K, N = plan.heads, plan.head_dim, plan.num_seqs
    ga, ba, cen = _flat2(g_atk, plan), _flat2(beta_atk, plan), _f32(center)
    f32 = dict(device=dev, dtype=torch.float32)
    dg_atk = torch.empty(plan.num_tokens, H, **f32)
    dbeta_atk = torch.empty(plan.num_tokens, H, **f32)
    dcenter_part = torch.empty(max(plan.num_chunks, 1), H, **f32)
    lam_chunk = torch.empty(plan.num_chunks, H, K, **f32)
    decay = torch.empty(plan.num_chunks, H, **f32) if handoff else None
    dcenter = torch.empty(H, **f32)
    dA0 = torch.empty(N, H, K, **f32) if want_dA0 else None
    dAT = None if dA_T is None else _f32(dA_T)
    narrow = dkw.dtype != torch.float32
    if narrow and (dkw.dtype != kf.dtype or dk.dtype != kf.dtype or dk_final is None):
        raise ValueError("dkw and dk must be FP32, or both in k's dtype with dk_final given")
    if not narrow and dk.dtype != torch.float32:
        raise ValueError("dk must be FP32 when dkw is")
    args = _lib.PrecondArgs(
        dtype=_dtype_code(kf), num_seqs=N, seqlen=plan.seqlen, heads=H, head_dim=K,
        cu_seqlens=_ptr(plan.cu_seqlens), k=_ptr(kf), g_atk=_ptr(ga), beta_atk=_ptr(ba), center=_ptr(cen),
        squash_x=float(x), squash_eps=float(eps), a_chunk=_ptr(state.a_chunk), num_chunks=plan.num_chunks,
        dkw=_ptr(dkw), dk=_ptr(dk), dg_atk=_ptr(dg_atk), dbeta_atk=_ptr(dbeta_atk),
        dcenter_part=_ptr(dcenter_part), dcenter=_ptr(dcenter), dA0=_ptr(dA0), dA_T=_ptr(dAT),
        table=_ptr(plan.table), lam_chunk=_ptr(lam_chunk), dk_final=_ptr(dk_final),
        grad_dtype=_dtype_code(dkw) if narrow else _lib.PKDA_F32, chunk_decay=_ptr(decay),
    )
    if dk_final is not None and (dk_final.shape != kf.shape or dk_final.dtype != kf.dtype
                                 or not dk_final.is_contiguous()):
        raise ValueError("dk_final must be contiguous with k's shape and dtype")
    _lib.call("pkda_precond_bwd", args, _stream(dev))
    return dg_atk, dbeta_atk, dcenter, dA0
