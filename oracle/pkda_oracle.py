"""CPU restatement of the PKDA recurrence -- TEST INFRASTRUCTURE ONLY.

This module is the parity checker for the HIP path.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never routes through it.

It restates, token by token and in the same FP32 evaluation order, the
reference's portable recurrence ``PreconditionedKDA._portable_recurrence``
(``delta_feedback_experiment/pkda.py:355-410``) together with the pieces the
reference composes around it:

* per-head Q/K L2 normalisation ``x * rsqrt(sum(x^2) + 1e-6)``
  (``delta_feedback_experiment/pkda.py:37-44``);
* the in-kernel gate ``g = -exp(A_log[h]) * softplus(g_raw + dt_bias[h, c])``
  (``delta_feedback_experiment/pkda.py:375-377``);
* the diagonal write-key preconditioner
  ``A_t = exp(g_atk) A_{t-1} + beta_atk k*k``, ``r = log(A + eps) - center``,
  ``k_write = k * exp(-ln(x) r / (1 + |r|))``
  (``delta_feedback_experiment/pkda.py:392-398``);
* the delta rule with the prediction read by the raw key and the write by the
  preconditioned key, and the output read from the updated state
  (``delta_feedback_experiment/pkda.py:399-406``).

Extensions the reference exposes through FLA's signature but never exercises
(``cu_seqlens`` document packing, a per-head scalar log-decay passed directly)
are restated here as compositions of the same literal loop: packed documents
run independently from their own initial state, and a ``[B, T, H]`` log-decay
is the ``[B, T, H, K]`` one broadcast over key channels.

Pinning: ``tests/test_oracle.py`` checks this module against golden vectors
written from the reference's own ``_portable_recurrence`` (``tests/golden``),
against closed forms (single step, zero write strength, associative recall
with orthonormal keys, the constant preconditioner at ``beta_atk = 0``) and
against an independent FP64 chunk-form evaluation (``pkda_chunk_oracle``).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

QK_NORM_EPS = 1e-6
"""Epsilon of the per-head Q/K normalisation (pkda.py:37)."""


def l2norm(t: Tensor) -> Tensor:
    """FP32 per-head L2 normalisation returned in the input dtype (pkda.py:41-44)."""
    f = t.float()
    return (f * torch.rsqrt(f.square().sum(-1, keepdim=True) + QK_NORM_EPS)).to(t.dtype)


def gate_log_decay(g_raw: Tensor, A_log: Tensor, dt_bias: Tensor, dtype=torch.float32) -> Tensor:
    """``-exp(A_log[h]) * softplus(g_raw + dt_bias[h, c])`` (pkda.py:375-377).

    ``g_raw`` is ``[B, T, H, K]``; ``A_log`` is ``[H]``; ``dt_bias`` is ``[H*K]``.
    """
    H, K = g_raw.shape[-2], g_raw.shape[-1]
    return -A_log.to(dtype).exp()[None, None, :, None] * F.softplus(
        g_raw.to(dtype) + dt_bias.to(dtype).view(1, 1, H, K)
    )


def precond_gate_log_decay(logits: Tensor, A_log_p: Tensor, dt_bias_p: Tensor) -> Tensor:
    """Preconditioner log-decay ``-exp(A_log_p) softplus(logit + dt_bias_p)``
    (pkda.py:343-345); the operator receives it already activated, in FP32."""
    return -A_log_p.float().exp() * F.softplus(logits.float() + dt_bias_p)


def _expand_gate(g_log: Tensor, K: int) -> Tensor:
    if g_log.dim() == 3:
        return g_log.unsqueeze(-1).expand(*g_log.shape, K)
    return g_log


def recurrence(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g_log: Tensor,
    beta: Tensor,
    *,
    scale: float,
    g_atk: Tensor | None = None,
    beta_atk: Tensor | None = None,
    center: Tensor | None = None,
    squash_x: float = 1.0,
    squash_eps: float = 1e-6,
    state: Tensor | None = None,
    a_state: Tensor | None = None,
    dtype: torch.dtype = torch.float32,
) -> tuple[Tensor, Tensor, Tensor | None]:
    """The literal recurrence over one batch of equal-length rows.

    Shapes: ``q, k [B,T,H,K]``, ``v [B,T,H,V]``, ``g_log [B,T,H,K]`` or
    ``[B,T,H]`` (natural-log decay, <= 0), ``beta [B,T,H]``, ``g_atk, beta_atk
    [B,T,H]``, ``center [H]``, ``state [B,H,K,V]``, ``a_state [B,H,K]``.

    Returns ``(o [B,T,H,V] in dtype, S_T [B,H,K,V], A_T [B,H,K] or None)``.
    The preconditioner runs whenever ``g_atk`` is given (the reference always
    runs it, pkda.py:392-398); without it the write key is the raw key, which
    is what ``squash_x = 1`` gives exactly.  Follows pkda.py:372-410 line by
    line; ``dtype`` selects FP32 (the reference's precision) or FP64.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    q = q.to(dtype) * scale  # pkda.py:372
    k = k.to(dtype)
    v = v.to(dtype)
    decay = _expand_gate(g_log.to(dtype), K)  # pkda.py:375-377 (already activated)
    beta = beta.to(dtype)
    precond = g_atk is not None
    if precond:
        g_atk = g_atk.to(dtype)
        beta_atk = beta_atk.to(dtype)
        center_b = center.to(dtype)[None, :, None]  # pkda.py:389
        log_x = math.log(squash_x)  # pkda.py:388
    if state is None:
        state = q.new_zeros(B, H, K, V)
    else:
        state = state.to(dtype)
    if precond:
        a_state = q.new_zeros(B, H, K) if a_state is None else a_state.to(dtype)
    outputs = []
    for index in range(T):
        q_i, k_i, v_i = q[:, index], k[:, index], v[:, index]
        if precond:
            # pkda.py:392-398
            a_state = (
                g_atk[:, index].exp().unsqueeze(-1) * a_state
                + beta_atk[:, index].unsqueeze(-1) * k_i.square()
            )
            deviation = torch.log(a_state + squash_eps) - center_b
            squashed = deviation / (1 + deviation.abs())
            write_key = k_i * torch.exp(-log_x * squashed)
        else:
            write_key = k_i
        # pkda.py:399-406
        state = state * decay[:, index].exp().unsqueeze(-1)
        residual = v_i - torch.einsum("bhkv,bhk->bhv", state, k_i)
        state = state + torch.einsum(
            "bhk,bhv->bhkv", beta[:, index].unsqueeze(-1) * write_key, residual
        )
        outputs.append(torch.einsum("bhk,bhkv->bhv", q_i, state))
    if T:
        output = torch.stack(outputs, dim=1)
    else:
        output = q.new_zeros(B, 0, H, V)
    return output, state, (a_state if precond else None)


def pkda_reference(
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
    dtype: torch.dtype = torch.float32,
    out_dtype: torch.dtype | None = None,
) -> tuple[Tensor, Tensor | None, Tensor | None]:
    """The stateful chunk operator's contract (pkda.py:450-475) on the CPU.

    ``g`` is the raw gate (``use_gate_in_kernel``, activated with ``A_log`` and
    ``dt_bias`` as pkda.py:375-377) or the natural-log decay itself, ``[B,T,H]``
    or ``[B,T,H,K]``.  ``scale`` defaults to ``K ** -0.5`` (pkda.py:372,444).
    With ``cu_seqlens`` (int, ``[N+1]``) the batch must be 1 and every document
    runs from its own row of ``initial_state`` (``[N,H,K,V]``; zeros if absent).
    Output ``o`` is returned in ``out_dtype`` (default ``v.dtype``, pkda.py:407).
    """
    K = q.shape[-1]
    if scale is None:
        scale = K ** -0.5
    if use_gate_in_kernel:
        if A_log is None or dt_bias is None:
            raise ValueError("use_gate_in_kernel needs A_log and dt_bias")
        g_log = gate_log_decay(_expand_gate(g, K), A_log, dt_bias, dtype)
    else:
        g_log = g.to(dtype)
    if g_atk is not None and log_atk_scale is None:
        raise ValueError("the preconditioner needs log_atk_scale (its log-space center)")
    out_dtype = out_dtype or v.dtype

    def run(sl, s0, a0):
        o, s, a = recurrence(
            q[:, sl], k[:, sl], v[:, sl], g_log[:, sl], beta[:, sl], scale=scale,
            g_atk=None if g_atk is None else g_atk[:, sl],
            beta_atk=None if beta_atk is None else beta_atk[:, sl],
            center=log_atk_scale, squash_x=x, squash_eps=eps,
            state=s0, a_state=a0, dtype=dtype,
        )
        return o, s, a

    if cu_seqlens is None:
        o, s, a = run(slice(None), initial_state, initial_A_state)
        o = o.to(out_dtype)
        return (o, s, a) if output_final_state else (o, None, None)
    if q.shape[0] != 1:
        raise ValueError("cu_seqlens requires batch size 1")
    bounds = [int(b) for b in cu_seqlens.tolist()]
    outs, states, a_states = [], [], []
    for n in range(len(bounds) - 1):
        sl = slice(bounds[n], bounds[n + 1])
        s0 = None if initial_state is None else initial_state[n : n + 1]
        a0 = None if initial_A_state is None else initial_A_state[n : n + 1]
        o, s, a = run(sl, s0, a0)
        outs.append(o)
        states.append(s)
        a_states.append(a)
    o = torch.cat(outs, dim=1).to(out_dtype)
    if not output_final_state:
        return o, None, None
    s = torch.cat(states, dim=0)
    a = None if g_atk is None else torch.cat(a_states, dim=0)
    return o, s, a


def decode_step_reference(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    state_pool: Tensor,
    slot_idx: Tensor,
    *,
    scale: float | None = None,
    g_atk: Tensor | None = None,
    beta_atk: Tensor | None = None,
    a_pool: Tensor | None = None,
    log_atk_scale: Tensor | None = None,
    x: float = 1.0,
    eps: float = 1e-6,
    dtype: torch.dtype = torch.float32,
) -> Tensor:
    """One token per live sequence against a slot-indexed state pool.

    ``q, k, v [N,H,K]``, ``g [N,H]`` or ``[N,H,K]`` (natural-log decay),
    ``beta [N,H]``, ``state_pool [P,H,K,V]`` FP32, ``slot_idx [N]`` int.
    Updates ``state_pool`` (and ``a_pool``) in place at the indexed slots and
    returns ``o [N,H,V]`` in ``v.dtype``.  Equals a ``T = 1`` run of
    :func:`recurrence` on the gathered slots (pkda.py:390-406).
    """
    K = q.shape[-1]
    if scale is None:
        scale = K ** -0.5
    idx = slot_idx.long()
    s0 = state_pool[idx]
    a0 = None if a_pool is None else a_pool[idx]
    o, s, a = recurrence(
        q[:, None], k[:, None], v[:, None], g[:, None], beta[:, None], scale=scale,
        g_atk=None if g_atk is None else g_atk[:, None],
        beta_atk=None if beta_atk is None else beta_atk[:, None],
        center=log_atk_scale, squash_x=x, squash_eps=eps,
        state=s0, a_state=a0, dtype=dtype,
    )
    state_pool[idx] = s.to(state_pool.dtype)
    if a_pool is not None and a is not None:
        a_pool[idx] = a.to(a_pool.dtype)
    return o[:, 0].to(v.dtype)
