"""The stateless training/prefill PKDA operator, as a graph-friendly custom op.

Mirrors ``delta_feedback::pkda_recurrence`` and its backward op
(``delta_feedback_experiment/fla_ops.py:252-569``): same argument list and
meaning, the gate computed inside from the raw decay projection, the
preconditioner always applied, no cache state, no final state, no packing.
``PreconditionedKDA._cuda_recurrence`` calls it for dense training and prefill
(``delta_feedback_experiment/pkda.py:429-449``).

The saved list is this library's own (the caller treats it as opaque,
``pkda.py:433``): the write keys and the preconditioner's chunk checkpoints
always; the WY factors, corrected values, intra-chunk products and chunk
states as well unless ``lean``, in which case the backward rebuilds them with
the same kernels the forward ran.  The gate's chunk cumsum is one of the
retained tensors; under ``lean`` the backward relaunches the gate, as the
reference's backward always does (``fla_ops.py:423-432``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .chunk import (CHUNK_SIZE, ChunkPlan, chunk_backward, chunk_forward, gate_backward, gate_forward,
                    wants_gcum_lo)
from .pkda import _f32
from . import precond as pre

SAVED_ALWAYS = ("k_write", "a_chunk")
"""Saved by every forward: the preconditioned write keys and the
preconditioner state entering each chunk."""

SAVED_WIDE_KEY = "k_write32"
"""Saved after ``k_write`` when the activations are narrower than FP32: the
write keys in FP32, from which the backward sums the gate gradient's
in-block pairs."""

SAVED_RETAINED = ("w", "v_new", "Aqk", "T", "h", "qg", "kg", "gcum")
"""Saved as well unless ``lean``: W, the corrected values U, the intra-chunk
query-key products, the inverted WY matrix, the chunk-entry states, the
gated query and write key, and the gate's chunk-local cumulative log-decay
(FP32)."""

SAVED_GCUM_LO = "gcum_lo"
"""Saved after ``gcum`` for FP32 activations unless ``lean``: the remainder
of the gate's FP64 cumsum, from which the chunk kernels form the decay
between two tokens of a chunk (``chunk.wants_gcum_lo``)."""


def intermediate_meta(q: Tensor, v: Tensor, lean: bool) -> tuple[tuple[tuple[int, ...], torch.dtype], ...]:
    """What ``_setup_context`` saves, as (shape, dtype) pairs in save order:
    a function of the shapes of ``q`` and ``v``, their dtype and ``lean`` only,
    so the fake kernel and the real one agree without running either."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    chunks = -(-T // CHUNK_SIZE)
    act = q.dtype
    ntok = B * T
    meta = [((ntok, H, K), act)]                  # k_write
    if act != torch.float32:
        meta.append(((ntok, H, K), torch.float32))  # k_write32
    meta.append(((B * chunks, H, K), torch.float32))  # a_chunk
    if not lean:
        meta += [
            ((ntok, H, K), act),                  # w
            ((ntok, H, V), act),                  # v_new
            ((ntok, H, CHUNK_SIZE), act),         # Aqk
            ((ntok, H, CHUNK_SIZE), act),         # T
            ((B * chunks, H, K, V), act),         # h
            ((ntok, H, K), act),                  # qg
            ((ntok, H, K), act),                  # kg
            ((ntok, H, K), torch.float32),        # gcum
        ]
        if act == torch.float32:
            meta.append(((ntok, H, K), torch.float32))  # gcum_lo
    return tuple(meta)


def saved_names(q: Tensor, lean: bool) -> tuple[str, ...]:
    """Names of the saved intermediates, in the order of :func:`intermediate_meta`."""
    wide = (SAVED_WIDE_KEY,) if q.dtype != torch.float32 else ()
    retained = () if lean else SAVED_RETAINED + ((SAVED_GCUM_LO,) if q.dtype == torch.float32 else ())
    return SAVED_ALWAYS[:1] + wide + SAVED_ALWAYS[1:] + retained


def _check_saved(saved: list[Tensor], q: Tensor, v: Tensor, lean: bool) -> None:
    expected = intermediate_meta(q, v, lean)
    names = saved_names(q, lean)
    if len(saved) != len(expected):
        raise RuntimeError(f"pkda_recurrence saved {len(saved)} tensors, not {len(expected)}")
    for name, t, (shape, dtype) in zip(names, saved, expected):
        if tuple(t.shape) != shape or t.dtype != dtype or t.device != q.device or not t.is_contiguous():
            raise RuntimeError(
                f"pkda_recurrence intermediate {name} is {(tuple(t.shape), t.dtype, t.device)}, "
                f"not {(shape, dtype, q.device)}: the forward and intermediate_meta (the fake's shapes) disagree"
            )


def _check_inputs(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale) -> None:
    B, T, H, K = q.shape
    if k.shape != q.shape or v.shape[:3] != q.shape[:3] or v.shape[-1] != K:
        raise ValueError("pkda_recurrence needs q, k, v [B, T, H, D] with one D")
    if g.shape != q.shape:
        raise ValueError(f"g (raw decay) must be {tuple(q.shape)}, got {tuple(g.shape)}")
    for name, t in (("g_atk", g_atk), ("beta_atk", beta_atk), ("beta", beta)):
        if tuple(t.shape) != (B, T, H):
            raise ValueError(f"{name} must be {(B, T, H)}, got {tuple(t.shape)}")
    if A_log.numel() != H or dt_bias.numel() != H * K or log_atk_scale.numel() != H:
        raise ValueError("A_log [H], dt_bias [H*D] and log_atk_scale [H] expected")
    if not q.is_cuda:
        raise RuntimeError("pkda_recurrence needs tensors on a HIP device; there is no CPU fallback")


_GATE_STREAMS: dict[int, torch.cuda.Stream] = {}


def _gate_stream(dev: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for the per-channel
    gate, which neither reads nor writes anything of the preconditioner's:
    the two run side by side, joined before the first kernel that needs
    both (the chunk forward; the end of the backward)."""
    i = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _GATE_STREAMS.get(i)
    if s is None:
        s = _GATE_STREAMS[i] = torch.cuda.Stream(device=i)
    return s


def _forward(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale, scale, squash_x, squash_eps,
             save_all: bool):
    plan = ChunkPlan.make(q, None)
    flat = lambda t: t.contiguous().reshape(plan.num_tokens, plan.heads, *t.shape[3:])  # noqa: E731
    qf, kf, vf, gf = flat(q), flat(k), flat(v), flat(g)
    if gf.dtype not in (torch.float32, torch.bfloat16):
        gf = gf.float()
    A32, dt32 = _f32(A_log), _f32(dt_bias)
    gcum_lo = _gcum_lo(plan, qf)
    # the gate on its own stream beside the preconditioner (both read only
    # the inputs); gcum is allocated there and recorded as used by this one
    cur, side = torch.cuda.current_stream(q.device), _gate_stream(q.device)
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        gcum = gate_forward(plan, gf, _lib.GATE_RAW_CHANNEL, A32, dt32, gcum_lo=gcum_lo)
    pstate = pre.precond_forward(plan, kf, g_atk, beta_atk, log_atk_scale, squash_x, squash_eps, None,
                                 want_kw32=True)
    cur.wait_stream(side)
    gcum.record_stream(cur)
    beta32 = _f32(beta).reshape(plan.num_tokens, plan.heads)
    o, _, fs = chunk_forward(plan, qf, kf, pstate.kw, vf, gcum, beta32, scale, None, False, save_states=save_all,
                             gcum_lo=gcum_lo)
    return plan, qf, kf, vf, gf, A32, dt32, gcum, gcum_lo, pstate, beta32, o, fs


def _gcum_lo(plan: ChunkPlan, qf: Tensor) -> Tensor | None:
    """The gate's FP64 remainder buffer for FP32 activations, else None."""
    if not wants_gcum_lo(_lib.GATE_RAW_CHANNEL, qf.dtype):
        return None
    return torch.empty(plan.num_tokens, plan.heads, plan.head_dim, device=qf.device, dtype=torch.float32)


@torch.library.custom_op("pkda_mi355x::pkda_recurrence", mutates_args=(), device_types="cuda")
def pkda_recurrence(
    q: Tensor, k: Tensor, v: Tensor, g: Tensor, g_atk: Tensor, beta_atk: Tensor, beta: Tensor,
    A_log: Tensor, dt_bias: Tensor, log_atk_scale: Tensor,
    scale: float, squash_x: float, squash_eps: float, lean: bool,
) -> tuple[Tensor, list[Tensor]]:
    """Chunked PKDA forward over the gfx950 kernels: ``(o, saved)``.

    ``g`` is the raw decay projection ``[B,T,H,D]``; the log gate
    ``-exp(A_log) softplus(g + dt_bias)`` and its chunk-local cumsum are
    computed on the device.  ``o`` is in ``q.dtype``.
    """
    _check_inputs(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale)
    with torch.cuda.device(q.device):
        (plan, qf, kf, vf, gf, A32, dt32, gcum, gcum_lo, pstate, beta32, o, fs) = _forward(
            q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale, scale, squash_x, squash_eps,
            save_all=not lean)
    saved = [pstate.kw] + ([] if pstate.kw32 is None else [pstate.kw32]) + [pstate.a_chunk]
    if not lean:
        saved += [fs.w, fs.u, fs.aqk, fs.akk, fs.h, fs.qg, fs.kg, gcum]
        if gcum_lo is not None:
            saved.append(gcum_lo)
    _check_saved(saved, q, v, lean)
    return o.reshape(*q.shape[:3], v.shape[-1]).to(q.dtype), saved


@pkda_recurrence.register_fake
def _pkda_recurrence_fake(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale,
                          scale, squash_x, squash_eps, lean):
    out = torch.empty((*q.shape[:3], v.shape[-1]), device=q.device, dtype=q.dtype)
    saved = [torch.empty(shape, device=q.device, dtype=dtype) for shape, dtype in intermediate_meta(q, v, lean)]
    return out, saved


@torch.library.custom_op("pkda_mi355x::pkda_recurrence_backward", mutates_args=(), device_types="cuda")
def pkda_recurrence_backward(
    q: Tensor, k: Tensor, v: Tensor, g: Tensor, g_atk: Tensor, beta_atk: Tensor, beta: Tensor,
    A_log: Tensor, dt_bias: Tensor, log_atk_scale: Tensor, saved: list[Tensor], do: Tensor,
    scale: float, squash_x: float, squash_eps: float, autocast_dtype: torch.dtype | None, lean: bool,
) -> list[Tensor]:
    """Gradients of :func:`pkda_recurrence` for its ten tensor inputs, each in
    that input's dtype (``delta_feedback_experiment/fla_ops.py:488-499``).

    ``autocast_dtype`` is the autocast state the forward ran under (None:
    disabled); the backward runs under it, as the reference's does
    (``fla_ops.py:433-437``), whatever state the caller's ``backward()`` is
    in.  The gfx950 kernels take their dtypes from the tensors, so the
    gradients do not depend on it."""
    from .chunk import FwdSaved

    with torch.cuda.device(q.device), torch.autocast(
            "cuda", enabled=autocast_dtype is not None, dtype=autocast_dtype or torch.bfloat16):
        plan = ChunkPlan.make(q, None)
        flat = lambda t: t.contiguous().reshape(plan.num_tokens, plan.heads, *t.shape[3:])  # noqa: E731
        qf, kf, vf, gf = flat(q), flat(k), flat(v), flat(g)
        if gf.dtype not in (torch.float32, torch.bfloat16):
            gf = gf.float()
        A32, dt32 = _f32(A_log), _f32(dt_bias)
        beta32 = _f32(beta).reshape(plan.num_tokens, plan.heads)
        named = dict(zip(saved_names(q, lean), saved))
        kw, kw32, a_chunk = named["k_write"], named.get(SAVED_WIDE_KEY), named["a_chunk"]
        if lean:  # the gate and the chunk quantities again, as the forward ran them
            gcum_lo = _gcum_lo(plan, qf)
            gcum = gate_forward(plan, gf, _lib.GATE_RAW_CHANNEL, A32, dt32, gcum_lo=gcum_lo)
            _, _, fs = chunk_forward(plan, qf, kf, kw, vf, gcum, beta32, scale, None, False, save_states=True,
                                     gcum_lo=gcum_lo)
        else:
            gcum, gcum_lo = named["gcum"], named.get(SAVED_GCUM_LO)
            fs = FwdSaved(*(named[n] for n in SAVED_RETAINED[:-1]))
        dof = flat(do.to(q.dtype))
        # every gradient leaves the kernel in the input dtype; the
        # preconditioner's reverse scan reads dk, dkw that way and writes the
        # final dk
        gr = chunk_backward(plan, qf, kf, kw, vf, gcum, beta32, scale, None, fs, dof, None, False,
                            grad_dtype=qf.dtype, key_grad_dtype=qf.dtype, kw32=kw32, gcum_lo=gcum_lo)
        pstate = pre.PrecondState(kw, a_chunk, None, None)
        dk = torch.empty_like(kf)  # the preconditioner's scan writes the final dk in k's dtype
        # the gate's backward (dgcum only) beside the preconditioner's (dk, dkw)
        cur, side = torch.cuda.current_stream(q.device), _gate_stream(q.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            dg, dA_log, ddt_bias = gate_backward(plan, gf, _lib.GATE_RAW_CHANNEL, A32, dt32, gr.dgcum,
                                                 dg_dtype=gf.dtype)
        dg_atk, dbeta_atk, dcenter, _ = pre.precond_backward(
            plan, kf, g_atk, beta_atk, log_atk_scale, squash_x, squash_eps, pstate, gr.dkw, gr.dk, None, False,
            dk_final=dk)
        cur.wait_stream(side)
        for t in (dg, dA_log, ddt_bias):
            t.record_stream(cur)
    shape = tuple(q.shape)
    lead = shape[:3]
    return [
        gr.dq.reshape(shape).to(q.dtype), dk.reshape(shape).to(k.dtype), gr.dv.reshape(v.shape).to(v.dtype),
        dg.reshape(g.shape).to(g.dtype), dg_atk.reshape(lead).to(g_atk.dtype),
        dbeta_atk.reshape(lead).to(beta_atk.dtype), gr.dbeta.reshape(lead).to(beta.dtype),
        dA_log.reshape(A_log.shape).to(A_log.dtype), ddt_bias.reshape(dt_bias.shape).to(dt_bias.dtype),
        dcenter.reshape(log_atk_scale.shape).to(log_atk_scale.dtype),
    ]


@pkda_recurrence_backward.register_fake
def _pkda_recurrence_backward_fake(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale, saved, do,
                                   scale, squash_x, squash_eps, autocast_dtype, lean):
    return [torch.empty_like(t) for t in (q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale)]


def _setup_context(ctx, inputs, output) -> None:
    q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale, *scalars = inputs
    _o, saved = output
    ctx.save_for_backward(q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, log_atk_scale, *saved)
    ctx.scalars = tuple(scalars)
    # the autocast state of the forward, for the backward (fla_ops.py:546-548)
    ctx.autocast_dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
    ctx.mark_non_differentiable(*saved)
    # the saved intermediates never receive gradients: do not fill zeros for them
    ctx.set_materialize_grads(False)


def _backward(ctx, do, _dsaved):
    if do is None:
        return (None,) * 14
    tensors = ctx.saved_tensors
    inputs, saved = tensors[:10], list(tensors[10:])
    scale, squash_x, squash_eps, lean = ctx.scalars
    grads = pkda_recurrence_backward(*inputs, saved, do, scale, squash_x, squash_eps, ctx.autocast_dtype, lean)
    return (*grads, None, None, None, None)


pkda_recurrence.register_autograd(_backward, setup_context=_setup_context)
