"""Chunked PKDA: host orchestration of the gate, preconditioner and chunk kernels.

This is the MI355X replacement for FLA's ``chunk_precond_kda`` family as the
reference drives it (``delta_feedback_experiment/fla_ops.py:290-339`` forward,
``:423-487`` backward, ``delta_feedback_experiment/pkda.py:450-475``).  The
launch sequence per forward is: gate cumsum -> (preconditioner scan) -> chunk
forward; per backward: chunk backward -> (preconditioner reverse scan) ->
gate backward.  Every buffer is allocated here, by PyTorch's caching
allocator, and handed to the library, which only enqueues kernels on the
current stream -- so a forward+backward can be captured in one HIP graph.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .pkda import _dtype_code, _f32, _ptr, _stream

CHUNK_SIZE = 64


@dataclass
class ChunkPlan:
    """Document and chunk geometry of one call."""

    num_seqs: int
    seqlen: int          # equal rows; 0 for packed documents
    heads: int
    head_dim: int
    num_tokens: int
    num_chunks: int      # exact (equal rows) or the launch bound (packed)
    cu_seqlens: Tensor | None
    table: Tensor | None

    @staticmethod
    def make(q: Tensor, cu_seqlens: Tensor | None, check: bool = False) -> "ChunkPlan":
        """The geometry of ``q [B, T, H, D]``; with ``cu_seqlens`` the chunk
        table is built on the device.  A malformed ``cu_seqlens`` is clamped
        there (every kernel reads the table's sanitised copy, so no access
        leaves the tensors) and flagged; ``check`` reads the flag back
        (synchronising) and raises."""
        B, T, H, D = q.shape
        if cu_seqlens is None:
            nt = -(-T // CHUNK_SIZE)
            return ChunkPlan(B, T, H, D, B * T, B * nt, None, None)
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1")
        cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
        N = cu.numel() - 1
        if N < 0:
            raise ValueError("cu_seqlens needs at least one element")
        bound = -(-T // CHUNK_SIZE) + N
        table = torch.empty(4 * bound + 3 * N + 3, device=q.device, dtype=torch.int32)
        with torch.cuda.device(q.device):
            status = _lib.lib().pkda_chunk_table(
                _ptr(cu), N, T, bound, _ptr(table), _stream(q.device)
            )
        if status != 0:
            raise RuntimeError(f"pkda_chunk_table failed ({status}): {_lib.lib().pkda_last_error().decode()}")
        plan = ChunkPlan(N, 0, H, D, T, bound, cu, table)
        if check and not plan.cu_seqlens_ok():
            raise ValueError(f"cu_seqlens must rise from 0 to the packed length {T} without decreasing")
        return plan

    @property
    def sanitized_cu(self) -> Tensor | None:
        """The table's copy of ``cu_seqlens`` that the kernels read: the running
        maximum clamped to ``[0, N_tok]`` (equal to the input when it is well
        formed), int32 ``[N + 1]`` on the device."""
        if self.table is None:
            return None
        off = 4 * self.num_chunks + 2 * self.num_seqs + 1
        return self.table[off:off + self.num_seqs + 1]

    def cu_seqlens_ok(self) -> bool:
        """Whether ``cu_seqlens`` was well formed (reads the table's flag
        back: synchronises)."""
        return self.table is None or int(self.table[-1].item()) == 0

    def common(self) -> dict:
        return dict(
            num_seqs=self.num_seqs, seqlen=self.seqlen, heads=self.heads, head_dim=self.head_dim,
            cu_seqlens=_ptr(self.cu_seqlens), num_chunks=self.num_chunks, table=_ptr(self.table),
        )


def validate_cu_seqlens(cu_seqlens: Tensor, num_tokens: int) -> None:
    """Raise ``ValueError`` unless ``cu_seqlens`` rises from 0 to the packed
    length ``num_tokens`` without decreasing (reads it back: synchronises).
    Without this check a malformed array is clamped on the device and the
    tokens it leaves outside every document keep unwritten outputs."""
    cu = cu_seqlens.detach().to("cpu", torch.int64).reshape(-1)
    if cu.numel() < 1 or int(cu[0]) != 0 or int(cu[-1]) != num_tokens or bool((cu[1:] < cu[:-1]).any()):
        raise ValueError(f"cu_seqlens must rise from 0 to the packed length {num_tokens} without decreasing, "
                         f"got {cu.tolist() if cu.numel() <= 16 else '[...]'}")


def wants_gcum_lo(kind: int, dtype: torch.dtype) -> bool:
    """Whether the chunk kernels take the gate's FP64 remainder: FP32
    activations with a per-channel gate.  There the decay between two tokens
    of a chunk is the difference of two cumsums that reach a few hundred
    under strong gates; from FP32 cumsums alone that difference carries their
    rounding (~1e-5 relative to it), which the gate gradient's sums over a
    head amplify past the FP32 tolerance."""
    return kind != _lib.GATE_LOG_HEAD and dtype == torch.float32


def gate_forward(plan: ChunkPlan, g: Tensor, kind: int, A_log: Tensor | None, dt_bias: Tensor | None,
                 up_weight: Tensor | None = None, gcum_lo: Tensor | None = None) -> Tensor:
    """Chunk-local cumulative natural-log decay, FP32, ``[N_tok, H]`` or ``[N_tok, H, K]``.

    The low-rank form takes ``g`` as the decay hidden rows ``[N_tok, R]``
    (unit column stride, any row stride) and ``up_weight [H*K, R]``.  With
    ``gcum_lo`` (per-channel forms, FP32 of gcum's shape) the cumsum is formed
    in FP64 and ``gcum_lo`` receives its remainder past the FP32 result."""
    shape = (plan.num_tokens, plan.heads) if kind == _lib.GATE_LOG_HEAD else (plan.num_tokens, plan.heads, plan.head_dim)
    gcum = torch.empty(shape, device=g.device, dtype=torch.float32)
    if gcum_lo is not None and (tuple(gcum_lo.shape) != shape or gcum_lo.dtype != torch.float32
                                or not gcum_lo.is_contiguous()):
        raise ValueError(f"gcum_lo must be a contiguous float32 tensor of shape {shape}")
    args = _lib.GateArgs(
        num_seqs=plan.num_seqs, seqlen=plan.seqlen, heads=plan.heads, head_dim=plan.head_dim,
        gate_kind=kind, g_dtype=_dtype_code(g), cu_seqlens=_ptr(plan.cu_seqlens), g=_ptr(g),
        A_log=_ptr(A_log), dt_bias=_ptr(dt_bias), gcum=_ptr(gcum),
        num_chunks=plan.num_chunks, table=_ptr(plan.table), gcum_lo=_ptr(gcum_lo),
    )
    if kind == _lib.GATE_LOW_RANK:
        args.up_weight, args.rank, args.g_stride = _ptr(up_weight), g.shape[-1], g.stride(0)
    _lib.call("pkda_gate_fwd", args, _stream(g.device))
    return gcum


def low_rank_rows(hidden: Tensor, num_tokens: int) -> Tensor:
    """The decay hidden ``[..., R]`` as ``[N_tok, R]`` rows the gate kernels
    read with 16-byte loads: a view when its rows are evenly strided and
    aligned (the reference's slice of the packed control projection), else a
    contiguous copy."""
    R = hidden.shape[-1]
    rows = hidden.reshape(num_tokens, R)
    vec = 16 // hidden.element_size()
    if rows.stride(1) != 1 or rows.stride(0) % vec or rows.data_ptr() % 16:
        rows = rows.contiguous()
    return rows


@dataclass
class FwdSaved:
    w: Tensor | None   # None for BF16 with a per-head gate (never stored)
    u: Tensor
    aqk: Tensor
    akk: Tensor
    h: Tensor | None
    qg: Tensor | None = None   # per-channel gates: scale e^G q
    kg: Tensor | None = None   # per-channel gates: e^{G_last - G} kw
    tri_packed: bool = False   # aqk, akk as each chunk's ten lower 16 x 16 blocks (:func:`tri_packed`)


def tri_packed(q: Tensor, k: Tensor, kw: Tensor, gcum: Tensor) -> bool:
    """Whether Aqk and T are stored packed -- only the ten 16 x 16 blocks on
    and below each chunk's diagonal, ``[num_chunks, H, 10, 256]`` -- which
    the kernels do for BF16 with a per-head gate and no separate write key
    (3/8 fewer bytes to write and to read back twice)."""
    return q.dtype == torch.bfloat16 and gcum.dim() == 2 and kw.data_ptr() == k.data_ptr()


def chunk_forward(
    plan: ChunkPlan, q: Tensor, k: Tensor, kw: Tensor, v: Tensor, gcum: Tensor, beta32: Tensor,
    scale: float, initial_state: Tensor | None, output_final_state: bool, save_states: bool,
    *, slot_idx: Tensor | None = None, final_state: Tensor | None = None, out: Tensor | None = None,
    gcum_lo: Tensor | None = None, pack_triangular: bool | None = None,
) -> tuple[Tensor, Tensor | None, FwdSaved]:
    """Run the chunk forward on flat ``[N_tok, H, D]`` operands.

    With ``slot_idx`` (int32 ``[N]``) the states are rows of a pool:
    ``initial_state`` (or zero when ``None``) and ``final_state`` are
    ``[P, H, D, D]`` and document ``n`` uses row ``slot_idx[n]`` of each.
    ``gcum_lo``: the gate's FP64 remainder (:func:`wants_gcum_lo`).
    ``pack_triangular``: None stores Aqk and T packed where :func:`tri_packed`
    allows it; False keeps them ``[N_tok, H, 64]`` (the same values)."""
    dev = q.device
    N, H, D = plan.num_seqs, plan.heads, plan.head_dim
    o = torch.empty_like(v) if out is None else out
    per_channel = gcum.dim() == 3
    # BF16 with a per-head gate: the state passes form W S and W^T dU from T and k
    w = None if (q.dtype == torch.bfloat16 and not per_channel) else torch.empty_like(k)
    u = torch.empty_like(v)
    tri = tri_packed(q, k, kw, gcum) if pack_triangular is None else bool(pack_triangular)
    if tri and not tri_packed(q, k, kw, gcum):
        raise ValueError("Aqk and T are stored packed only for BF16, a per-head gate and kw is k")
    tshape = (plan.num_chunks, H, 10, 256) if tri else (plan.num_tokens, H, CHUNK_SIZE)
    aqk = torch.empty(tshape, device=dev, dtype=q.dtype)
    akk = torch.empty(tshape, device=dev, dtype=q.dtype)
    h = torch.empty(plan.num_chunks, H, D, D, device=dev, dtype=q.dtype) if save_states else None
    if slot_idx is not None:
        S_T = final_state
    else:
        S_T = torch.empty(N, H, D, D, device=dev, dtype=torch.float32) if output_final_state else None
    qg = torch.empty_like(q) if per_channel else None
    kg = torch.empty_like(k) if per_channel else None
    args = _lib.ChunkFwdArgs(
        dtype=_dtype_code(q), **plan.common(),
        q=_ptr(q), k=_ptr(k), kw=_ptr(kw), v=_ptr(v), gcum=_ptr(gcum),
        gate_per_channel=int(per_channel), beta=_ptr(beta32), scale=float(scale),
        initial_state=_ptr(initial_state), final_state=_ptr(S_T), o=_ptr(o),
        w=_ptr(w), u=_ptr(u), aqk=_ptr(aqk), akk=_ptr(akk), h=_ptr(h), qg=_ptr(qg), kg=_ptr(kg),
        slot_idx=_ptr(slot_idx), pool_size=0 if S_T is None else S_T.shape[0], gcum_lo=_ptr(gcum_lo),
        tri_packed=int(tri),
    )
    _lib.call("pkda_chunk_fwd", args, _stream(dev))
    return o, S_T, FwdSaved(w, u, aqk, akk, h, qg, kg, tri)


@dataclass
class BwdGrads:
    dq: Tensor
    dk: Tensor
    dkw: Tensor | None
    dv: Tensor
    dbeta: Tensor
    dgcum: Tensor
    dh0: Tensor | None


def chunk_backward(
    plan: ChunkPlan, q: Tensor, k: Tensor, kw: Tensor, v: Tensor, gcum: Tensor, beta32: Tensor, scale: float,
    initial_state: Tensor | None, saved: FwdSaved, do: Tensor, dht: Tensor | None, want_dh0: bool,
    grad_dtype: torch.dtype = torch.float32, key_grad_dtype: torch.dtype | None = None,
    kw32: Tensor | None = None, gcum_lo: Tensor | None = None,
) -> BwdGrads:
    """Chunk backward on flat operands.  ``dq, dv`` come in ``grad_dtype``
    (FP32, or ``q.dtype``: the FP32 value rounded once in the kernel), ``dk,
    dkw`` in ``key_grad_dtype`` (default ``grad_dtype``; FP32 with a
    ``q.dtype`` ``grad_dtype`` for a caller that adds the preconditioner's
    terms into them); the other gradients are FP32.  ``kw32``: the write keys
    in FP32 (per-channel gates with a BF16 write key), which the in-block
    pair sums of the gate gradient then read.  ``gcum_lo``: the gate's FP64
    remainder, as the forward took it."""
    dev = q.device
    N, H, D = plan.num_seqs, plan.heads, plan.head_dim
    ntok = plan.num_tokens
    f32 = dict(device=dev, dtype=torch.float32)
    if grad_dtype not in (torch.float32, q.dtype):
        raise ValueError(f"grad_dtype must be float32 or {q.dtype}, got {grad_dtype}")
    if key_grad_dtype is None:
        key_grad_dtype = grad_dtype
    if key_grad_dtype not in (grad_dtype, torch.float32):
        raise ValueError(f"key_grad_dtype must be {grad_dtype} or float32, got {key_grad_dtype}")
    gd = dict(device=dev, dtype=grad_dtype)
    kd = dict(device=dev, dtype=key_grad_dtype)
    kw_is_k = kw.data_ptr() == k.data_ptr()
    dq = torch.empty(ntok, H, D, **gd)
    dk = torch.empty(ntok, H, D, **kd)
    dkw = None if kw_is_k else torch.empty(ntok, H, D, **kd)
    dv = torch.empty(ntok, H, D, **gd)
    dbeta = torch.empty(ntok, H, **f32)
    dgcum = torch.empty_like(gcum)
    dh0 = torch.empty(N, H, D, D, **f32) if want_dh0 else None
    dh = torch.empty(plan.num_chunks, H, D, D, device=dev, dtype=q.dtype)
    du = torch.empty(ntok, H, D, device=dev, dtype=q.dtype)
    args = _lib.ChunkBwdArgs(
        dtype=_dtype_code(q), **plan.common(),
        q=_ptr(q), k=_ptr(k), kw=_ptr(kw), v=_ptr(v), gcum=_ptr(gcum),
        gate_per_channel=int(gcum.dim() == 3), beta=_ptr(beta32), scale=float(scale),
        initial_state=_ptr(initial_state),
        w=_ptr(saved.w), u=_ptr(saved.u), aqk=_ptr(saved.aqk), akk=_ptr(saved.akk), h=_ptr(saved.h),
        do=_ptr(do), dht=_ptr(dht), dh=_ptr(dh), du=_ptr(du),
        dq=_ptr(dq), dk=_ptr(dk), dkw=_ptr(dkw), dv=_ptr(dv), dbeta=_ptr(dbeta), dgcum=_ptr(dgcum),
        dh0=_ptr(dh0), qg=_ptr(saved.qg), kg=_ptr(saved.kg),
        grad_dtype=_lib.PKDA_F32 if grad_dtype == torch.float32 else _dtype_code(q),
        key_grad_dtype=_lib.PKDA_F32 if key_grad_dtype == torch.float32 else _dtype_code(q),
        kw32=_ptr(kw32), gcum_lo=_ptr(gcum_lo), tri_packed=int(saved.tri_packed),
    )
    if kw32 is not None and (kw32.dtype != torch.float32 or kw32.shape != kw.shape or not kw32.is_contiguous()):
        raise ValueError("kw32 must be a contiguous float32 tensor of kw's shape")
    _lib.call("pkda_chunk_bwd", args, _stream(dev))
    return BwdGrads(dq, dk, dkw, dv, dbeta, dgcum, dh0)


def gate_backward(
    plan: ChunkPlan, g: Tensor, kind: int, A_log: Tensor | None, dt_bias: Tensor | None, dgcum: Tensor,
    up_weight: Tensor | None = None, dg_dtype: torch.dtype = torch.float32,
) -> tuple[Tensor, Tensor | None, Tensor | None]:
    """``dg`` (``dg_dtype``: FP32, or ``g.dtype`` for the per-channel forms;
    shape of ``g``) and, for the raw gate, ``dA_log``, ``ddt_bias``.

    The low-rank form returns the raw gate's gradient ``[N_tok, H, K]`` as
    ``dg``; the hidden rows' and the weight's gradients are two GEMMs of it
    (:func:`low_rank_grads`)."""
    dev = dgcum.device
    dg = torch.empty(dgcum.shape, device=dev, dtype=dg_dtype)
    raw = kind in (_lib.GATE_RAW_CHANNEL, _lib.GATE_LOW_RANK)
    dA_part = ddt_part = dA_log = ddt_bias = None
    if raw:
        H, D = plan.heads, plan.head_dim
        dA_part = torch.empty(plan.num_chunks, H, device=dev, dtype=torch.float32)
        ddt_part = torch.empty(plan.num_chunks, H, D, device=dev, dtype=torch.float32)
        dA_log = torch.empty(H, device=dev, dtype=torch.float32)
        ddt_bias = torch.empty(H * D, device=dev, dtype=torch.float32)
    args = _lib.GateArgs(
        num_seqs=plan.num_seqs, seqlen=plan.seqlen, heads=plan.heads, head_dim=plan.head_dim,
        gate_kind=kind, g_dtype=_dtype_code(g), cu_seqlens=_ptr(plan.cu_seqlens), g=_ptr(g),
        A_log=_ptr(A_log), dt_bias=_ptr(dt_bias), dgcum=_ptr(dgcum), dg=_ptr(dg),
        dA_log_part=_ptr(dA_part), ddt_bias_part=_ptr(ddt_part), dA_log=_ptr(dA_log), ddt_bias=_ptr(ddt_bias),
        num_chunks=plan.num_chunks, table=_ptr(plan.table),
        dg_dtype=_lib.PKDA_F32 if dg_dtype == torch.float32 else _dtype_code(g),
    )
    if kind == _lib.GATE_LOW_RANK:
        args.up_weight, args.rank, args.g_stride = _ptr(up_weight), g.shape[-1], g.stride(0)
    _lib.call("pkda_gate_bwd", args, _stream(dev))
    return dg, dA_log, ddt_bias


def low_rank_grads(draw: Tensor, hidden_rows: Tensor, up_weight: Tensor) -> tuple[Tensor, Tensor]:
    """Gradients of ``raw = hidden up_weight^T`` from the raw gate's gradient
    ``draw [N_tok, H, K]`` (FP32): ``(d hidden [N_tok, R], d up_weight [H*K, R])``,
    FP32 library GEMMs (the backward of the reference's ``F.linear``,
    delta_feedback_experiment/pkda.py:334-339)."""
    d2 = draw.reshape(draw.shape[0], -1)
    with torch.autocast("cuda", enabled=False):  # FP32 whatever autocast state the backward runs under
        return d2 @ up_weight.float(), d2.t() @ hidden_rows.float()


def _flat(t: Tensor, plan: ChunkPlan) -> Tensor:
    return t.reshape(plan.num_tokens, plan.heads, *t.shape[3:]) if t.dim() >= 3 else t


class _ChunkPKDA(torch.autograd.Function):
    """Differentiable chunked PKDA over the gfx950 kernels.

    Saving: ``lean`` keeps only the inputs and rebuilds the chunk quantities
    (WY factors, chunk states) with a second forward inside the backward;
    otherwise they are kept from the forward.  Either way the gradients are
    those of the same kernels on the same inputs.
    """

    # the backward runs under the autocast state of the forward, as FLA's
    # custom_fwd / custom_bwd pair does for chunk_precond_kda
    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, q, k, v, g, beta, g_atk, beta_atk, A_log, dt_bias, log_atk_scale,
                initial_state, initial_A_state, cu_seqlens, decay_up, opts):
        from .pkda import gate_form
        from . import precond as pre

        use_gate, scale, output_final_state, x, eps, lean = opts
        plan = ChunkPlan.make(q, cu_seqlens)
        if decay_up is not None:  # g is the decay hidden; the expansion runs in the gate kernel
            kind, g_used = _lib.GATE_LOW_RANK, low_rank_rows(g, plan.num_tokens)
            decay_up = decay_up.to(g_used.dtype).contiguous()
        else:
            kind, g_used = gate_form(g, q.shape[:-1], q.shape[-1], use_gate, A_log, dt_bias)
            g_used = g_used.contiguous()
            if g_used.dtype not in (torch.float32, torch.bfloat16):
                g_used = g_used.float()
        A_log32, dt32 = _f32(A_log), _f32(dt_bias)
        qf, kf, vf = (_flat(t.contiguous(), plan) for t in (q, k, v))
        beta32 = _f32(beta).reshape(plan.num_tokens, plan.heads)
        s0 = _f32(initial_state)
        gcum_lo = None
        if wants_gcum_lo(kind, q.dtype):
            shp = (plan.num_tokens, plan.heads, plan.head_dim)
            gcum_lo = torch.empty(shp, device=q.device, dtype=torch.float32)
        gcum = gate_forward(plan, _flat(g_used, plan), kind, A_log32, dt32, decay_up, gcum_lo=gcum_lo)
        precond = g_atk is not None
        needs_grad = any(ctx.needs_input_grad)
        if precond:
            pstate = pre.precond_forward(plan, kf, g_atk, beta_atk, log_atk_scale, x, eps, initial_A_state,
                                         want_kw32=needs_grad and gcum.dim() == 3)
            kwf, A_T = pstate.kw, pstate.final_A
        else:
            pstate, kwf, A_T = None, kf, None
        o, S_T, saved = chunk_forward(plan, qf, kf, kwf, vf, gcum, beta32, scale, s0,
                                      output_final_state, save_states=needs_grad and not lean, gcum_lo=gcum_lo)
        if needs_grad:
            ctx.plan, ctx.kind, ctx.scale, ctx.lean, ctx.x, ctx.eps = plan, kind, scale, lean, x, eps
            ctx.per_head_raw = use_gate and decay_up is None and g.dim() == q.dim() - 1
            ctx.g_shape = tuple(g.shape)
            ctx.precond = precond
            ctx.up_dtype = None if decay_up is None else decay_up.dtype
            ctx.dtypes = tuple(None if t is None else t.dtype for t in (q, k, v, g, beta, g_atk, beta_atk,
                                                                          A_log, dt_bias, log_atk_scale,
                                                                          initial_state, initial_A_state))
            # every tensor the backward reads goes through save_for_backward
            # (none through ctx attributes: A_T is an output, and keeping the
            # scan state on ctx would tie output -> grad_fn -> ctx -> output)
            fwd = (None,) * 7 if lean else (saved.w, saved.u, saved.aqk, saved.akk, saved.h, saved.qg, saved.kg)
            ctx.tri_packed = saved.tri_packed
            ctx.save_for_backward(qf, kf, kwf, vf, gcum, beta32, s0, g_used, A_log32, dt32,
                                  None if g_atk is None else _f32(g_atk),
                                  None if beta_atk is None else _f32(beta_atk),
                                  None if log_atk_scale is None else _f32(log_atk_scale),
                                  decay_up,
                                  None if pstate is None else pstate.a_chunk,
                                  None if pstate is None else pstate.kw32,
                                  gcum_lo, *fwd)
        o = o.reshape(v.shape)
        return o, S_T, A_T

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, do, dS_T, dA_T):
        from . import precond as pre

        (qf, kf, kwf, vf, gcum, beta32, s0, g_used, A_log32, dt32,
         g_atk32, beta_atk32, center32, decay_up, a_chunk, kw32, gcum_lo, *fwd) = ctx.saved_tensors
        plan = ctx.plan
        if ctx.lean:  # rebuild the chunk quantities
            _, _, saved = chunk_forward(plan, qf, kf, kwf, vf, gcum, beta32, ctx.scale, s0, False, True,
                                        gcum_lo=gcum_lo)
        else:
            saved = FwdSaved(*fwd, tri_packed=ctx.tri_packed)
        pstate = pre.PrecondState(kwf, a_chunk, None, None, kw32) if ctx.precond else None
        dof = _flat(do.to(qf.dtype).contiguous(), plan)
        dht = None if dS_T is None else dS_T.float().contiguous()
        want_dh0 = ctx.needs_input_grad[10]
        # nothing consumes dq, dv after the kernel but the cast to the input
        # dtype, which the kernel then does; dk and dkw too (the
        # preconditioner's reverse scan reads them in that dtype and writes
        # the final dk)
        direct = ctx.dtypes[0] == qf.dtype and ctx.dtypes[2] == qf.dtype
        key_direct = direct and ctx.dtypes[1] == qf.dtype
        gr = chunk_backward(plan, qf, kf, kwf, vf, gcum, beta32, ctx.scale, s0, saved, dof, dht, want_dh0,
                            grad_dtype=qf.dtype if direct else torch.float32,
                            key_grad_dtype=qf.dtype if key_direct else torch.float32, kw32=kw32, gcum_lo=gcum_lo)
        dk = gr.dk
        dg_atk = dbeta_atk = dcenter = dA0 = None
        if pstate is not None:
            dk_final = torch.empty_like(kf) if dk.dtype != torch.float32 else None
            pg = pre.precond_backward(plan, kf, g_atk32, beta_atk32, center32, ctx.x, ctx.eps, pstate,
                                      gr.dkw, dk, None if dA_T is None else dA_T.float().contiguous(),
                                      want_dA0=ctx.needs_input_grad[11], dk_final=dk_final)
            dg_atk, dbeta_atk, dcenter, dA0 = pg
            if dk_final is not None:
                dk = dk_final
        dg, dA_log, ddt_bias = gate_backward(plan, _flat(g_used, plan), ctx.kind, A_log32, dt32, gr.dgcum,
                                             decay_up)
        shape = tuple(do.shape)
        dt = ctx.dtypes

        def cast(x, i, shp=None):
            if x is None or dt[i] is None or not ctx.needs_input_grad[i]:
                return None
            x = x if shp is None else x.reshape(shp)
            return x.to(dt[i])

        d_up = None
        if ctx.kind == _lib.GATE_LOW_RANK:
            dg, d_up = low_rank_grads(dg, g_used, decay_up)
            dg = dg.reshape(ctx.g_shape)
            d_up = d_up.to(ctx.up_dtype) if ctx.needs_input_grad[13] else None
        else:
            dg = dg.reshape(*shape[:-1], *dg.shape[2:])
            if ctx.per_head_raw:
                dg = dg.sum(-1)
        return (
            cast(gr.dq, 0, shape), cast(dk, 1, shape), cast(gr.dv, 2, shape), cast(dg, 3),
            cast(gr.dbeta, 4, shape[:-1]),
            cast(dg_atk, 5, shape[:-1]), cast(dbeta_atk, 6, shape[:-1]),
            cast(dA_log, 7), cast(ddt_bias, 8), cast(dcenter, 9),
            cast(gr.dh0, 10), cast(dA0, 11), None, d_up, None,
        )


def chunk_pkda(
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
    lean: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    decay_up: Tensor | None = None,
    check_cu_seqlens: bool = False,
    **_ignored,
) -> tuple[Tensor, Tensor | None, Tensor | None]:
    """Stateful, differentiable chunked PKDA: ``(o, S_T, A_T)``.

    The call surface of FLA's ``chunk_precond_kda`` as
    ``PreconditionedKDA._cuda_recurrence`` uses it (pkda.py:450-475).  ``g`` is
    the raw gate (``use_gate_in_kernel``, with ``A_log``/``dt_bias``) or the
    natural-log decay, per head ``[B,T,H]`` or per channel ``[B,T,H,K]``.
    The preconditioner (``g_atk``, ``beta_atk``, ``log_atk_scale``, ``x``,
    ``eps``) runs when ``g_atk`` is given.  ``scale`` defaults to ``K**-0.5``.
    Gradients flow to every tensor input including ``initial_state`` and
    ``initial_A_state``.

    With ``decay_up`` (the module's ``decay_up.weight [H*K, K]``,
    pkda.py:168) ``g`` is the decay hidden ``[B, T, K]`` -- e.g. the first
    slice of the packed control projection -- and the raw gate
    ``g @ decay_up^T`` (pkda.py:334-339) is formed inside the gate kernel on
    MFMA instead of being materialised; ``use_gate_in_kernel`` must be set.
    ``decay_up`` receives its gradient too.

    ``check_cu_seqlens`` verifies on the host (synchronising) that
    ``cu_seqlens`` rises from 0 to the packed length; without it a malformed
    array is clamped on the device, and tokens outside every document keep
    unwritten outputs and gradients.
    """
    from .pkda import _check_common, _require_cuda

    if use_qk_l2norm_in_kernel:
        raise ValueError("q and k arrive L2-normalised (pkda.py:464-465); in-kernel norm is not provided")
    _check_common(q, k, v, beta)
    _require_cuda(q, k, v, g, beta, g_atk, beta_atk, initial_state, initial_A_state, cu_seqlens, A_log, dt_bias,
                  log_atk_scale)
    if g_atk is not None and (beta_atk is None or log_atk_scale is None):
        raise ValueError("the preconditioner needs g_atk, beta_atk and log_atk_scale")
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    if decay_up is not None:
        _require_cuda(decay_up)
        H = q.shape[2]
        if not use_gate_in_kernel or A_log is None or dt_bias is None:
            raise ValueError("decay_up forms the raw gate: it needs use_gate_in_kernel with A_log and dt_bias")
        if tuple(decay_up.shape) != (H * D, D) or tuple(g.shape) != (*q.shape[:2], D):
            raise ValueError(f"decay_up [{H * D}, {D}] with g the decay hidden {(*q.shape[:2], D)} expected, got "
                             f"{tuple(decay_up.shape)} and {tuple(g.shape)}")
    if check_cu_seqlens and cu_seqlens is not None:
        validate_cu_seqlens(cu_seqlens, q.shape[1])
    N = q.shape[0] if cu_seqlens is None else cu_seqlens.numel() - 1
    if initial_state is not None and tuple(initial_state.shape) != (N, q.shape[2], D, D):
        raise ValueError(f"initial_state must be {(N, q.shape[2], D, D)}")
    opts = (use_gate_in_kernel, float(scale), output_final_state, float(x), float(eps), lean)
    with torch.cuda.device(q.device):
        o, S_T, A_T = _ChunkPKDA.apply(q, k, v, g, beta, g_atk, beta_atk, A_log, dt_bias, log_atk_scale,
                                      initial_state, initial_A_state, cu_seqlens, decay_up, opts)
    if not output_final_state:
        return o, None, None
    return o, S_T, A_T
