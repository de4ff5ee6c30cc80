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
    def make(q: Tensor, cu_seqlens: Tensor | None) -> "ChunkPlan":
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
        table = torch.empty(4 * bound + N + 1, device=q.device, dtype=torch.int32)
        with torch.cuda.device(q.device):
            status = _lib.lib().pkda_chunk_table(
                _ptr(cu), N, bound, _ptr(table), _stream(q.device)
            )
        if status != 0:
            raise RuntimeError(f"pkda_chunk_table failed ({status}): {_lib.lib().pkda_last_error().decode()}")
        return ChunkPlan(N, 0, H, D, T, bound, cu, table)

    def common(self) -> dict:
        return dict(
            num_seqs=self.num_seqs, seqlen=self.seqlen, heads=self.heads, head_dim=self.head_dim,
            cu_seqlens=_ptr(self.cu_seqlens), num_chunks=self.num_chunks, table=_ptr(self.table),
        )


def gate_forward(plan: ChunkPlan, g: Tensor, kind: int, A_log: Tensor | None, dt_bias: Tensor | None) -> Tensor:
    """Chunk-local cumulative natural-log decay, FP32, ``[N_tok, H]`` or ``[N_tok, H, K]``."""
    shape = (plan.num_tokens, plan.heads) if kind == _lib.GATE_LOG_HEAD else (plan.num_tokens, plan.heads, plan.head_dim)
    gcum = torch.empty(shape, device=g.device, dtype=torch.float32)
    args = _lib.GateArgs(
        num_seqs=plan.num_seqs, seqlen=plan.seqlen, heads=plan.heads, head_dim=plan.head_dim,
        gate_kind=kind, g_dtype=_dtype_code(g), cu_seqlens=_ptr(plan.cu_seqlens), g=_ptr(g),
        A_log=_ptr(A_log), dt_bias=_ptr(dt_bias), gcum=_ptr(gcum),
        num_chunks=plan.num_chunks, table=_ptr(plan.table),
    )
    _lib.call("pkda_gate_fwd", args, _stream(g.device))
    return gcum


@dataclass
class FwdSaved:
    w: Tensor
    u: Tensor
    aqk: Tensor
    akk: Tensor
    h: Tensor | None


def chunk_forward(
    plan: ChunkPlan, q: Tensor, k: Tensor, kw: Tensor, v: Tensor, gcum: Tensor, beta32: Tensor,
    scale: float, initial_state: Tensor | None, output_final_state: bool, save_states: bool,
) -> tuple[Tensor, Tensor | None, FwdSaved]:
    """Run the chunk forward on flat ``[N_tok, H, D]`` operands."""
    dev = q.device
    N, H, D = plan.num_seqs, plan.heads, plan.head_dim
    o = torch.empty_like(v)
    w = torch.empty_like(k)
    u = torch.empty_like(v)
    aqk = torch.empty(plan.num_tokens, H, CHUNK_SIZE, device=dev, dtype=q.dtype)
    akk = torch.empty(plan.num_tokens, H, CHUNK_SIZE, device=dev, dtype=q.dtype)
    h = torch.empty(plan.num_chunks, H, D, D, device=dev, dtype=q.dtype) if save_states else None
    S_T = torch.empty(N, H, D, D, device=dev, dtype=torch.float32) if output_final_state else None
    args = _lib.ChunkFwdArgs(
        dtype=_dtype_code(q), **plan.common(),
        q=_ptr(q), k=_ptr(k), kw=_ptr(kw), v=_ptr(v), gcum=_ptr(gcum),
        gate_per_channel=int(gcum.dim() == 3), beta=_ptr(beta32), scale=float(scale),
        initial_state=_ptr(initial_state), final_state=_ptr(S_T), o=_ptr(o),
        w=_ptr(w), u=_ptr(u), aqk=_ptr(aqk), akk=_ptr(akk), h=_ptr(h),
    )
    _lib.call("pkda_chunk_fwd", args, _stream(dev))
    return o, S_T, FwdSaved(w, u, aqk, akk, h)
