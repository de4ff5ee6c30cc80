"""FP64 chunk-form evaluation of the PKDA recurrence -- TEST INFRASTRUCTURE ONLY.

An independent second evaluation of the same function as
:mod:`oracle.pkda_oracle`: instead of stepping token by token it applies the
chunkwise (WY / UT-transform) form the HIP kernels implement.  Inside a chunk of
``C`` tokens with entering state ``S0`` and per-channel cumulative log-decay
``G[t] = sum_{s<=t} g[s]``:

    Akk[t,s] = beta_t sum_c k[t,c] kw[s,c] exp(G[t,c]-G[s,c])      (s < t)
    T        = (I + Akk)^-1
    W        = T diag(beta) (exp(G) * k),   Uu = T diag(beta) v
    U        = Uu - W S0
    Aqk[t,s] = sum_c qs[t,c] kw[s,c] exp(G[t,c]-G[s,c])              (s <= t)
    O        = (exp(G) * qs) S0 + Aqk U
    S_C      = diag(exp(G[C-1])) S0 + (exp(G[C-1]-G) * kw)^T U

(``qs`` = scaled query, ``kw`` = preconditioned write key.)  This is derived
from the recurrence of ``delta_feedback_experiment/pkda.py:390-406``; agreement
with the literal loop to ~1e-12 in FP64 is what ``tests/test_oracle.py`` uses
to pin both the algebra the kernels rely on and the loop itself.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def precond_write_key(
    k: Tensor, g_atk: Tensor, beta_atk: Tensor, center: Tensor, x: float, eps: float,
    a0: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Diagonal preconditioner scan (pkda.py:392-398), FP64, ``[B,T,H,K]``."""
    B, T, H, K = k.shape
    k = k.double()
    a = k.new_zeros(B, H, K) if a0 is None else a0.double().clone()
    out = torch.empty_like(k)
    log_x = math.log(x)
    for t in range(T):
        a = g_atk[:, t].double().exp()[..., None] * a + beta_atk[:, t].double()[..., None] * k[:, t] ** 2
        r = torch.log(a + eps) - center.double()[None, :, None]
        out[:, t] = k[:, t] * torch.exp(-log_x * r / (1 + r.abs()))
    return out, a


def chunk_forward(
    q: Tensor, k: Tensor, kw: Tensor, v: Tensor, g_log: Tensor, beta: Tensor,
    scale: float, state: Tensor | None = None, chunk: int = 64,
) -> tuple[Tensor, Tensor]:
    """Chunk-form forward for equal-length rows; returns ``(o, S_T)`` in FP64.

    ``g_log`` is the natural-log decay ``[B,T,H]`` or ``[B,T,H,K]``.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    q, k, kw, v = (t.double() for t in (q, k, kw, v))
    g = g_log.double()
    if g.dim() == 3:
        g = g[..., None].expand(B, T, H, K)
    beta = beta.double()
    S = q.new_zeros(B, H, K, V) if state is None else state.double().clone()
    o = q.new_empty(B, T, H, V)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        n = c1 - c0
        # [B,H,n,*] views of the chunk
        qc = q[:, c0:c1].transpose(1, 2) * scale
        kc = k[:, c0:c1].transpose(1, 2)
        kwc = kw[:, c0:c1].transpose(1, 2)
        vc = v[:, c0:c1].transpose(1, 2)
        bc = beta[:, c0:c1].transpose(1, 2)  # [B,H,n]
        G = g[:, c0:c1].transpose(1, 2).cumsum(2)  # [B,H,n,K]
        # exact pairwise decay exp(G[t]-G[s]) for s <= t, zero above
        diff = G[:, :, :, None, :] - G[:, :, None, :, :]  # [B,H,t,s,K]
        lower = torch.tril(torch.ones(n, n, dtype=torch.bool))
        E = torch.where(lower[None, None, :, :, None], diff, torch.full_like(diff, -math.inf)).exp()
        strict = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
        Akk = torch.einsum("bhtc,bhsc,bhtsc->bhts", kc, kwc, E) * bc[..., None]
        Akk = Akk * strict
        Aqk = torch.einsum("bhtc,bhsc,bhtsc->bhts", qc, kwc, E) * lower
        eye = torch.eye(n, dtype=torch.float64)
        Tm = torch.linalg.solve_triangular(eye + Akk, eye.expand(B, H, n, n), upper=False, unitriangular=True)
        eG = G.exp()
        W = Tm @ (bc[..., None] * eG * kc)
        Uu = Tm @ (bc[..., None] * vc)
        U = Uu - W @ S
        oc = (eG * qc) @ S + Aqk @ U
        o[:, c0:c1] = oc.transpose(1, 2)
        GC = G[:, :, -1:, :]  # [B,H,1,K]
        S = GC.transpose(2, 3).exp() * S + ((GC - G).exp() * kwc).transpose(2, 3) @ U
    return o, S
