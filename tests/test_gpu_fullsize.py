"""Chunked PKDA at the benchmark's full sizes, through properties that do not
need the CPU oracle to run at that size.

* Forward (c2 B8 T4096 H16, c3 packed 32,768 tokens, c5 B2 T16384 H32 with
  S0 != 0 and strong decays): the BF16 chunked path against the token-recurrent
  kernel run in FP32 on the same BF16-rounded inputs -- an independent
  algorithm (one token at a time, FP32 state and FP32 I/O) whose agreement
  with the CPU oracle is pinned at small sizes in test_gpu_recurrent.py.
  Bar: relative L2 <= 2e-2 (BF16 inputs against an FP32 reference).
* Gradients at the full c2 length: one batch row and four heads of the full
  B8 T4096 H16 step against the CPU oracle's FP32 autograd on the same
  BF16-rounded values (all 4,096 tokens; the rows and heads of the recurrence
  are independent, so the slice's gradients are the full step's).
* Exact structure at full size: gradients of the other rows and heads are
  bitwise unchanged when dO changes in one row and head (deterministic
  kernels, no cross-row or cross-head leakage).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from conftest import rel_l2
from oracle import pkda_oracle as oracle

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _l2norm(t):
    f = t.float()
    return f * torch.rsqrt(f.square().sum(-1, keepdim=True) + 1e-6)


def make_inputs(dev, B, T, H, D, seed, strong=False):
    gen = torch.Generator(device=dev).manual_seed(seed)

    def randn(*s):
        return torch.randn(*s, generator=gen, device=dev)

    q = _l2norm(randn(B, T, H, D)).to(torch.bfloat16)
    k = _l2norm(randn(B, T, H, D)).to(torch.bfloat16)
    v = randn(B, T, H, D).to(torch.bfloat16)
    beta = torch.sigmoid(randn(B, T, H))
    g = -F.softplus(randn(B, T, H))
    if strong:  # 10% of tokens (all heads) decay with g = -8
        mask = torch.rand(B, T, generator=gen, device=dev) < 0.1
        g = torch.where(mask[:, :, None], torch.full_like(g, -8.0), g)
    return q, k, v, g, beta


def geometric_cu_seqlens(total, seed):
    """Document lengths 16 + Geometric(p = 1/1009) (mean 1024), the last truncated."""
    gen = torch.Generator().manual_seed(seed)
    p = 1.0 / 1009.0
    cu = [0]
    while cu[-1] < total:
        u = torch.rand((), generator=gen, dtype=torch.float64).item()
        n = 16 + int(math.floor(math.log1p(-u) / math.log1p(-p)))
        cu.append(min(total, cu[-1] + n))
    return torch.tensor(cu, dtype=torch.int32)


@pytest.mark.parametrize("case", ["c2", "c3", "c5"])
def test_full_size_forward_matches_fp32_recurrence(dev, case):
    from delta_feedback_experiment_amd import chunk_pkda, fused_recurrent_pkda

    B, T, H, D, strong, with_s0, varlen = {
        "c2": (8, 4096, 16, 128, False, False, False),
        "c3": (1, 32768, 16, 128, False, False, True),
        "c5": (2, 16384, 32, 128, True, True, False),
    }[case]
    print(f"[gpu] full-size forward {case}: B{B} T{T} H{H} D{D}", flush=True)
    q, k, v, g, beta = make_inputs(dev, B, T, H, D, seed=11, strong=strong)
    cu = geometric_cu_seqlens(T, seed=42).to(dev) if varlen else None
    N = B if cu is None else cu.numel() - 1
    s0 = None
    if with_s0:
        gen = torch.Generator(device=dev).manual_seed(12)
        s0 = 0.02 * torch.randn(N, H, D, D, generator=gen, device=dev)
    o, S, _ = chunk_pkda(q, k, v, g, beta, initial_state=s0, output_final_state=True, cu_seqlens=cu)
    o_ref, S_ref, _ = fused_recurrent_pkda(q.float(), k.float(), v.float(), g, beta, initial_state=s0,
                                           output_final_state=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    e_o, e_s = rel_l2(o.float(), o_ref), rel_l2(S, S_ref)
    print(f"  rel o {e_o:.3e} S {e_s:.3e} ({N} sequences)", flush=True)
    assert e_o < BF16_TOL
    assert e_s < BF16_TOL


def test_full_length_gradients_match_oracle_on_a_slice(dev):
    """c2 (B8 T4096 H16 D128): batch row 5, heads 0..3 against the oracle."""
    from delta_feedback_experiment_amd import chunk_pkda

    B, T, H, D = 8, 4096, 16, 128
    row, heads = 5, slice(0, 4)
    q, k, v, g, beta = make_inputs(dev, B, T, H, D, seed=21)
    gen = torch.Generator(device=dev).manual_seed(22)
    do = torch.randn(B, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    print("[gpu] full-length gradients c2, row 5 heads 0-3 vs oracle", flush=True)
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v, g, beta)]
    o, _, _ = chunk_pkda(*leaves)
    got = torch.autograd.grad(o, leaves, do)
    torch.cuda.synchronize()

    def cut(t):
        return t[row:row + 1, :, heads].detach().cpu()

    ref_leaves = [cut(t).float().requires_grad_() for t in (q, k, v, g, beta)]
    o_ref, _, _ = oracle.pkda_reference(*ref_leaves, out_dtype=torch.float32)
    ref = torch.autograd.grad(o_ref, ref_leaves, cut(do).float())
    errs = {"o": rel_l2(cut(o).float(), o_ref)}
    errs.update({n: rel_l2(cut(a).float(), b) for n, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"), got, ref)})
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    bad = {n: e for n, e in errs.items() if not e < BF16_TOL}
    assert not bad, bad


def test_full_size_gradients_stay_in_their_row_and_head(dev):
    """c2: changing dO in one (row, head) leaves every other row's and head's
    gradients bitwise unchanged."""
    from delta_feedback_experiment_amd import chunk_pkda

    B, T, H, D = 8, 4096, 16, 128
    q, k, v, g, beta = make_inputs(dev, B, T, H, D, seed=31)
    gen = torch.Generator(device=dev).manual_seed(32)
    do = torch.randn(B, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    do2 = do.clone()
    do2[3, :, 7] = torch.randn(T, D, generator=gen, device=dev).to(torch.bfloat16)
    print("[gpu] full-size row/head independence c2", flush=True)

    def grads(d):
        leaves = [t.detach().clone().requires_grad_() for t in (q, k, v, g, beta)]
        o, _, _ = chunk_pkda(*leaves)
        return torch.autograd.grad(o, leaves, d)

    a, b = grads(do), grads(do2)
    torch.cuda.synchronize()
    keep = torch.ones(B, H, dtype=torch.bool, device=dev)
    keep[3, 7] = False
    for name, x, y in zip(("dq", "dk", "dv", "dg", "dbeta"), a, b):
        xs, ys = x.transpose(1, 2)[keep], y.transpose(1, 2)[keep]
        assert torch.equal(xs, ys), f"{name} changed outside row 3 head 7"
        assert not torch.equal(x.transpose(1, 2)[3, 7], y.transpose(1, 2)[3, 7]), f"{name} ignores dO"


def test_c3_full_size_gradients_per_document(dev):
    """c3 (one packed row of 32,768 tokens, geometric documents, H16 d128 bf16),
    forward and backward at full size.

    * Document independence, bitwise: the gradients of three documents (the
      first, the longest and the last) equal those of the same document run
      on its own -- chunks start at document boundaries and every state
      resets there, so the arithmetic is the same.
    * The leading documents (those ending by token 1,024) against the CPU
      oracle's FP32 autograd on the same BF16-rounded values."""
    from delta_feedback_experiment_amd import chunk_pkda

    T, H, D = 32768, 16, 128
    q, k, v, g, beta = make_inputs(dev, 1, T, H, D, seed=41)
    cu = geometric_cu_seqlens(T, seed=42).to(dev)
    gen = torch.Generator(device=dev).manual_seed(43)
    do = torch.randn(1, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    print(f"[gpu] c3 full-size gradients ({cu.numel() - 1} documents)", flush=True)

    def run(sl, cu_part):
        leaves = [t[:, sl].detach().clone().requires_grad_() for t in (q, k, v, g, beta)]
        o, _, _ = chunk_pkda(*leaves, cu_seqlens=cu_part)
        return (o, *torch.autograd.grad(o, leaves, do[:, sl]))

    full = run(slice(0, T), cu)
    cuh = cu.cpu().tolist()
    lens = [b - a for a, b in zip(cuh, cuh[1:])]
    for n in sorted({0, max(range(len(lens)), key=lambda i: lens[i]), len(lens) - 1}):
        a, b = cuh[n], cuh[n + 1]
        one = run(slice(a, b), torch.tensor([0, b - a], dtype=torch.int32, device=dev))
        for name, x, y in zip(("o", "dq", "dk", "dv", "dg", "dbeta"), full, one):
            assert torch.equal(x[:, a:b], y), f"document {n}: {name} differs from its own run"
    lead = max(i for i in range(len(cuh)) if cuh[i] <= 1024)
    end = cuh[lead]
    assert end > 0
    leaves = [t[:, :end].detach().cpu().float().requires_grad_() for t in (q, k, v, g, beta)]
    o_r, _, _ = oracle.pkda_reference(*leaves, cu_seqlens=torch.tensor(cuh[:lead + 1]), out_dtype=torch.float32)
    ref = torch.autograd.grad(o_r, leaves, do[:, :end].cpu().float())
    errs = {"o": rel_l2(full[0][:, :end].float(), o_r)}
    errs.update({n: rel_l2(a[:, :end].float(), b) for n, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"),
                                                                        full[1:], ref)})
    print(f"  documents 0..{lead - 1} (tokens 0..{end - 1}): " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    bad = {n: e for n, e in errs.items() if not e < BF16_TOL}
    assert not bad, bad


def test_c5_full_size_gradients_with_initial_state(dev):
    """c5 (B2 T16384 H32 d128 bf16, S0 ~ N(0, 0.02), 10% of tokens g = -8),
    forward and backward at full size including dS0.

    * Row independence, bitwise: row 1 run alone gives row 1's gradients
      and dS0 of the batch run.
    * A slice against the oracle: with these decays (g <= -softplus(.)
      everywhere) a token's influence on S0's gradient, and the later tokens'
      influence on the first 256 tokens' gradients, fall below e^-150 within
      a few hundred tokens, so dS0 and the gradients of tokens 0..255 of the
      full run equal those of the oracle's run over the first 1,024 tokens
      (loss on those outputs only) to far below the BF16 bar."""
    from delta_feedback_experiment_amd import chunk_pkda

    B, T, H, D = 2, 16384, 32, 128
    q, k, v, g, beta = make_inputs(dev, B, T, H, D, seed=51, strong=True)
    gen = torch.Generator(device=dev).manual_seed(52)
    s0 = 0.02 * torch.randn(B, H, D, D, generator=gen, device=dev)
    do = torch.randn(B, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    dS = torch.randn(B, H, D, D, generator=gen, device=dev)
    print("[gpu] c5 full-size gradients with dS0", flush=True)

    def run(rows):
        leaves = [t[rows].detach().clone().requires_grad_() for t in (q, k, v, g, beta, s0)]
        o, S, _ = chunk_pkda(*leaves[:5], initial_state=leaves[5], output_final_state=True)
        return (o, S, *torch.autograd.grad([o, S], leaves, [do[rows], dS[rows]]))

    full = run(slice(0, B))
    alone = run(slice(1, 2))
    for name, x, y in zip(("o", "S", "dq", "dk", "dv", "dg", "dbeta", "dS0"), full, alone):
        assert torch.equal(x[1:2], y), f"row 1: {name} differs from its own run"
    Ts, keep = 1024, 256
    cut = [t[:1, :Ts].detach().cpu().float() for t in (q, k, v, g, beta)]
    leaves = [t.clone().requires_grad_() for t in cut] + [s0[:1].detach().cpu().clone().requires_grad_()]
    o_r, _, _ = oracle.pkda_reference(*leaves[:5], initial_state=leaves[5], out_dtype=torch.float32)
    ref = torch.autograd.grad(o_r, leaves, do[:1, :Ts].cpu().float())
    errs = {"o": rel_l2(full[0][:1, :Ts].float(), o_r)}
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"), full[2:7], ref[:5]):
        errs[name] = rel_l2(a[:1, :keep].float(), b[:, :keep])
    errs["dS0"] = rel_l2(full[7][:1], ref[5])
    print("  row 0, tokens 0..255 and dS0: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    bad = {n: e for n, e in errs.items() if not e < BF16_TOL}
    assert not bad, bad


def _production_inputs(dev, B, T, H, D, seed):
    """The production operator's inputs as the reference's bench draws them
    (scripts/pkda_bench.py:162-187): raw per-channel gate, A_log = log U(1, 16),
    preconditioner with x = 1.5; BF16 activations."""
    gen = torch.Generator(device=dev).manual_seed(seed)

    def rn(*s):
        return torch.randn(*s, generator=gen, device=dev)

    q = _l2norm(rn(B, T, H, D)).to(torch.bfloat16)
    k = _l2norm(rn(B, T, H, D)).to(torch.bfloat16)
    v = rn(B, T, H, D).to(torch.bfloat16)
    g_raw = (0.2 * rn(B, T, H, D)).to(torch.bfloat16)
    beta = torch.sigmoid(0.2 * rn(B, T, H))
    A_log = torch.empty(H, device=dev).uniform_(1, 16, generator=gen).log()
    dt_bias = 0.1 * rn(H * D)
    g_atk = -F.softplus(0.2 * rn(B, T, H) + 0.3)
    beta_atk = torch.sigmoid(rn(B, T, H))
    center = -0.2 + 0.1 * rn(H)
    do = rn(B, T, H, D).to(torch.bfloat16)
    return [q, k, v, g_raw, g_atk, beta_atk, beta, A_log, dt_bias, center], do


PRODUCTION_NAMES = ("q", "k", "v", "g", "g_atk", "beta_atk", "beta", "A_log", "dt_bias", "log_atk_scale")


def test_production_operator_full_length(dev):
    """pkda_recurrence (the reference model's training operator: raw
    per-channel gate, preconditioner x = 1.5, all ten gradients) at the c2
    geometry B8 T4096 H16 d128 -- 64 chunks per document through the
    per-channel state passes and the preconditioner's chunk scan.

    * Independence, bitwise: row 2, heads 4..7 run alone give the full run's
      output and per-token gradients of that row and those heads.
    * That slice (all 4,096 tokens) against the CPU oracle's FP32 autograd on
      the same BF16-rounded values, every gradient including dA_log,
      ddt_bias and dlog_atk_scale (which the slice run sums over its own row
      and heads)."""
    from delta_feedback_experiment_amd import pkda_recurrence

    B, T, H, D = 8, 4096, 16, 128
    row, hs = 2, slice(4, 8)
    inputs, do = _production_inputs(dev, B, T, H, D, seed=61)
    print("[gpu] production operator c2 geometry: full run, row 2 heads 4-7 alone, oracle", flush=True)

    def run(ins, d):
        leaves = [x.detach().clone().requires_grad_() for x in ins]
        o, _ = pkda_recurrence(*leaves, D ** -0.5, 1.5, 1e-6, False)
        return (o, *torch.autograd.grad(o, leaves, d))

    full = run(inputs, do)
    tok = lambda t: t[row:row + 1, :, hs].contiguous()  # noqa: E731
    q, k, v, g, g_atk, beta_atk, beta, A_log, dt_bias, center = inputs
    part_in = [tok(q), tok(k), tok(v), tok(g), tok(g_atk), tok(beta_atk), tok(beta), A_log[hs].contiguous(),
               dt_bias.view(H, D)[hs].reshape(-1).contiguous(), center[hs].contiguous()]
    part = run(part_in, tok(do))
    torch.cuda.synchronize()
    for name, x, y in zip(("o",) + PRODUCTION_NAMES[:7], full[:8], part[:8]):
        assert torch.equal(tok(x), y), f"{name}: row {row} heads 4-7 differ from their own run"
    del full
    cl = [x.detach().float().cpu().clone().requires_grad_() for x in part_in]
    o_r = oracle.pkda_reference(cl[0], cl[1], cl[2], cl[3], cl[6], A_log=cl[7], dt_bias=cl[8],
                                use_gate_in_kernel=True, g_atk=cl[4], beta_atk=cl[5], log_atk_scale=cl[9],
                                x=1.5, eps=1e-6, out_dtype=torch.float32)[0]
    ref = torch.autograd.grad(o_r, cl, tok(do).float().cpu())
    errs = {"o": rel_l2(part[0].float(), o_r)}
    for n, a, b, x in zip(PRODUCTION_NAMES, part[1:], ref, part_in):
        assert a.dtype == x.dtype, (n, a.dtype, x.dtype)
        errs["d" + n] = rel_l2(a.float(), b)
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    bad = {n: e for n, e in errs.items() if not e < BF16_TOL}
    assert not bad, bad
