"""The drop-in under its caller's compiler and autocast.

The reference compiles each PKDA block with ``torch.compile(fullgraph=True)``
and inductor (``delta_feedback_experiment/model.py:925-935``) and runs it under
BF16 autocast; its recurrence op records the forward's autocast state and runs
the backward under it (``delta_feedback_experiment/fla_ops.py:433-437,
540-553``).  Here a small block -- projections, per-head L2 norm, controls,
``pkda_recurrence``, ``pkda_norm_gate``, output projection -- is compiled the
same way, forward and backward, and compared with the same block run eagerly;
and the backward op is checked to receive the forward's autocast dtype.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from conftest import rel_l2

pytestmark = pytest.mark.gpu

COMPILE_TOL = 5e-3


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


class PkdaBlock(torch.nn.Module):
    """The PKDA mixer's dataflow around the recurrence (pkda.py:477-559, with
    plain projections in place of the fused conv)."""

    def __init__(self, dm: int, H: int, d: int, gen: torch.Generator):
        super().__init__()
        self.H, self.d = H, d
        lin = lambda o, i: torch.nn.Parameter(torch.randn(o, i, generator=gen) / math.sqrt(i))  # noqa: E731
        self.w_qkv, self.w_decay, self.w_ctl = lin(3 * H * d, dm), lin(H * d, dm), lin(3 * H, dm)
        self.w_gate, self.w_out = lin(H * d, dm), lin(dm, H * d)
        self.A_log = torch.nn.Parameter(torch.empty(H).uniform_(0, math.log(16), generator=gen))
        self.dt_bias = torch.nn.Parameter(0.1 * torch.randn(H * d, generator=gen))
        self.A_log_p = torch.nn.Parameter(torch.zeros(H))
        self.dt_bias_p = torch.nn.Parameter(torch.zeros(H))
        self.center = torch.nn.Parameter(torch.full((H,), -0.2))
        self.norm_w = torch.nn.Parameter(torch.ones(d))

    def forward(self, x, act=torch.bfloat16):
        """``act``: the activation dtype the recurrence and the norm gate see
        (the projections run in the dtype of ``x`` and the weights, or under
        the caller's autocast)."""
        from delta_feedback_experiment_amd import pkda_norm_gate, pkda_recurrence

        B, T, _ = x.shape
        H, d = self.H, self.d
        q, k, v = F.linear(x, self.w_qkv).view(B, T, 3, H, d).unbind(2)
        q, k = (t.float() * torch.rsqrt(t.float().square().sum(-1, keepdim=True) + 1e-6) for t in (q, k))
        c = F.linear(x, self.w_ctl).view(B, T, 3, H).float()
        beta = torch.sigmoid(c[:, :, 0])
        g_atk = -self.A_log_p.exp() * F.softplus(c[:, :, 1] + self.dt_bias_p)
        beta_atk = torch.sigmoid(c[:, :, 2])
        g = F.linear(x, self.w_decay).view(B, T, H, d)
        o, _ = pkda_recurrence(q.to(act).contiguous(), k.to(act).contiguous(), v.to(act).contiguous(), g.to(act),
                               g_atk, beta_atk, beta, self.A_log, self.dt_bias, self.center, d ** -0.5, 1.5, 1e-6,
                               False)
        gate = F.linear(x, self.w_gate).view(B, T, H, d)
        y, _ = pkda_norm_gate(o, gate.to(act), self.norm_w, 1e-6)
        return F.linear(y.reshape(B, T, H * d).to(x.dtype), self.w_out)


def _step(block, x, dy, autocast=True):
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        y = block(x)
    grads = torch.autograd.grad((y.float() * dy).sum(), [x] + list(block.parameters()))
    return y, grads


@pytest.mark.timeout(600)
def test_compiled_block_matches_eager(dev):
    """FP32 projections with the recurrence and the norm gate fed BF16 (the
    explicit casts are rounding points in both runs, so the compiled and the
    eager block see the same BF16 operands up to the last bit of a few
    normalised values): compiled within 5e-3 of eager on the output and every
    gradient, and the compiled graph's replays repeat bitwise."""
    import torch._inductor.config as inductor_config

    print("[gpu] torch.compile(fullgraph=True, inductor) PKDA block vs eager", flush=True)
    gen = torch.Generator().manual_seed(0)
    B, T, H, d, dm = 2, 128, 2, 64, 128
    block = PkdaBlock(dm, H, d, gen).to(dev)
    x = torch.randn(B, T, dm, generator=gen).to(dev).requires_grad_()
    dy = torch.randn(B, T, dm, generator=gen).to(dev)
    y_e, g_e = _step(block, x, dy, autocast=False)
    inductor_config.compile_threads = 1  # no compile worker pool on the GPU box
    torch._dynamo.reset()
    compiled = torch.compile(block, fullgraph=True, backend="inductor")
    y_c, g_c = _step(compiled, x, dy, autocast=False)
    torch.cuda.synchronize()
    names = ["x"] + [n for n, _ in block.named_parameters()]
    res = {"y": rel_l2(y_c.float(), y_e.float())}
    res.update({"d" + n: rel_l2(a.float(), b.float()) for n, a, b in zip(names, g_c, g_e)})
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in res.items()), flush=True)
    for n, val in res.items():
        assert val < COMPILE_TOL, (n, val)
    # a second call replays the compiled graph: the same values again
    y_c2, g_c2 = _step(compiled, x, dy, autocast=False)
    torch.cuda.synchronize()
    assert torch.equal(y_c2, y_c)
    for a, b in zip(g_c2, g_c):
        assert torch.equal(a, b)


def test_backward_runs_under_the_forward_autocast_state(dev, monkeypatch):
    """_setup_context records the forward's autocast dtype and the backward op
    receives it (fla_ops.py:546-553), whatever state backward() runs in; the
    kernels take their dtypes from the tensors, so the gradients are the same
    bits either way."""
    from delta_feedback_experiment_amd import ops

    seen = []
    real = ops.pkda_recurrence_backward

    def spy(*args):
        seen.append(args[-2])  # the autocast dtype it is handed (the op enters that state itself)
        return real(*args)

    monkeypatch.setattr(ops, "pkda_recurrence_backward", spy)
    gen = torch.Generator().manual_seed(1)
    block = PkdaBlock(128, 2, 64, gen).to(dev)
    x = torch.randn(1, 96, 128, generator=gen).to(dev).requires_grad_()
    dy = torch.randn(1, 96, 128, generator=gen).to(dev)
    print("[gpu] backward under the forward's autocast state", flush=True)
    _, g_auto = _step(block, x, dy)  # forward under autocast, backward() outside it
    assert seen[-1] == torch.bfloat16, seen
    # the op on its own, forward outside and inside autocast (its inputs are
    # BF16 either way, so only the recorded state differs)
    with torch.autocast("cuda", enabled=False):
        q = torch.randn(1, 64, 2, 64, generator=gen).to(dev, torch.bfloat16)
        leaves = [q.clone().requires_grad_(), q.clone().requires_grad_(), q.clone().requires_grad_(),
                  torch.zeros(1, 64, 2, 64, device=dev, dtype=torch.bfloat16).requires_grad_()]
        lead = [torch.full((1, 64, 2), v, device=dev).requires_grad_() for v in (-0.1, 0.5, 0.5)]
        par = [torch.zeros(2, device=dev).requires_grad_(), torch.zeros(128, device=dev).requires_grad_(),
               torch.full((2,), -0.2, device=dev).requires_grad_()]
        args = leaves + lead + par
        o1, _ = ops.pkda_recurrence(*args, 0.125, 1.5, 1e-6, False)
        g1 = torch.autograd.grad(o1.float().sum(), args)
    assert seen[-1] is None, seen
    with torch.autocast("cuda", dtype=torch.bfloat16):
        o2, _ = ops.pkda_recurrence(*args, 0.125, 1.5, 1e-6, False)
    g2 = torch.autograd.grad(o2.float().sum(), args)  # backward() outside autocast
    assert seen[-1] == torch.bfloat16, seen
    assert torch.equal(o1, o2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    assert all(t is not None for t in g_auto)
