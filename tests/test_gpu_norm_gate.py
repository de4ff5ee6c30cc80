"""The norm-gate kernels on the GPU against the CPU oracle (FP32 autograd is
the gradient oracle).  Bars: FP32 <= 1e-5, BF16 <= 2e-2 relative L2 (against
the FP32 oracle on the same BF16-rounded inputs).  Includes the c2 shape of
the recurrence output (B8 T4096 H16 d128) at full size."""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2
from oracle import norm_gate_oracle as ng

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def run_case(dev, shape, dtype, w_dtype=torch.float32, seed=0):
    from delta_feedback_experiment_amd import pkda_norm_gate

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen).to(dtype)
    g = torch.randn(*shape, generator=gen).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=gen)).to(w_dtype)
    dy = torch.randn(*shape, generator=gen).to(dtype)
    leaves = [t.float().requires_grad_() for t in (x, g, w)]
    y_ref, rstd_ref = ng.norm_gate_reference(*leaves, EPS, out_dtype=torch.float32)
    ref = torch.autograd.grad(y_ref, leaves, dy.float())
    dl = [t.to(dev).requires_grad_() for t in (x, g, w)]
    y, rstd = pkda_norm_gate(*dl, EPS)
    got = torch.autograd.grad(y, dl, dy.to(dev))
    torch.cuda.synchronize()
    assert y.dtype == dtype and got[0].dtype == dtype and got[1].dtype == dtype and got[2].dtype == w_dtype
    errs = {"y": rel_l2(y.float(), y_ref), "rstd": rel_l2(rstd, rstd_ref)}
    errs.update({n: rel_l2(a.float(), b) for n, a, b in zip(("dx", "dgate", "dweight"), got, ref)})
    return errs


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm_gate_matches_oracle(dev, d, dtype):
    print(f"[gpu] norm gate d={d} {dtype}", flush=True)
    errs = run_case(dev, (2, 77, 3, d), dtype, seed=d)
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert all(e < tol for e in errs.values()), errs


def test_norm_gate_single_row_and_bf16_weight(dev):
    errs = run_case(dev, (1, 1, 1, 128), torch.float32, seed=3)
    assert all(e < 1e-5 for e in errs.values()), errs
    errs = run_case(dev, (2, 40, 4, 128), torch.bfloat16, w_dtype=torch.bfloat16, seed=4)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_norm_gate_c2_full_size(dev):
    print("[gpu] norm gate c2 shape B8 T4096 H16 d128", flush=True)
    errs = run_case(dev, (8, 4096, 16, 128), torch.bfloat16, seed=7)
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_norm_gate_backward_is_deterministic(dev):
    from delta_feedback_experiment_amd.norm_gate import pkda_norm_gate, pkda_norm_gate_backward

    gen = torch.Generator(device=dev).manual_seed(5)
    x, g, dy = (torch.randn(4, 999, 8, 128, generator=gen, device=dev).to(torch.bfloat16) for _ in range(3))
    w = torch.ones(128, device=dev)
    _, rstd = pkda_norm_gate(x, g, w, EPS)
    a = pkda_norm_gate_backward(x, g, w, rstd, dy, EPS)
    b = pkda_norm_gate_backward(x, g, w, rstd, dy, EPS)
    torch.cuda.synchronize()
    assert all(torch.equal(u, v) for u, v in zip(a, b))
