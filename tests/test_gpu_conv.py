"""The fused Q/K/V convolution kernels on the GPU against the CPU oracle.

Bars: FP32 inputs <= 1e-5 relative L2 against the FP32 oracle; BF16 inputs
<= 2e-2 against the FP32 oracle on the same BF16-rounded inputs.  Outputs
q, k, v and gradients dx, dw.  Includes the reference's screen geometry
(8 rows x 4,096 tokens, 8 heads of 128, conv_size 4) at full size.
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2
from oracle import qkv_conv_oracle as co

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2
EPS = 1e-6


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def make(B, T, H, d, W, dtype, w_dtype=torch.float32, seed=0):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, 3 * H * d, generator=gen).to(dtype)
    w = (0.5 * torch.randn(3 * H * d, W, generator=gen)).to(w_dtype)
    do = [torch.randn(B, T, H * d, generator=gen).to(dtype) for _ in range(3)]
    return x, w, do


def run_case(dev, B, T, H, d, W, dtype, w_dtype=torch.float32, seed=0):
    from delta_feedback_experiment_amd import pkda_qkv_conv

    x, w, do = make(B, T, H, d, W, dtype, w_dtype, seed)
    P = H * d
    xl = x.float().requires_grad_()
    wl = w.float().requires_grad_()
    ref = co.qkv_conv_reference(xl, wl, d, 2 * P, EPS, out_dtype=torch.float32)
    gref = torch.autograd.grad(ref, (xl, wl), [t.float() for t in do])
    xd, wd = x.to(dev).requires_grad_(), w.to(dev).requires_grad_()
    out = pkda_qkv_conv(xd, wd, d, 2 * P, EPS)
    got = torch.autograd.grad(out, (xd, wd), [t.to(dev) for t in do])
    torch.cuda.synchronize()
    errs = {n: rel_l2(a.float(), b) for n, a, b in zip(("q", "k", "v"), out, ref)}
    errs["dx"] = rel_l2(got[0].float(), gref[0])
    errs["dw"] = rel_l2(got[1].float(), gref[1])
    assert out[0].dtype == dtype and got[0].dtype == dtype and got[1].dtype == w_dtype
    return errs


@pytest.mark.parametrize("W", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_matches_oracle(dev, W, d, dtype):
    print(f"[gpu] qkv conv W={W} d={d} {dtype}", flush=True)
    errs = run_case(dev, 2, 100, 3, d, W, dtype, seed=W + d)  # 100 = one full tile + a partial one
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    assert all(e < tol for e in errs.values()), errs


@pytest.mark.parametrize("T", [1, 2, 3, 64, 65])
def test_conv_short_and_boundary_lengths(dev, T):
    print(f"[gpu] qkv conv T={T}", flush=True)
    errs = run_case(dev, 3, T, 2, 32, 4, torch.float32, seed=T)
    assert all(e < FP32_TOL for e in errs.values()), errs


def test_conv_bf16_weights(dev):
    print("[gpu] qkv conv bf16 weights", flush=True)
    errs = run_case(dev, 2, 70, 2, 64, 4, torch.bfloat16, w_dtype=torch.bfloat16, seed=9)
    assert all(e < BF16_TOL for e in errs.values()), errs


def test_conv_backward_is_deterministic(dev):
    from delta_feedback_experiment_amd.conv import pkda_qkv_conv_backward

    x, w, do = make(4, 300, 4, 64, 4, torch.bfloat16, seed=11)
    args = [t.to(dev) for t in (x, w, *do)]
    a = pkda_qkv_conv_backward(*args, 64, 2 * 256, EPS)
    b = pkda_qkv_conv_backward(*args, 64, 2 * 256, EPS)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_conv_screen_geometry_full_size(dev):
    """8 rows x 4,096 tokens, 8 heads of 128 (projection width 1,024), 4 taps."""
    print("[gpu] qkv conv screen geometry B8 T4096 P1024", flush=True)
    errs = run_case(dev, 8, 4096, 8, 128, 4, torch.bfloat16, seed=21)
    print("  " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert all(e < BF16_TOL for e in errs.values()), errs
