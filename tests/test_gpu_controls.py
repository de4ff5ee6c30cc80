"""The control path on the GPU: control activations with their packed
gradient, and the decay expansion fused into the gate kernel.

Bars: FP32 inputs <= 1e-5 relative L2 against the FP32 oracle; BF16 inputs
<= 2e-2 against the FP32 oracle on the same BF16-rounded inputs.  The hidden
slices must be views of the packed projection, as the reference's split
returns them (delta_feedback_experiment/pkda.py:56-74).
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2
from oracle import controls_oracle as co
from oracle import pkda_oracle as oracle
from test_gpu_chunk import make_inputs

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _tol(dtype):
    return FP32_TOL if dtype == torch.float32 else BF16_TOL


def _control_inputs(B, T, H, d, dtype, seed, pad=0):
    """The packed projection at the scale the module produces it: unit-RMS
    activations through nn.Linear's default init give std 1/sqrt(3)."""
    gen = torch.Generator().manual_seed(seed)
    width = 2 * d + 3 * H
    full = (torch.randn(B, T, width + pad, generator=gen) / 3 ** 0.5).to(dtype)
    A_log_p = torch.empty(H).uniform_(1, 16, generator=gen).log()
    dt_bias_p = 0.1 * torch.randn(H, generator=gen)
    return full, A_log_p, dt_bias_p


@pytest.mark.parametrize("dtype,pad", [(torch.bfloat16, 0), (torch.float32, 0), (torch.bfloat16, 8)])
def test_controls_forward_and_packed_gradient(dev, dtype, pad):
    """pad > 0: the packed projection is a strided slice of a wider buffer,
    as the reference's aligned linear output (pkda.py:322-328)."""
    from delta_feedback_experiment_amd import pkda_controls

    print(f"[gpu] controls {dtype} pad={pad}", flush=True)
    B, T, H, d = 2, 70, 4, 64
    width = 2 * d + 3 * H
    full, A_log_p, dt_bias_p = _control_inputs(B, T, H, d, dtype, seed=7 + pad, pad=pad)
    gen = torch.Generator().manual_seed(99)
    grads = [torch.randn(B, T, d, generator=gen).to(dtype), torch.randn(B, T, H, generator=gen).to(dtype),
             torch.randn(B, T, H, generator=gen), torch.randn(B, T, H, generator=gen).to(dtype),
             torch.randn(B, T, d, generator=gen).to(dtype)]

    leaves = [full[..., :width].float().clone().requires_grad_(), A_log_p.clone().requires_grad_(),
              dt_bias_p.clone().requires_grad_()]
    ref = co.controls_reference(leaves[0], leaves[1], leaves[2], d, H)
    gref = torch.autograd.grad(ref, leaves, [g.float() for g in grads])

    fd = full.to(dev)
    packed = fd[..., :width].detach().requires_grad_() if pad == 0 else fd[..., :width]
    if pad:
        fd.requires_grad_()
        packed = fd[..., :width]
    A_d, dt_d = A_log_p.to(dev).requires_grad_(), dt_bias_p.to(dev).requires_grad_()
    out = pkda_controls(packed, A_d, dt_d, d, H)
    assert out[0].data_ptr() == packed.data_ptr() and out[4].data_ptr() == packed[..., d + 3 * H:].data_ptr()
    assert out[1].dtype == dtype and out[2].dtype == torch.float32 and out[3].dtype == dtype
    src = fd if pad else packed
    got = torch.autograd.grad(out, [src, A_d, dt_d], [g.to(dev) for g in grads])
    torch.cuda.synchronize()
    res = {n: rel_l2(a.float(), b) for n, a, b in zip(("hidden", "beta", "pdecay", "pbeta", "gate"), out, ref)}
    dpacked = got[0][..., :width] if pad else got[0]
    res.update({"dpacked": rel_l2(dpacked.float(), gref[0]), "dA_log_p": rel_l2(got[1], gref[1]),
                "ddt_bias_p": rel_l2(got[2], gref[2])})
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in res.items()), flush=True)
    for name, val in res.items():
        assert val < _tol(dtype), (name, val)
    if pad:
        assert torch.all(got[0][..., width:] == 0)


def test_controls_missing_gradients_are_zero(dev):
    from delta_feedback_experiment_amd import pkda_controls

    B, T, H, d = 1, 9, 2, 64
    full, A_log_p, dt_bias_p = _control_inputs(B, T, H, d, torch.float32, seed=3)
    packed = full.to(dev).requires_grad_()
    out = pkda_controls(packed, A_log_p.to(dev), dt_bias_p.to(dev), d, H)
    (gp,) = torch.autograd.grad(out[1].sum(), [packed])  # only beta is used
    torch.cuda.synchronize()
    beta = torch.sigmoid(full[..., d:d + H])
    assert torch.all(gp[..., :d] == 0) and torch.all(gp[..., d + H:] == 0)
    assert rel_l2(gp[..., d:d + H].cpu(), beta * (1 - beta)) < FP32_TOL


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_decay_expansion_in_the_gate_matches_the_oracle(dev, dtype, D):
    """chunk_pkda(decay_up=...) with the decay hidden a strided slice of the
    packed controls, the whole production control path composed: every input
    gradient, decay_up's and the packed projection's included."""
    from delta_feedback_experiment_amd import chunk_pkda, pkda_controls

    print(f"[gpu] decay expansion {dtype} D={D}", flush=True)
    B, T, H = 2, 150, 2
    q, k, v, _, _ = make_inputs(B, T, H, D, dtype, seed=D + 3)
    full, A_log_p, dt_bias_p = _control_inputs(B, T, H, D, dtype, seed=D + 4)
    gen = torch.Generator().manual_seed(D + 5)
    # nn.Linear's default init, as the module's decay_up (pkda.py:168): U(-1/sqrt(d), 1/sqrt(d))
    up = ((torch.rand(H * D, D, generator=gen) * 2 - 1) / D ** 0.5).to(dtype)
    A_log = torch.empty(H).uniform_(1, 16, generator=gen).log()
    dt_bias = 0.1 * torch.randn(H * D, generator=gen)
    center = torch.full((H,), -0.2)
    do = torch.randn(B, T, H, D, generator=gen).to(dtype)
    names = ("q", "k", "v", "packed", "decay_up", "A_log_p", "dt_bias_p", "A_log", "dt_bias")
    base = (q, k, v, full, up, A_log_p, dt_bias_p, A_log, dt_bias)

    def run(t, device):
        if device is None:
            raw, beta, pdecay, pbeta, _ = co.controls_reference(t[3], t[5], t[6], D, H, decay_up=t[4])
            o, _, _ = oracle.pkda_reference(t[0], t[1], t[2], raw, beta, A_log=t[7], dt_bias=t[8],
                                            use_gate_in_kernel=True, g_atk=pdecay, beta_atk=pbeta,
                                            log_atk_scale=center, x=1.5, eps=1e-6, out_dtype=torch.float32)
        else:
            hidden, beta, pdecay, pbeta, _ = pkda_controls(t[3], t[5], t[6], D, H)
            assert hidden.data_ptr() == t[3].data_ptr()
            o, _, _ = chunk_pkda(t[0], t[1], t[2], hidden, beta, decay_up=t[4], A_log=t[7], dt_bias=t[8],
                                 use_gate_in_kernel=True, g_atk=pdecay, beta_atk=pbeta,
                                 log_atk_scale=center.to(device), x=1.5, eps=1e-6)
        loss = (o.float() * do.to(o.device).float()).sum()
        return o, torch.autograd.grad(loss, t)

    o_r, g_r = run([x.float().clone().requires_grad_() for x in base], None)
    o, g_d = run([x.to(dev).clone().requires_grad_() for x in base], dev)
    torch.cuda.synchronize()
    res = {"o": rel_l2(o.float(), o_r)}
    for n, a, b in zip(names, g_d, g_r):
        res["d" + n] = rel_l2(a.float(), b)
    print("  " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in res.items()), flush=True)
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    for name, val in res.items():
        assert val < tol, (name, val)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.bfloat16, 64), (torch.float32, 64)])
def test_decay_expansion_equals_the_materialised_raw_gate(dev, dtype, D):
    """The fused expansion against the same chunk kernels fed the raw decay
    that F.linear materialises (the reference's dataflow, pkda.py:334-339):
    the raw values agree up to the rounding of two different GEMMs, so the
    outputs and q/k/v gradients agree to FP32 rounding; the hidden's and
    decay_up's gradients differ by the backward GEMMs' dtype (FP32 here,
    the activation dtype in F.linear's backward)."""
    from delta_feedback_experiment_amd import chunk_pkda

    print(f"[gpu] decay expansion vs materialised {dtype} D={D}", flush=True)
    B, T, H = 2, 150, 2
    q, k, v, _, _ = make_inputs(B, T, H, D, dtype, seed=D + 13)
    gen = torch.Generator().manual_seed(D + 14)
    hidden = (torch.randn(B, T, D, generator=gen) / 3 ** 0.5).to(dtype)
    up = ((torch.rand(H * D, D, generator=gen) * 2 - 1) / D ** 0.5).to(dtype)
    A_log = torch.empty(H).uniform_(1, 16, generator=gen).log()
    dt_bias = 0.1 * torch.randn(H * D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    do = torch.randn(B, T, H, D, generator=gen).to(dtype)
    base = (q, k, v, hidden, up, A_log, dt_bias)

    def run(fused):
        t = [x.to(dev).clone().requires_grad_() for x in base]
        if fused:
            o, _, _ = chunk_pkda(t[0], t[1], t[2], t[3], beta.to(dev), decay_up=t[4], A_log=t[5], dt_bias=t[6],
                                 use_gate_in_kernel=True)
        else:
            raw = torch.nn.functional.linear(t[3], t[4]).reshape(B, T, H, D)
            o, _, _ = chunk_pkda(t[0], t[1], t[2], raw, beta.to(dev), A_log=t[5], dt_bias=t[6],
                                 use_gate_in_kernel=True)
        return o, torch.autograd.grad((o.float() * do.to(dev).float()).sum(), t)

    o_f, g_f = run(True)
    o_m, g_m = run(False)
    torch.cuda.synchronize()
    res = {"o": rel_l2(o_f.float(), o_m.float())}
    for n, a, b in zip(("q", "k", "v", "hidden", "decay_up", "A_log", "dt_bias"), g_f, g_m):
        res["d" + n] = rel_l2(a.float(), b.float())
    print("  " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in res.items()), flush=True)
    # the gate parameters' gradients are sums of cancelling per-token terms:
    # the two GEMMs' different rounding of raw moves them most
    bf16 = dtype == torch.bfloat16
    for name, val in res.items():
        bar = (1e-2 if bf16 else 1e-3) if name in ("dhidden", "ddecay_up", "dA_log", "ddt_bias") else 1e-4
        assert val < bar, (name, val)
