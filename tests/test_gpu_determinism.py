"""Run-twice determinism of the recurrence: no floating-point atomics in any
output or gradient reduction (dbeta, dg, dA_log, ddt_bias, dcenter, dS0,
dA0 are all summed in a fixed order), so the same inputs give the same bits.

* the production training op (``pkda_recurrence``: raw per-channel gate and
  preconditioner, all ten gradients), at a size with many chunks per head;
* ``chunk_pkda`` with packed documents, initial states and the
  preconditioner (per-head gate), output, final states and every gradient.
"""

from __future__ import annotations

import pytest
import torch

from test_gpu_chunk import _precond_inputs, _production_inputs, make_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _same(a, b, what):
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"{what}: output {i} differs between two runs"


def test_production_op_is_bitwise_repeatable(dev):
    from delta_feedback_experiment_amd import pkda_recurrence

    print("[gpu] determinism: pkda_recurrence twice", flush=True)
    B, T, H, D = 2, 1000, 4, 128
    base = _production_inputs(B, T, H, D, torch.bfloat16, seed=81)
    (q, k, v, g_raw, beta, A_log, dt_bias, g_atk, beta_atk, center) = base
    inputs = (q, k, v, g_raw, g_atk, beta_atk, beta, A_log, dt_bias, center)
    do = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(82)).to(torch.bfloat16).to(dev)

    def run():
        leaves = [x.to(dev).clone().requires_grad_() for x in inputs]
        o, _ = pkda_recurrence(*leaves, D ** -0.5, 1.5, 1e-6, False)
        grads = torch.autograd.grad([o], leaves, [do])
        torch.cuda.synchronize()
        return [o, *grads]

    _same(run(), run(), "pkda_recurrence")


def test_chunk_pkda_is_bitwise_repeatable(dev):
    from delta_feedback_experiment_amd import chunk_pkda

    print("[gpu] determinism: chunk_pkda twice", flush=True)
    T, H, D = 700, 8, 128
    cu = torch.tensor([0, 64, 65, 400, 700], dtype=torch.int32)
    N = cu.numel() - 1
    q, k, v, g, beta = make_inputs(1, T, H, D, torch.bfloat16, seed=83, strong=True)
    gen = torch.Generator().manual_seed(84)
    g_atk, beta_atk, center = _precond_inputs(1, T, H, gen)
    S0 = 0.02 * torch.randn(N, H, D, D, generator=gen)
    A0 = 0.1 * torch.randn(N, H, D, generator=gen).abs()
    do = torch.randn(1, T, H, D, generator=gen).to(torch.bfloat16).to(dev)
    dS = torch.randn(N, H, D, D, generator=gen).to(dev)
    dA = torch.randn(N, H, D, generator=gen).to(dev)
    inputs = (q, k, v, g, beta, g_atk, beta_atk, center, S0, A0)

    def run():
        t = [x.to(dev).clone().requires_grad_() for x in inputs]
        o, S, A = chunk_pkda(*t[:5], g_atk=t[5], beta_atk=t[6], log_atk_scale=t[7], initial_state=t[8],
                             initial_A_state=t[9], output_final_state=True, x=1.5, eps=1e-6,
                             cu_seqlens=cu.to(dev))
        grads = torch.autograd.grad([o, S, A], t, [do, dS, dA])
        torch.cuda.synchronize()
        return [o, S, A, *grads]

    _same(run(), run(), "chunk_pkda")
