"""The training custom op's fake implementations and schema, on the CPU.

``pkda_recurrence`` must trace under fake tensors exactly like the
reference's ``delta_feedback::pkda_recurrence`` (its fake implementation
gives the output and every saved intermediate; the backward op's gives one
gradient per tensor input), so a compiled block keeps one graph
(``delta_feedback_experiment/fla_ops.py:352-378,502-537``).
"""

from __future__ import annotations

import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

from delta_feedback_experiment_amd.ops import intermediate_meta, pkda_recurrence, saved_names

B, T, H, D = 2, 100, 3, 64


def _args(device="meta", dtype=torch.bfloat16):
    def mk(*s, dt=torch.float32):
        return torch.randn(*s, dtype=dt, device=device)

    return [mk(B, T, H, D, dt=dtype) for _ in range(4)] + [mk(B, T, H), mk(B, T, H), mk(B, T, H), mk(H),
                                                           mk(H * D), mk(H)]


@pytest.mark.parametrize("lean", [False, True])
def test_fake_forward_shapes(lean):
    o, saved = pkda_recurrence(*_args(), D ** -0.5, 1.5, 1e-6, lean)
    assert o.shape == (B, T, H, D) and o.dtype == torch.bfloat16
    meta = intermediate_meta(torch.empty(B, T, H, D, dtype=torch.bfloat16), torch.empty(B, T, H, D), lean)
    assert [(tuple(s.shape), s.dtype) for s in saved] == [m for m in meta]
    named = dict(zip(saved_names(torch.empty(1, dtype=torch.bfloat16), lean), saved))
    # T = 100 -> two chunks per row
    assert named["a_chunk"].shape == (B * 2, H, D)
    # BF16 activations also keep the write keys in FP32
    assert named["k_write"].dtype == torch.bfloat16 and named["k_write32"].dtype == torch.float32
    assert len(saved) == (3 if lean else 10)


def test_fp32_activations_save_one_write_key():
    meta = intermediate_meta(torch.empty(B, T, H, D), torch.empty(B, T, H, D), True)
    assert saved_names(torch.empty(1), True) == ("k_write", "a_chunk")
    assert [dt for _, dt in meta] == [torch.float32, torch.float32]


def test_forward_and_backward_trace_as_two_opaque_ops():
    args = [a.requires_grad_() for a in _args()]

    def step(*a):
        o, _ = pkda_recurrence(*a, D ** -0.5, 1.5, 1e-6, True)
        return torch.autograd.grad(o.float().sum(), a)

    gm = make_fx(step, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert "pkda_mi355x.pkda_recurrence.default" in targets
    assert "pkda_mi355x.pkda_recurrence_backward.default" in targets
    out = [n for n in gm.graph.nodes if n.op == "output"][0]
    grads = out.args[0]
    assert len(grads) == 10
    for g, a in zip(grads, args):
        assert tuple(g.meta["val"].shape) == tuple(a.shape)
        assert g.meta["val"].dtype == a.dtype


def test_operator_has_no_cpu_kernel():
    """Registered for the device only, like the reference's op: CPU tensors
    are refused by the dispatcher instead of running a fallback."""
    with pytest.raises(NotImplementedError, match="CPU"):
        pkda_recurrence(*_args(device="cpu"), D ** -0.5, 1.5, 1e-6, True)


def test_operator_validates_shapes():
    from delta_feedback_experiment_amd.ops import _check_inputs

    args = _args(device="cpu")
    args[3] = torch.randn(B, T, H)  # a per-head g is not the raw projection
    with pytest.raises(ValueError, match="raw decay"):
        _check_inputs(*args)
    args = _args(device="cpu")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _check_inputs(*args)
