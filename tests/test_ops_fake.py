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
    assert len(saved) == (3 if lean else 11)
    if not lean:  # the gate's chunk cumsum is retained for the backward
        assert named["gcum"].shape == (B * T, H, D) and named["gcum"].dtype == torch.float32


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


def _serving_args(N=3, P=8, H=2, D=64, T=40):
    def mk(*s, dt=torch.float32):
        return torch.randn(*s, dtype=dt, device="meta")

    dec = (mk(N, H, D, dt=torch.bfloat16), mk(N, H, D, dt=torch.bfloat16), mk(N, H, D, dt=torch.bfloat16),
           mk(N, H), mk(N, H), mk(P, H, D, D), torch.zeros(N, dtype=torch.int32, device="meta"))
    pre = (mk(N, T, H, D, dt=torch.bfloat16), mk(N, T, H, D, dt=torch.bfloat16), mk(N, T, H, D, dt=torch.bfloat16),
           mk(N, T, H), mk(N, T, H))
    return dec, pre


def test_serving_ops_trace_as_mutating_custom_ops():
    """Prefill into pool slots, then a decode step: both trace as opaque
    custom ops whose schema marks the pools as mutated (``mutates_args``:
    an in-place serving operator must declare what it writes, or a compiled
    caller would reorder or drop its writes)."""
    from delta_feedback_experiment_amd import pkda_decode_step_, pkda_prefill_

    (q, k, v, g, beta, pool, idx), (pq, pk, pv, pg, pb) = _serving_args()

    def serve(pq, pk, pv, pg, pb, q, k, v, g, beta, pool, idx):
        o_pre = pkda_prefill_(pq, pk, pv, pg, pb, pool, idx)
        o_dec = pkda_decode_step_(q, k, v, g, beta, pool, idx)
        return o_pre, o_dec

    gm = make_fx(serve, tracing_mode="fake")(pq, pk, pv, pg, pb, q, k, v, g, beta, pool, idx)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert "pkda_mi355x.prefill_.default" in targets
    assert "pkda_mi355x.decode_step_.default" in targets
    for name in ("decode_step_", "prefill_"):
        schema = getattr(torch.ops.pkda_mi355x, name).default._schema
        mutated = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert mutated == {"state_pool", "a_pool", "o"}, (name, mutated)
    schema = torch.ops.pkda_mi355x.qkv_conv_cached_.default._schema
    assert {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write} == {"conv_pool"}


def test_serving_ops_compile_fullgraph():
    """torch.compile(fullgraph=True) over prefill + decode (functionalized
    by AOT autograd): no graph break, outputs of the documented shapes."""
    from delta_feedback_experiment_amd import pkda_decode_step_, pkda_prefill_

    (q, k, v, g, beta, pool, idx), (pq, pk, pv, pg, pb) = _serving_args()

    def serve(pq, pk, pv, pg, pb, q, k, v, g, beta, pool, idx):
        o_pre = pkda_prefill_(pq, pk, pv, pg, pb, pool, idx)
        return o_pre, pkda_decode_step_(q, k, v, g, beta, pool, idx)

    torch._dynamo.reset()
    o_pre, o_dec = torch.compile(serve, fullgraph=True, backend="aot_eager")(pq, pk, pv, pg, pb, q, k, v, g, beta,
                                                                              pool, idx)
    assert o_pre.shape == pv.shape and o_dec.shape == v.shape and o_dec.dtype == torch.bfloat16


def test_serving_ops_refuse_cpu_tensors():
    from delta_feedback_experiment_amd import pkda_decode_step_

    q = torch.zeros(2, 1, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkda_decode_step_(q, q, q, torch.zeros(2, 1), torch.zeros(2, 1), torch.zeros(4, 1, 64, 64), None)
