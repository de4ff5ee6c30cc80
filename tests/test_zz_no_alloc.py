"""pkda_gate_bwd_noalloc (partials in the library's static device array)
against pkda_gate_bwd (partials in a caller workspace), through the C ABI.

Same kernels, same reduction order: dg, dA_log and ddt_bias must agree
bitwise.  Two calls in a row, the second smaller than the first, so the
second reads the scratch the first one left behind -- it must not see any
of it.  (A call past the scratch's capacity is refused before any HIP call:
that case runs in the CPU suite, tests/test_capi.py.)
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _gate_args(plan, g, A_log, dt_bias, dgcum, dg, dA_part, ddt_part, dA_log, ddt_bias):
    from delta_feedback_experiment_amd import _lib
    from delta_feedback_experiment_amd.pkda import _dtype_code, _ptr

    return _lib.GateArgs(
        num_seqs=plan.num_seqs, seqlen=plan.seqlen, heads=plan.heads, head_dim=plan.head_dim,
        gate_kind=_lib.GATE_RAW_CHANNEL, g_dtype=_dtype_code(g), cu_seqlens=_ptr(plan.cu_seqlens), g=_ptr(g),
        A_log=_ptr(A_log), dt_bias=_ptr(dt_bias), dgcum=_ptr(dgcum), dg=_ptr(dg),
        dA_log_part=_ptr(dA_part), ddt_bias_part=_ptr(ddt_part), dA_log=_ptr(dA_log), ddt_bias=_ptr(ddt_bias),
        num_chunks=plan.num_chunks, table=_ptr(plan.table), dg_dtype=_lib.PKDA_F32,
    )


def _run(dev, B, T, H, D, seed, noalloc, cu=None):
    from delta_feedback_experiment_amd import _lib
    from delta_feedback_experiment_amd.chunk import ChunkPlan
    from delta_feedback_experiment_amd.pkda import _stream

    gen = torch.Generator().manual_seed(seed)
    g = (0.5 * torch.randn(B, T, H, D, generator=gen)).to(torch.bfloat16).to(dev)
    A_log = torch.empty(H).uniform_(0, 2.7, generator=gen).to(dev)
    dt_bias = (0.1 * torch.randn(H * D, generator=gen)).to(dev)
    dgcum = torch.randn(B * T, H, D, generator=gen).to(dev)
    plan = ChunkPlan.make(g, None if cu is None else cu.to(dev))
    dg = torch.empty(B * T, H, D, device=dev)
    dA_log = torch.empty(H, device=dev)
    ddt_bias = torch.empty(H * D, device=dev)
    if noalloc:
        parts = (None, None)
    else:
        parts = (torch.empty(plan.num_chunks, H, device=dev), torch.empty(plan.num_chunks, H, D, device=dev))
    args = _gate_args(plan, g.reshape(B * T, H, D), A_log, dt_bias, dgcum, dg, *parts, dA_log, ddt_bias)
    _lib.call("pkda_gate_bwd_noalloc" if noalloc else "pkda_gate_bwd", args, _stream(dev))
    torch.cuda.synchronize()
    return dg.cpu(), dA_log.cpu(), ddt_bias.cpu()


@pytest.mark.parametrize("shapes", [
    ((4, 1024, 8, 128, 1), (1, 300, 4, 64, 2)),     # 64 chunks x 8 heads, then 5 x 4
    ((2, 4096, 16, 128, 3), (2, 130, 2, 128, 4)),   # c2-sized partials (8 MiB), then 6 x 2
])
def test_noalloc_gate_backward_equals_workspace_form(dev, shapes):
    for B, T, H, D, seed in shapes:
        print(f"[gpu] gate bwd noalloc B={B} T={T} H={H} D={D}", flush=True)
        want = _run(dev, B, T, H, D, seed, noalloc=False)
        got = _run(dev, B, T, H, D, seed, noalloc=True)
        for name, a, b in zip(("dg", "dA_log", "ddt_bias"), got, want):
            assert torch.equal(a, b), (name, rel_l2(a, b))


def test_noalloc_gate_backward_packed_documents(dev):
    """Packed documents: the launch bound counts empty chunk slots, whose
    partials are written as zeros on every call."""
    cu = torch.tensor([0, 17, 17, 100, 164, 300, 301], dtype=torch.int32)
    print("[gpu] gate bwd noalloc packed", flush=True)
    _run(dev, 1, 1024, 8, 128, 5, noalloc=True)  # leave other values in the scratch
    want = _run(dev, 1, 301, 4, 64, 6, noalloc=False, cu=cu)
    got = _run(dev, 1, 301, 4, 64, 6, noalloc=True, cu=cu)
    for name, a, b in zip(("dg", "dA_log", "ddt_bias"), got, want):
        assert torch.equal(a, b), (name, rel_l2(a, b))

