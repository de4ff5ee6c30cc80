"""Slot-pool serving on the GPU: cached prefill into decode slots, the
convolution histories, and prefill followed by decode steps.

What pins each result:
* A prefill into pool slots runs the same kernels as ``chunk_pkda`` with
  explicit initial/final states, so its output and the slot contents must be
  bitwise those of that call; slots no sequence names stay bitwise untouched.
* A cached convolution row computes each position from the same inputs in the
  same order as the uncached kernel over the whole row, so prefill + decode
  tokens must reproduce ``pkda_qkv_conv`` of the whole row bitwise, and the
  slot must hold the row's last ``conv_size - 1`` projections.
* A prompt prefilled in two pieces, or prefilled and then decoded token by
  token, must match the CPU oracle over the whole sequence: relative L2
  <= 1e-5 for FP32 inputs, <= 2e-2 for BF16 inputs against the FP32 oracle on
  the same BF16-rounded inputs.
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2
from oracle import pkda_oracle as oracle
from oracle import qkv_conv_oracle as co
from test_gpu_chunk import _production_inputs, make_inputs

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


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_conv_cached_prefill_and_decode_equal_the_whole_row(dev, dtype, d):
    from delta_feedback_experiment_amd import pkda_qkv_conv, pkda_qkv_conv_cached_

    print(f"[gpu] conv cached {dtype} d={d}", flush=True)
    B, H, W, T1, steps, P = 3, 2, 4, 37, 5, 5
    C = 3 * H * d
    gen = torch.Generator().manual_seed(d)
    x = torch.randn(B, T1 + steps, C, generator=gen).to(dtype).to(dev)
    w = (0.5 * torch.randn(C, W, generator=gen)).to(dev)
    slots = torch.tensor([4, 0, 2], dtype=torch.int32, device=dev)
    pool = torch.randn(P, W - 1, C, generator=gen).to(dtype).to(dev)
    untouched = pool[[1, 3]].clone()
    whole = pkda_qkv_conv(x, w, d, 2 * H * d, 1e-6)
    outs = [pkda_qkv_conv_cached_(x[:, :T1], w, d, 2 * H * d, 1e-6, pool, slots, continue_state=False,
                                  check_slots=True)]
    for t in range(T1, T1 + steps):
        outs.append(pkda_qkv_conv_cached_(x[:, t:t + 1], w, d, 2 * H * d, 1e-6, pool, slots))
        assert torch.equal(pool[slots.long()], x[:, t + 1 - (W - 1):t + 1])
    torch.cuda.synchronize()
    for i, name in enumerate("qkv"):
        got = torch.cat([o[i] for o in outs], dim=1)
        assert torch.equal(got, whole[i]), name
    assert torch.equal(pool[[1, 3]], untouched)
    ref = co.qkv_conv_reference(x.cpu(), w.cpu(), d, 2 * H * d, 1e-6, out_dtype=torch.float32)
    err = max(rel_l2(whole[i].float(), ref[i]) for i in range(3))
    print(f"  whole row vs oracle {err:.2e}", flush=True)
    assert err < _tol(dtype)


def test_conv_short_continuation_keeps_older_history(dev):
    """Two new rows after a 3-row history: the slot keeps one old row."""
    from delta_feedback_experiment_amd import pkda_qkv_conv_cached_

    print("[gpu] conv short continuation", flush=True)
    B, H, d, W = 2, 1, 64, 4
    C = 3 * H * d
    gen = torch.Generator().manual_seed(3)
    hist = torch.randn(B, W - 1, C, generator=gen)
    x = torch.randn(B, 2, C, generator=gen)
    w = torch.randn(C, W, generator=gen)
    pool = hist.clone().to(dev)
    q, k, v = pkda_qkv_conv_cached_(x.to(dev), w.to(dev), d, 2 * H * d, 1e-6, pool)
    torch.cuda.synchronize()
    ref = co.qkv_conv_reference(x, w, d, 2 * H * d, 1e-6, history=hist, out_dtype=torch.float32)
    for a, b in zip((q, k, v), ref):
        assert rel_l2(a, b) < FP32_TOL
    assert torch.equal(pool.cpu(), co.history_after(x, hist, W))


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_prefill_into_slots_equals_chunk_pkda(dev, dtype, D):
    from delta_feedback_experiment_amd import chunk_pkda, pkda_prefill_

    print(f"[gpu] prefill into slots {dtype} D={D}", flush=True)
    B, T, H, P = 3, 150, 2, 6
    q, k, v, g, beta = (t.to(dev) for t in make_inputs(B, T, H, D, dtype, seed=D + 1, strong=True))
    slots = torch.tensor([5, 1, 3], dtype=torch.int32, device=dev)
    pool = torch.randn(P, H, D, D, device=dev)
    s_prev = pool[slots.long()].clone()
    untouched = pool[[0, 2, 4]].clone()
    o_ref, S_ref, _ = chunk_pkda(q, k, v, g, beta, output_final_state=True)
    o = pkda_prefill_(q, k, v, g, beta, pool, slots, check_slots=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(pool[slots.long()], S_ref)
    assert torch.equal(pool[[0, 2, 4]], untouched)
    # continuing from the slots equals explicit initial states
    o_ref2, S_ref2, _ = chunk_pkda(q, k, v, g, beta, initial_state=S_ref, output_final_state=True)
    o2 = pkda_prefill_(q, k, v, g, beta, pool, slots, continue_state=True)
    torch.cuda.synchronize()
    assert torch.equal(o2, o_ref2)
    assert torch.equal(pool[slots.long()], S_ref2)
    assert not torch.equal(pool[slots.long()], s_prev)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_prompt_in_two_pieces_matches_the_oracle(dev, dtype, D):
    """Production controls (raw per-channel gate, preconditioner x = 1.5):
    a 70-token piece then a 90-token piece continuing from the slots."""
    from delta_feedback_experiment_amd import DecodePool, pkda_prefill_

    print(f"[gpu] prefill two pieces {dtype} D={D}", flush=True)
    B, T1, T2, H = 2, 70, 90, 2
    (q, k, v, g_raw, beta, A_log, dt_bias, g_atk, beta_atk, center) = _production_inputs(B, T1 + T2, H, D, dtype,
                                                                                         41)
    o_ref, S_ref, A_ref = oracle.pkda_reference(q, k, v, g_raw, beta, A_log=A_log, dt_bias=dt_bias,
                                                use_gate_in_kernel=True, g_atk=g_atk, beta_atk=beta_atk,
                                                log_atk_scale=center, x=1.5, eps=1e-6, output_final_state=True,
                                                out_dtype=torch.float32)
    pool = DecodePool.zeros(4, H, D, conv_size=4, dtype=dtype, device=dev)
    slots = torch.tensor([2, 0], dtype=torch.int32, device=dev)
    ctl = dict(A_log=A_log.to(dev), dt_bias=dt_bias.to(dev), use_gate_in_kernel=True, log_atk_scale=center.to(dev),
               x=1.5, eps=1e-6)
    outs = []
    for sl, cont in ((slice(0, T1), False), (slice(T1, T1 + T2), True)):
        t = [x[:, sl].contiguous().to(dev) for x in (q, k, v, g_raw, beta, g_atk, beta_atk)]
        outs.append(pkda_prefill_(t[0], t[1], t[2], t[3], t[4], pool.state, slots, a_pool=pool.a, g_atk=t[5],
                                  beta_atk=t[6], continue_state=cont, **ctl))
    torch.cuda.synchronize()
    o = torch.cat(outs, dim=1)
    res = {"o": rel_l2(o.float(), o_ref), "S": rel_l2(pool.state[slots.long()], S_ref),
           "A": rel_l2(pool.a[slots.long()], A_ref)}
    print("  " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in res.items()), flush=True)
    for name, val in res.items():
        assert val < _tol(dtype), (name, val)


def test_packed_documents_into_slots(dev):
    from delta_feedback_experiment_amd import pkda_prefill_

    print("[gpu] prefill packed documents", flush=True)
    D, H, P = 64, 2, 8
    cu = torch.tensor([0, 17, 17, 100, 164, 300, 301], dtype=torch.int32)
    q, k, v, g, beta = make_inputs(1, 301, H, D, torch.float32, seed=6)
    slots = torch.tensor([7, 2, 5, 0, 3, 6], dtype=torch.int32)
    pool = 0.02 * torch.randn(P, H, D, D)
    S0 = pool[slots.long()].clone()
    o_ref, S_ref, _ = oracle.pkda_reference(q, k, v, g, beta, initial_state=S0, output_final_state=True,
                                            cu_seqlens=cu)
    pd = pool.to(dev)
    o = pkda_prefill_(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pd, slots.to(dev),
                      cu_seqlens=cu.to(dev), continue_state=True)
    torch.cuda.synchronize()
    res = {"o": rel_l2(o, o_ref), "S": rel_l2(pd[slots.long()], S_ref)}
    print("  " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in res.items()), flush=True)
    assert max(res.values()) < FP32_TOL
    assert torch.equal(pd[slots[1].long()].cpu(), S0[1])  # the empty document keeps its state
    assert torch.equal(pd[[1, 4]].cpu(), pool[[1, 4]])


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_prefill_then_decode_matches_the_oracle(dev, dtype, D):
    """Prefill 100 tokens into the slots, then decode 6 tokens in place."""
    from delta_feedback_experiment_amd import DecodePool, pkda_decode_step_, pkda_prefill_

    print(f"[gpu] prefill then decode {dtype} D={D}", flush=True)
    B, T, steps, H = 3, 100, 6, 2
    (q, k, v, g_raw, beta, A_log, dt_bias, g_atk, beta_atk, center) = _production_inputs(B, T + steps, H, D, dtype,
                                                                                         53)
    o_ref, S_ref, A_ref = oracle.pkda_reference(q, k, v, g_raw, beta, A_log=A_log, dt_bias=dt_bias,
                                                use_gate_in_kernel=True, g_atk=g_atk, beta_atk=beta_atk,
                                                log_atk_scale=center, x=1.5, eps=1e-6, output_final_state=True,
                                                out_dtype=torch.float32)
    pool = DecodePool.zeros(5, H, D, conv_size=4, dtype=dtype, device=dev)
    slots = torch.tensor([3, 4, 1], dtype=torch.int32, device=dev)
    ctl = dict(A_log=A_log.to(dev), dt_bias=dt_bias.to(dev), use_gate_in_kernel=True, log_atk_scale=center.to(dev),
               x=1.5, eps=1e-6)
    t = [x[:, :T].contiguous().to(dev) for x in (q, k, v, g_raw, beta, g_atk, beta_atk)]
    outs = [pkda_prefill_(t[0], t[1], t[2], t[3], t[4], pool.state, slots, a_pool=pool.a, g_atk=t[5],
                          beta_atk=t[6], **ctl)]
    for s in range(T, T + steps):
        t = [x[:, s].contiguous().to(dev) for x in (q, k, v, g_raw, beta, g_atk, beta_atk)]
        o = pkda_decode_step_(t[0], t[1], t[2], t[3], t[4], pool.state, slots, a_pool=pool.a, g_atk=t[5],
                              beta_atk=t[6], **ctl)
        outs.append(o[:, None])
    torch.cuda.synchronize()
    o = torch.cat(outs, dim=1)
    res = {"o": rel_l2(o.float(), o_ref), "o_decode": rel_l2(o[:, T:].float(), o_ref[:, T:]),
           "S": rel_l2(pool.state[slots.long()], S_ref), "A": rel_l2(pool.a[slots.long()], A_ref)}
    print("  " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in res.items()), flush=True)
    for name, val in res.items():
        assert val < _tol(dtype), (name, val)


def test_prefill_rejects_bad_slots(dev):
    from delta_feedback_experiment_amd import pkda_prefill_

    q, k, v, g, beta = (t.to(dev) for t in make_inputs(2, 64, 1, 64, torch.float32, seed=2))
    pool = torch.zeros(4, 1, 64, 64, device=dev)
    with pytest.raises(ValueError):
        pkda_prefill_(q, k, v, g, beta, pool, torch.tensor([1, 1], dtype=torch.int32, device=dev), check_slots=True)
    with pytest.raises(IndexError):
        pkda_prefill_(q, k, v, g, beta, pool, torch.tensor([0, 4], dtype=torch.int32, device=dev), check_slots=True)
    with pytest.raises(ValueError):
        pkda_prefill_(q, k, v, g, beta, pool, torch.tensor([0, 1], dtype=torch.int64, device=dev))


def test_serving_custom_ops_pass_opcheck(dev):
    """torch.library.opcheck on the three in-place serving ops with real
    launches: the schema's mutation marks match what the kernels write, and
    the fake implementations agree with the real ones in shape and dtype."""
    print("[gpu] serving ops opcheck", flush=True)
    gen = torch.Generator().manual_seed(7)
    N, P, H, D, T = 3, 6, 2, 64, 70
    q, k, v, g, beta = (t.to(dev) for t in make_inputs(N, T, H, D, torch.bfloat16, seed=3))
    pool = (0.02 * torch.randn(P, H, D, D, generator=gen)).to(dev)
    a_pool = (0.1 * torch.randn(P, H, D, generator=gen).abs()).to(dev)
    idx = torch.tensor([5, 1, 3], dtype=torch.int32, device=dev)
    g_atk = -torch.nn.functional.softplus(torch.randn(N, T, H, generator=gen)).to(dev)
    beta_atk = torch.sigmoid(torch.randn(N, T, H, generator=gen)).to(dev)
    center = torch.full((H,), -0.2, device=dev)
    o = torch.empty_like(v)
    utils = ("test_schema", "test_faketensor")
    torch.library.opcheck(torch.ops.pkda_mi355x.prefill_.default,
                          (q, k, v, g, beta, pool, idx, a_pool, False, None, g_atk, beta_atk, center, None, None,
                           False, D ** -0.5, 1.5, 1e-6, o), test_utils=utils)
    qd, kd, vd, gd, bd = (t[:, 0].contiguous() for t in (q, k, v, g, beta))
    od = torch.empty_like(vd)
    torch.library.opcheck(torch.ops.pkda_mi355x.decode_step_.default,
                          (qd, kd, vd, gd, bd, pool, idx, a_pool, g_atk[:, 0].contiguous(),
                           beta_atk[:, 0].contiguous(), center, None, None, False, D ** -0.5, 1.5, 1e-6, od),
                          test_utils=utils)
    C = 3 * H * D
    x = torch.randn(N, 5, C, generator=gen).to(torch.bfloat16).to(dev)
    w = (0.5 * torch.randn(C, 4, generator=gen)).to(dev)
    conv = torch.randn(P, 3, C, generator=gen).to(torch.bfloat16).to(dev)
    torch.library.opcheck(torch.ops.pkda_mi355x.qkv_conv_cached_.default,
                          (x, w, D, 2 * H * D, 1e-6, conv, idx, True), test_utils=utils)
