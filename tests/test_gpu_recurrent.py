"""Token-recurrent forward and slot-pool decode on the GPU vs the CPU oracle.

Tolerances (relative L2, ``||a-b|| / ||b||``): FP32 inputs <= 1e-5 against
the FP32 oracle on the same inputs; BF16 inputs <= 2e-2 against the FP32
oracle on the same BF16-rounded inputs.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import load_golden, rel_l2
from oracle import pkda_oracle as oracle

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


def _t(a):
    return torch.from_numpy(a).clone()


def _golden_call(gd, dev, fn_kwargs=None):
    from delta_feedback_experiment_amd import fused_recurrent_pkda

    x = {n: _t(gd[f"in_{n}"]) for n in ("q", "k", "v", "g_raw", "beta", "g_atk", "beta_atk")}
    S0 = _t(gd["in_S0"]).to(dev) if "in_S0" in gd else None
    A0 = _t(gd["in_A0"]).to(dev) if "in_A0" in gd else None
    o, S, A = fused_recurrent_pkda(
        x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), x["g_raw"].to(dev), x["beta"].to(dev),
        g_atk=x["g_atk"].to(dev), beta_atk=x["beta_atk"].to(dev),
        A_log=_t(gd["in_A_log"]).to(dev), dt_bias=_t(gd["in_dt_bias"]).to(dev), use_gate_in_kernel=True,
        scale=float(gd["scale"]), initial_state=S0, initial_A_state=A0, output_final_state=True,
        x=float(gd["squash_x"]), eps=float(gd["squash_eps"]), log_atk_scale=_t(gd["in_center"]).to(dev),
    )
    return o, S, A


@pytest.mark.parametrize("name", ["c1_fwd", "c1_grad", "prod_grad", "decode_t1"])
def test_recurrent_matches_reference_golden(dev, name):
    print(f"[gpu] recurrent golden {name}", flush=True)
    gd = load_golden(name)
    o, S, A = _golden_call(gd, dev)
    torch.cuda.synchronize()
    assert rel_l2(o, _t(gd["out_o"])) < FP32_TOL
    assert rel_l2(S, _t(gd["out_S"])) < FP32_TOL
    assert rel_l2(A, _t(gd["out_A"])) < FP32_TOL


def _inputs(B, T, H, D, dtype, seed=0, per_channel=False, strong=False):
    gen = torch.Generator().manual_seed(seed)

    def randn(*s):
        return torch.randn(*s, generator=gen)

    q = oracle.l2norm(randn(B, T, H, D)).to(dtype)
    k = oracle.l2norm(randn(B, T, H, D)).to(dtype)
    v = randn(B, T, H, D).to(dtype)
    beta = torch.sigmoid(randn(B, T, H))
    g = -F.softplus(randn(B, T, H, D) if per_channel else randn(B, T, H))
    if strong:
        mask = torch.rand(B, T, generator=gen) < 0.1
        g = torch.where(mask[:, :, None] if g.dim() == 3 else mask[:, :, None, None], torch.full_like(g, -8.0), g)
    return q, k, v, g, beta


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("per_channel", [False, True])
def test_recurrent_matches_oracle(dev, D, dtype, per_channel):
    print(f"[gpu] recurrent D={D} {dtype} per_channel={per_channel}", flush=True)
    from delta_feedback_experiment_amd import fused_recurrent_pkda

    B, T, H = 2, 67, 3
    q, k, v, g, beta = _inputs(B, T, H, D, dtype, seed=D, per_channel=per_channel, strong=True)
    S0 = 0.02 * torch.randn(B, H, D, D)
    o_ref, S_ref, _ = oracle.pkda_reference(q, k, v, g, beta, initial_state=S0, output_final_state=True,
                                            out_dtype=torch.float32)
    o, S, A = fused_recurrent_pkda(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                   initial_state=S0.to(dev), output_final_state=True)
    assert A is None and o.dtype == dtype
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    assert rel_l2(o.float(), o_ref) < tol
    assert rel_l2(S, S_ref) < tol


def test_recurrent_varlen_resets_state_per_document(dev):
    print("[gpu] recurrent varlen", flush=True)
    from delta_feedback_experiment_amd import fused_recurrent_pkda

    D, H = 64, 2
    cu = torch.tensor([0, 17, 17, 100, 164, 170], dtype=torch.int32)
    q, k, v, g, beta = _inputs(1, 170, H, D, torch.float32, seed=5)
    S0 = 0.02 * torch.randn(5, H, D, D)
    o_ref, S_ref, _ = oracle.pkda_reference(q, k, v, g, beta, initial_state=S0, output_final_state=True, cu_seqlens=cu)
    o, S, _ = fused_recurrent_pkda(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                   initial_state=S0.to(dev), output_final_state=True, cu_seqlens=cu.to(dev))
    assert rel_l2(o, o_ref) < FP32_TOL
    assert rel_l2(S, S_ref) < FP32_TOL
    assert torch.equal(S[1].cpu(), S0[1])  # empty document


@pytest.mark.parametrize("precond", [False, True])
def test_decode_step_pool_matches_oracle(dev, precond):
    print(f"[gpu] decode precond={precond}", flush=True)
    from delta_feedback_experiment_amd import pkda_decode_step_

    P, N, H, D = 96, 40, 4, 128
    gen = torch.Generator().manual_seed(11)
    pool = 0.02 * torch.randn(P, H, D, D, generator=gen)
    a_pool = 0.1 * torch.randn(P, H, D, generator=gen).abs()
    slots = torch.randperm(P, generator=gen)[:N].to(torch.int32)
    q, k, v, g, beta = _inputs(N, 1, H, D, torch.bfloat16, seed=12)
    q, k, v, g, beta = q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0]
    extra = {}
    if precond:
        extra = dict(g_atk=-F.softplus(torch.randn(N, H, generator=gen)),
                     beta_atk=torch.sigmoid(torch.randn(N, H, generator=gen)),
                     log_atk_scale=torch.full((H,), -0.2), x=1.5)
    pool_ref = pool.clone()
    a_ref = a_pool.clone()
    o_ref = oracle.decode_step_reference(q, k, v, g, beta, pool_ref, slots,
                                         a_pool=a_ref if precond else None, **extra)
    pool_d = pool.to(dev)
    a_d = a_pool.to(dev)
    o = pkda_decode_step_(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d, slots.to(dev),
                          a_pool=a_d if precond else None, check_slots=True,
                          **{kk: (vv.to(dev) if torch.is_tensor(vv) else vv) for kk, vv in extra.items()})
    torch.cuda.synchronize()
    assert rel_l2(o.float(), o_ref.float()) < BF16_TOL
    assert rel_l2(pool_d.cpu()[slots.long()], pool_ref[slots.long()]) < FP32_TOL
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[slots.long()] = False
    assert torch.equal(pool_d.cpu()[untouched], pool[untouched])
    if precond:
        assert rel_l2(a_d.cpu()[slots.long()], a_ref[slots.long()]) < FP32_TOL
        assert torch.equal(a_d.cpu()[untouched], a_pool[untouched])


@pytest.mark.parametrize("D,dtype,g_form,slots_given", [
    (32, torch.float32, "channel", True),    # 256-thread items, half a wave of channels
    (64, torch.bfloat16, "channel_bf16", False),  # slots 0..N-1 (slot_idx None), g in BF16
    (128, torch.bfloat16, "head", False),
])
def test_decode_step_input_forms_match_oracle(dev, D, dtype, g_form, slots_given):
    """The decode step reads each item's inputs one item ahead: the uniform
    ones (slot, beta, the preconditioner's per-token and per-head values) by
    scalar loads, the per-channel ones as raw bits widened where used.  Every
    form of those inputs against the oracle: FP32 and BF16 activations, a
    per-head or per-channel log decay in FP32 or BF16, with and without
    slot indices, d = 32 / 64 / 128, the preconditioner on, over enough
    items that every workgroup walks several."""
    from delta_feedback_experiment_amd import pkda_decode_step_

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 16
    N = -(-3 * 12 * cus // H)  # about three items per workgroup
    P = N + 7 if slots_given else N
    assert N * H > 12 * cus
    print(f"[gpu] decode input forms D={D} {dtype} g={g_form} slots={slots_given} items={N * H}", flush=True)
    gen = torch.Generator().manual_seed(300 + D)
    pool = 0.02 * torch.randn(P, H, D, D, generator=gen)
    a_pool = 0.1 * torch.randn(P, H, D, generator=gen).abs()
    slots = torch.randperm(P, generator=gen)[:N].to(torch.int32) if slots_given else torch.arange(N, dtype=torch.int32)
    q, k, v, g, beta = _inputs(N, 1, H, D, dtype, seed=301, per_channel=g_form != "head")
    q, k, v, g, beta = q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0]
    if g_form == "channel_bf16":
        g = g.to(torch.bfloat16)
    extra = dict(g_atk=-F.softplus(torch.randn(N, H, generator=gen)),
                 beta_atk=torch.sigmoid(torch.randn(N, H, generator=gen)),
                 log_atk_scale=-0.2 + 0.1 * torch.randn(H, generator=gen), x=1.5)
    pool_ref, a_ref = pool.clone(), a_pool.clone()
    o_ref = oracle.decode_step_reference(q, k, v, g.float(), beta, pool_ref, slots, a_pool=a_ref, **extra)
    pool_d, a_d = pool.to(dev), a_pool.to(dev)
    o = pkda_decode_step_(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d,
                          slots.to(dev) if slots_given else None, a_pool=a_d,
                          **{kk: (vv.to(dev) if torch.is_tensor(vv) else vv) for kk, vv in extra.items()})
    torch.cuda.synchronize()
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    sl = slots.long()
    assert rel_l2(o.float(), o_ref.float()) < tol
    assert rel_l2(pool_d.cpu()[sl], pool_ref[sl]) < FP32_TOL
    assert rel_l2(a_d.cpu()[sl], a_ref[sl]) < FP32_TOL
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[sl] = False
    assert torch.equal(pool_d.cpu()[untouched], pool[untouched])


@pytest.mark.parametrize("P,N,H,D,precond", [
    (512, 256, 32, 128, False),   # 8,192 (slot, head) items
    (512, 256, 32, 128, True),
    (256, 200, 32, 64, True),     # D = 64: 6,400 items
])
def test_decode_step_pool_full_size_matches_oracle(dev, P, N, H, D, precond):
    """The decode pool at the benchmark's own size.  The kernel's grid stops
    at 12 workgroups per compute unit (3,072 on 256 CUs); past that each
    workgroup walks several (slot, head) items and hands the next item's
    prefetched state and inputs over to the next iteration.  Three steps in a
    row, each with a fresh random slot subset, each checked against the
    oracle's step on the same pool, with every other slot bitwise unchanged."""
    from delta_feedback_experiment_amd import pkda_decode_step_

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert N * H > 12 * cus, "the case must exercise the multi-item path"
    print(f"[gpu] decode full size P={P} N={N} H={H} D={D} precond={precond} items={N * H}", flush=True)
    gen = torch.Generator().manual_seed(1000 + D + int(precond))
    pool = 0.02 * torch.randn(P, H, D, D, generator=gen)
    a_pool = 0.1 * torch.randn(P, H, D, generator=gen).abs()
    pool_d = pool.to(dev)
    a_d = a_pool.to(dev)
    center = torch.full((H,), -0.2)
    for step in range(3):
        slots = torch.randperm(P, generator=gen)[:N].to(torch.int32)
        q, k, v, g, beta = _inputs(N, 1, H, D, torch.bfloat16, seed=2000 + step)
        q, k, v, g, beta = q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0]
        extra = {}
        if precond:
            extra = dict(g_atk=-F.softplus(torch.randn(N, H, generator=gen)),
                         beta_atk=torch.sigmoid(torch.randn(N, H, generator=gen)),
                         log_atk_scale=center, x=1.5)
        before = pool.clone()
        a_before = a_pool.clone()
        o_ref = oracle.decode_step_reference(q, k, v, g, beta, pool, slots,
                                             a_pool=a_pool if precond else None, **extra)
        o = pkda_decode_step_(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d, slots.to(dev),
                              a_pool=a_d if precond else None,
                              **{kk: (vv.to(dev) if torch.is_tensor(vv) else vv) for kk, vv in extra.items()})
        torch.cuda.synchronize()
        got = pool_d.cpu()
        sl = slots.long()
        untouched = torch.ones(P, dtype=torch.bool)
        untouched[sl] = False
        e_o = rel_l2(o.float(), o_ref.float())
        e_s = rel_l2(got[sl], pool[sl])
        print(f"  step {step}: o={e_o:.2e} S={e_s:.2e}", flush=True)
        assert e_o < BF16_TOL
        assert e_s < FP32_TOL
        assert torch.equal(got[untouched], before[untouched])
        if precond:
            a_got = a_d.cpu()
            assert rel_l2(a_got[sl], a_pool[sl]) < FP32_TOL
            assert torch.equal(a_got[untouched], a_before[untouched])
        # carry the GPU's pool forward so later steps start from the same state
        pool.copy_(got)
        if precond:
            a_pool.copy_(a_d.cpu())
        del got, before, a_before


def test_decode_rejects_repeated_slots(dev):
    from delta_feedback_experiment_amd import pkda_decode_step_

    q = torch.zeros(2, 1, 64, device=dev)
    with pytest.raises(ValueError, match="repeated"):
        pkda_decode_step_(q, q, q, torch.zeros(2, 1, device=dev), torch.zeros(2, 1, device=dev),
                          torch.zeros(4, 1, 64, 64, device=dev), torch.tensor([1, 1], dtype=torch.int32, device=dev),
                          check_slots=True)
