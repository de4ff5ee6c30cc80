"""Pin the CPU oracle before it judges the HIP path.

* Golden vectors written from the reference's own ``_portable_recurrence``
  (``tests/golden/make_golden.py``): outputs, final states and every gradient.
* Closed forms and invariants that fix the recurrence independently of any
  restatement: the zero-write limit, associative recall with orthonormal keys,
  the constant preconditioner, state carry across a split, per-document
  independence for packed rows, per-row independence.
* An FP64 chunk-form evaluation (``oracle.pkda_chunk_oracle``) that must equal
  the FP64 literal loop to ~1e-12.
* Planted mistakes (in the oracle, on the CPU) that the golden vectors reject.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from conftest import load_golden, rel_l2
from oracle import pkda_chunk_oracle as chunk_oracle
from oracle import pkda_oracle as oracle


def _t(a, requires_grad=False):
    return torch.from_numpy(a).clone().requires_grad_(requires_grad)


def _golden_inputs(gd, requires_grad=False):
    names = ["q", "k", "v", "g_raw", "beta", "g_atk", "beta_atk"]
    x = {n: _t(gd[f"in_{n}"], requires_grad) for n in names}
    if "in_S0" in gd:
        x["S0"] = _t(gd["in_S0"], requires_grad)
        x["A0"] = _t(gd["in_A0"], requires_grad)
    x["A_log"] = _t(gd["in_A_log"], requires_grad)
    x["dt_bias"] = _t(gd["in_dt_bias"], requires_grad)
    x["center"] = _t(gd["in_center"], requires_grad)
    return x


def _run_oracle(gd, x, dtype=torch.float32):
    return oracle.pkda_reference(
        x["q"], x["k"], x["v"], x["g_raw"], x["beta"],
        g_atk=x["g_atk"], beta_atk=x["beta_atk"], A_log=x["A_log"], dt_bias=x["dt_bias"],
        use_gate_in_kernel=True, scale=float(gd["scale"]),
        initial_state=x.get("S0"), initial_A_state=x.get("A0"), output_final_state=True,
        x=float(gd["squash_x"]), eps=float(gd["squash_eps"]), log_atk_scale=x["center"],
        dtype=dtype,
    )


@pytest.mark.parametrize("name", ["c1_fwd", "c1_grad", "prod_grad", "decode_t1"])
def test_oracle_matches_reference_golden_forward(name):
    gd = load_golden(name)
    x = _golden_inputs(gd)
    o, S, A = _run_oracle(gd, x)
    # Same FP32 operations as the reference; only einsum's reduction order may differ.
    assert rel_l2(o, _t(gd["out_o"])) < 2e-6
    assert rel_l2(S, _t(gd["out_S"])) < 2e-6
    assert rel_l2(A, _t(gd["out_A"])) < 2e-6


@pytest.mark.parametrize("name", ["c1_grad", "prod_grad"])
def test_oracle_gradients_match_reference_golden(name):
    gd = load_golden(name)
    x = _golden_inputs(gd, requires_grad=True)
    o, S, A = _run_oracle(gd, x)
    loss = (o * _t(gd["cot_o"])).sum() + (S * _t(gd["cot_S"])).sum() + (A * _t(gd["cot_A"])).sum()
    names = [n for n in x if f"grad_{n}" in gd]
    assert len(names) >= 10
    grads = torch.autograd.grad(loss, [x[n] for n in names])
    for n, g in zip(names, grads):
        assert rel_l2(g, _t(gd[f"grad_{n}"])) < 2e-5, n


def _random_case(B=2, T=70, H=2, K=16, V=16, seed=0, per_channel=True, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)

    def randn(*s):
        return torch.randn(*s, generator=gen, dtype=dtype)

    q = oracle.l2norm(randn(B, T, H, K))
    k = oracle.l2norm(randn(B, T, H, K))
    v = randn(B, T, H, V)
    g = -F.softplus(randn(B, T, H, K) if per_channel else randn(B, T, H))
    beta = torch.sigmoid(randn(B, T, H))
    g_atk = -F.softplus(randn(B, T, H))
    beta_atk = torch.sigmoid(randn(B, T, H))
    center = -0.2 + 0.1 * randn(H)
    S0 = 0.1 * randn(B, H, K, V)
    A0 = 0.1 * randn(B, H, K).abs()
    return dict(q=q, k=k, v=v, g=g, beta=beta, g_atk=g_atk, beta_atk=beta_atk,
                center=center, S0=S0, A0=A0)


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("squash_x", [1.0, 1.5])
def test_chunk_form_equals_literal_loop_fp64(per_channel, squash_x):
    c = _random_case(per_channel=per_channel)
    K = c["q"].shape[-1]
    o_ref, S_ref, A_ref = oracle.recurrence(
        c["q"], c["k"], c["v"], c["g"], c["beta"], scale=K ** -0.5,
        g_atk=c["g_atk"], beta_atk=c["beta_atk"], center=c["center"], squash_x=squash_x,
        state=c["S0"], a_state=c["A0"], dtype=torch.float64,
    )
    kw, A_T = chunk_oracle.precond_write_key(c["k"], c["g_atk"], c["beta_atk"], c["center"], squash_x, 1e-6, c["A0"])
    for chunk in (64, 16, 7):
        o, S = chunk_oracle.chunk_forward(c["q"], c["k"], kw, c["v"], c["g"], c["beta"], K ** -0.5, c["S0"], chunk=chunk)
        assert rel_l2(o, o_ref) < 1e-12
        assert rel_l2(S, S_ref) < 1e-12
    assert rel_l2(A_T, A_ref) < 1e-12


def test_zero_write_strength_is_pure_decay():
    """beta = 0: o_t = (diag(exp(G_t)) S0)^T (scale q_t) with G the inclusive cumsum."""
    c = _random_case(T=20)
    beta = torch.zeros_like(c["beta"])
    K = c["q"].shape[-1]
    o, S, _ = oracle.recurrence(c["q"], c["k"], c["v"], c["g"], beta, scale=K ** -0.5, state=c["S0"], dtype=torch.float64)
    G = c["g"].cumsum(1)  # [B,T,H,K]
    expect = torch.einsum("bthk,bhkv->bthv", c["q"] * K ** -0.5 * G.exp(), c["S0"])
    assert rel_l2(o, expect) < 1e-13
    assert rel_l2(S, G[:, -1, :, :, None].exp() * c["S0"]) < 1e-13


def test_orthonormal_keys_give_exact_associative_recall():
    """No decay, beta = 1, orthonormal keys: S_T^T k_i = v_i for every written key."""
    K = V = 16
    T = 10
    Qm, _ = torch.linalg.qr(torch.randn(K, K, dtype=torch.float64, generator=torch.Generator().manual_seed(3)))
    k = Qm[:T].reshape(1, T, 1, K)
    v = torch.randn(1, T, 1, V, dtype=torch.float64)
    g = torch.zeros(1, T, 1)
    beta = torch.ones(1, T, 1, dtype=torch.float64)
    # Reading with q = k right after the write returns exactly v (o_t = S_t^T k_t).
    o, S, _ = oracle.recurrence(k, k, v, g, beta, scale=1.0, dtype=torch.float64)
    assert torch.allclose(o, v, atol=1e-12)
    recall = torch.einsum("hkv,thk->thv", S[0], k[0])
    assert torch.allclose(recall, v[0], atol=1e-12)
    # Overwriting one key replaces exactly its value and leaves the others.
    k2 = torch.cat([k, k[:, 3:4]], 1)
    v2 = torch.cat([v, torch.randn(1, 1, 1, V, dtype=torch.float64)], 1)
    o2, S2, _ = oracle.recurrence(k2, k2, v2, torch.zeros(1, T + 1, 1), torch.ones(1, T + 1, 1, dtype=torch.float64), scale=1.0, dtype=torch.float64)
    recall2 = torch.einsum("hkv,thk->thv", S2[0], k[0])
    expect = v[0].clone()
    expect[3] = v2[0, -1]
    assert torch.allclose(recall2, expect, atol=1e-12)


def test_constant_preconditioner_when_its_write_is_zero():
    """beta_atk = 0 and A0 = 0 keep A = 0, so k_write = k * exp(-ln x r/(1+|r|)),
    r = ln(eps) - center, a constant per head (pkda.py:392-398)."""
    c = _random_case(T=12, per_channel=False)
    K = c["q"].shape[-1]
    x = 1.5
    eps = 1e-6
    o, S, A = oracle.recurrence(
        c["q"], c["k"], c["v"], c["g"], c["beta"], scale=K ** -0.5,
        g_atk=c["g_atk"], beta_atk=torch.zeros_like(c["beta_atk"]), center=c["center"],
        squash_x=x, squash_eps=eps, dtype=torch.float64,
    )
    r = math.log(eps) - c["center"]  # [H]
    Bfac = torch.exp(-math.log(x) * r / (1 + r.abs()))
    assert torch.all(A == 0)
    # Equivalent un-preconditioned recurrence: the write key is a per-head constant
    # multiple of k, i.e. beta scaled by that constant.
    o2, S2, _ = oracle.recurrence(
        c["q"], c["k"], c["v"], c["g"], c["beta"] * Bfac[None, None, :], scale=K ** -0.5,
        dtype=torch.float64,
    )
    assert rel_l2(o, o2) < 1e-13
    assert rel_l2(S, S2) < 1e-13
    assert torch.all((Bfac >= 2 / 3) & (Bfac <= 1.5))


def test_state_carry_across_a_split():
    c = _random_case(T=50)
    K = c["q"].shape[-1]
    kw = dict(scale=K ** -0.5, center=c["center"], squash_x=1.5, dtype=torch.float64)

    def run(sl, S0, A0):
        return oracle.recurrence(c["q"][:, sl], c["k"][:, sl], c["v"][:, sl], c["g"][:, sl], c["beta"][:, sl],
                                 g_atk=c["g_atk"][:, sl], beta_atk=c["beta_atk"][:, sl], state=S0, a_state=A0, **kw)

    o, S, A = run(slice(None), c["S0"], c["A0"])
    o1, S1, A1 = run(slice(0, 23), c["S0"], c["A0"])
    o2, S2, A2 = run(slice(23, None), S1, A1)
    assert rel_l2(torch.cat([o1, o2], 1), o) < 1e-13
    assert rel_l2(S2, S) < 1e-13
    assert rel_l2(A2, A) < 1e-13


def test_packed_documents_run_independently():
    c = _random_case(B=1, T=60)
    K = c["q"].shape[-1]
    cu = torch.tensor([0, 5, 5, 37, 60], dtype=torch.int32)
    S0 = 0.1 * torch.randn(4, 2, K, K, dtype=torch.float64)
    o, S, A = oracle.pkda_reference(
        c["q"], c["k"], c["v"], c["g"], c["beta"], g_atk=c["g_atk"], beta_atk=c["beta_atk"],
        log_atk_scale=c["center"], x=1.5, initial_state=S0, output_final_state=True,
        cu_seqlens=cu, dtype=torch.float64,
    )
    for n in range(4):
        a, b = int(cu[n]), int(cu[n + 1])
        on, Sn, An = oracle.recurrence(
            c["q"][:, a:b], c["k"][:, a:b], c["v"][:, a:b], c["g"][:, a:b], c["beta"][:, a:b],
            scale=K ** -0.5, g_atk=c["g_atk"][:, a:b], beta_atk=c["beta_atk"][:, a:b],
            center=c["center"], squash_x=1.5, state=S0[n : n + 1], dtype=torch.float64,
        )
        assert torch.equal(o[:, a:b], on)
        assert torch.equal(S[n : n + 1], Sn)
        assert torch.equal(A[n : n + 1], An)
    # An empty document returns its initial state untouched.
    assert torch.equal(S[1], S0[1])


def test_rows_are_independent():
    c = _random_case(B=3, T=30)
    K = c["q"].shape[-1]
    o, S, A = oracle.recurrence(c["q"], c["k"], c["v"], c["g"], c["beta"], scale=K ** -0.5,
                                g_atk=c["g_atk"], beta_atk=c["beta_atk"], center=c["center"], squash_x=1.5,
                                state=c["S0"], a_state=c["A0"], dtype=torch.float64)
    for b in range(3):
        sl = slice(b, b + 1)
        ob, Sb, Ab = oracle.recurrence(c["q"][sl], c["k"][sl], c["v"][sl], c["g"][sl], c["beta"][sl], scale=K ** -0.5,
                                       g_atk=c["g_atk"][sl], beta_atk=c["beta_atk"][sl], center=c["center"], squash_x=1.5,
                                       state=c["S0"][sl], a_state=c["A0"][sl], dtype=torch.float64)
        assert rel_l2(ob, o[sl]) < 1e-14 and rel_l2(Sb, S[sl]) < 1e-14


def test_decode_step_equals_single_token_run_and_leaves_other_slots():
    c = _random_case(B=3, T=1)
    K = c["q"].shape[-1]
    pool = 0.1 * torch.randn(7, 2, K, K, dtype=torch.float64)
    a_pool = 0.1 * torch.randn(7, 2, K, dtype=torch.float64).abs()
    before = pool.clone()
    a_before = a_pool.clone()
    slots = torch.tensor([4, 0, 6], dtype=torch.int32)
    o = oracle.decode_step_reference(
        c["q"][:, 0], c["k"][:, 0], c["v"][:, 0], c["g"][:, 0], c["beta"][:, 0], pool, slots,
        g_atk=c["g_atk"][:, 0], beta_atk=c["beta_atk"][:, 0], a_pool=a_pool,
        log_atk_scale=c["center"], x=1.5, dtype=torch.float64,
    )
    o_ref, S_ref, A_ref = oracle.recurrence(
        c["q"], c["k"], c["v"], c["g"], c["beta"], scale=K ** -0.5, g_atk=c["g_atk"], beta_atk=c["beta_atk"],
        center=c["center"], squash_x=1.5, state=before[slots.long()], a_state=a_before[slots.long()],
        dtype=torch.float64,
    )
    assert torch.equal(o, o_ref[:, 0])
    assert torch.equal(pool[slots.long()], S_ref)
    assert torch.equal(a_pool[slots.long()], A_ref)
    untouched = [1, 2, 3, 5]
    assert torch.equal(pool[untouched], before[untouched])
    assert torch.equal(a_pool[untouched], a_before[untouched])


# -- planted mistakes: the golden vectors must reject each of them -----------------


def _mutated_recurrence(mistake):
    def run(q, k, v, g_log, beta, *, scale, g_atk=None, beta_atk=None, center=None, squash_x=1.0,
            squash_eps=1e-6, state=None, a_state=None, dtype=torch.float32):
        B, T, H, K = q.shape
        q = q.to(dtype) * scale
        k, v = k.to(dtype), v.to(dtype)
        decay = g_log.to(dtype)
        a = a_state.to(dtype) if a_state is not None else q.new_zeros(B, H, K)
        S = state.to(dtype) if state is not None else q.new_zeros(B, H, K, v.shape[-1])
        outs = []
        for i in range(T):
            a = g_atk[:, i].exp()[..., None] * a + beta_atk[:, i][..., None] * k[:, i] ** 2
            r = torch.log(a + squash_eps) - center[None, :, None]
            sign = 1.0 if mistake == "squash_sign" else -1.0
            kw = k[:, i] * torch.exp(sign * math.log(squash_x) * r / (1 + r.abs()))
            Sd = S * decay[:, i].exp()[..., None]
            read = kw if mistake == "read_with_write_key" else k[:, i]
            e = v[:, i] - torch.einsum("bhkv,bhk->bhv", Sd, read)
            S_new = Sd + torch.einsum("bhk,bhv->bhkv", beta[:, i][..., None] * kw, e)
            outs.append(torch.einsum("bhk,bhkv->bhv", q[:, i], Sd if mistake == "read_old_state" else S_new))
            S = S_new
        return torch.stack(outs, 1), S, a
    return run


@pytest.mark.parametrize("mistake", ["read_with_write_key", "squash_sign", "read_old_state"])
def test_golden_vectors_reject_planted_mistakes(monkeypatch, mistake):
    gd = load_golden("prod_grad")
    x = _golden_inputs(gd)
    monkeypatch.setattr(oracle, "recurrence", _mutated_recurrence(mistake))
    o, S, A = _run_oracle(gd, x)
    assert rel_l2(o, _t(gd["out_o"])) > 1e-3 or rel_l2(S, _t(gd["out_S"])) > 1e-3
