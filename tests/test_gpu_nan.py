"""An injected NaN: where it must reach and where it must not.

In the reference's token recurrence (``delta_feedback_experiment/pkda.py:
399-406``, evaluated per document, ``pkda.py:355-410``) a NaN in one token's
value enters the state at that token: that token's output and every later
output of the same head and document become NaN, and nothing else does --
other heads, other documents (the state restarts at each document) and other
sequences stay finite.  The slot-pool decode step updates each (slot, head)
on its own, so a NaN state in one slot reaches only that slot's output and
state.

* token-recurrent kernel: the NaN pattern equals the CPU oracle's exactly;
* chunked path (forward and backward, packed documents): every output the
  oracle has NaN is NaN, and everything outside the poisoned (document,
  head) -- outputs, final states and every gradient -- is finite.  Inside that
  document and head the chunked form may also mark earlier tokens of the same
  64-token chunk (its triangular products multiply the NaN row by zeros);
* decode: only the poisoned slot's (token, head) output and state are NaN;
  untouched slots keep their bits.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import pkda_oracle as oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _inputs(B, T, H, D, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    q = oracle.l2norm(torch.randn(B, T, H, D, generator=gen)).to(dtype)
    k = oracle.l2norm(torch.randn(B, T, H, D, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, D, generator=gen).to(dtype)
    g = -F.softplus(torch.randn(B, T, H, generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    return q, k, v, g, beta, gen


def test_recurrent_nan_reaches_exactly_the_later_tokens(dev):
    from delta_feedback_experiment_amd import fused_recurrent_pkda

    print("[gpu] NaN: token-recurrent kernel", flush=True)
    B, T, H, D = 3, 48, 3, 64
    q, k, v, g, beta, _ = _inputs(B, T, H, D, torch.float32, seed=71)
    v[1, 20, 1, 5] = float("nan")
    o_ref, S_ref = oracle.pkda_reference(q, k, v, g, beta, output_final_state=True)[:2]
    o, S, _ = fused_recurrent_pkda(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                   output_final_state=True)
    torch.cuda.synchronize()
    nan_ref = torch.isnan(o_ref).any(-1)
    assert bool(nan_ref[1, 20:, 1].all()) and int(nan_ref.sum()) == T - 20  # the reference's own pattern
    assert torch.equal(torch.isnan(o.cpu()).any(-1), nan_ref)
    assert torch.equal(torch.isnan(S.cpu()).any(-1).any(-1), torch.isnan(S_ref).any(-1).any(-1))


def test_chunked_nan_stays_in_its_document_and_head(dev):
    from delta_feedback_experiment_amd import chunk_pkda

    print("[gpu] NaN: chunked fwd+bwd, packed documents", flush=True)
    T, H, D = 300, 4, 64
    cu = torch.tensor([0, 100, 260, 300], dtype=torch.int32)
    q, k, v, g, beta, gen = _inputs(1, T, H, D, torch.bfloat16, seed=72)
    doc, head, tok = 1, 2, 130  # token 30 of document 1
    v[0, tok, head, 7] = float("nan")
    o_ref = oracle.pkda_reference(q.float(), k.float(), v.float(), g, beta, cu_seqlens=cu)[0]
    leaves = [t.to(dev).requires_grad_() for t in (q, k, v, g, beta)]
    o, S, _ = chunk_pkda(*leaves, output_final_state=True, cu_seqlens=cu.to(dev))
    do = torch.randn(o.shape, generator=gen).to(o.dtype).to(dev)
    grads = torch.autograd.grad([o], leaves, [do])
    torch.cuda.synchronize()

    inside = torch.zeros(1, T, H, dtype=torch.bool)
    inside[0, int(cu[doc]):int(cu[doc + 1]), head] = True
    nan_o = torch.isnan(o.float().cpu()).any(-1)
    nan_ref = torch.isnan(o_ref).any(-1)
    assert bool(nan_ref[0, tok:int(cu[doc + 1]), head].all())
    assert bool(nan_o[nan_ref].all()), "every output the reference has NaN is NaN"
    assert not bool(nan_o[~inside].any()), "NaN left its document and head"
    S_nan = torch.isnan(S.cpu()).any(-1).any(-1)  # [N, H]
    expect = torch.zeros_like(S_nan)
    expect[doc, head] = True
    assert torch.equal(S_nan, expect)
    for name, gval in zip(("dq", "dk", "dv", "dg", "dbeta"), grads):
        bad = torch.isnan(gval.float().cpu())
        if bad.dim() == 4:
            bad = bad.any(-1)
        assert not bool(bad[~inside].any()), f"{name}: NaN left its document and head"


def test_decode_nan_stays_in_its_slot(dev):
    from delta_feedback_experiment_amd import pkda_decode_step_

    print("[gpu] NaN: slot-pool decode", flush=True)
    P, N, H, D = 32, 12, 3, 128
    gen = torch.Generator().manual_seed(73)
    pool = 0.02 * torch.randn(P, H, D, D, generator=gen)
    slots = torch.randperm(P, generator=gen)[:N].to(torch.int32)
    bad_i, bad_h = 4, 1
    pool[int(slots[bad_i]), bad_h, 3, 9] = float("nan")
    q, k, v, g, beta, _ = _inputs(N, 1, H, D, torch.bfloat16, seed=74)
    q, k, v, g, beta = q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0]
    pool_d = pool.to(dev)
    o = pkda_decode_step_(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d, slots.to(dev))
    torch.cuda.synchronize()
    o_nan = torch.isnan(o.float().cpu()).any(-1)  # [N, H]
    expect = torch.zeros(N, H, dtype=torch.bool)
    expect[bad_i, bad_h] = True
    assert torch.equal(o_nan, expect)
    after = pool_d.cpu()
    s_nan = torch.isnan(after).any(-1).any(-1)  # [P, H]
    expect_s = torch.zeros(P, H, dtype=torch.bool)
    expect_s[int(slots[bad_i]), bad_h] = True
    assert torch.equal(s_nan, expect_s)
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[slots.long()] = False
    assert torch.equal(after[untouched], pool[untouched])
