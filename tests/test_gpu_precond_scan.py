"""The preconditioner scans with the chunk-decay hand-off against the scans
that sum the decays themselves, bit for bit.

With its ``chunk_decay`` workspace, each local chunk pass writes its chunk's
decay exp(sum g_atk), summed in token order with the document scan's
masking, and the scan reads it instead of loading and summing every chunk's
g_atk again.  Both forms give the same bits for every output: kw (and its
FP32 copy), the chunk checkpoints, the final A, and in the backward dk,
dg_atk, dbeta_atk, dcenter and dA_0.  The cases cover 64 chunks per row (one
scan block), 258 (several, the last one partial), packed documents mixing
empty, one-token, short and long ones, d = 32 (half the lanes idle), BF16
key gradients handed over narrow, and a slot-indexed pool updated in place.
Agreement with the oracle is the chunked and operator tests' part: they run
the hand-off form.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


CASES = {
    "equal rows, 64 chunks, bf16 narrow": dict(B=2, T=4096, H=4, D=128, dtype=torch.bfloat16, cu=None, narrow=True),
    "one row, 258 chunks": dict(B=1, T=16421, H=2, D=128, dtype=torch.bfloat16, cu=None, narrow=False),
    "packed, empty, short and long documents": dict(B=1, T=5000, H=3, D=64, dtype=torch.float32,
                                                    cu=[0, 17, 17, 100, 164, 300, 301, 301, 5000], narrow=False),
    "d32, partial last chunk": dict(B=3, T=150, H=2, D=32, dtype=torch.float32, cu=None, narrow=False),
}


def _inputs(B, T, H, D, dtype, N, seed):
    gen = torch.Generator().manual_seed(seed)
    k = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1).to(dtype)
    pA = torch.empty(H).uniform_(1, 16, generator=gen)
    pdt = torch.empty(H).uniform_(-6.9, -2.3, generator=gen).exp()
    pbias = pdt + torch.log(-torch.expm1(-pdt))
    g_atk = -pA * F.softplus(0.2 * torch.randn(B, T, H, generator=gen) + pbias)
    beta_atk = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    center = -0.2 + 0.1 * torch.randn(H, generator=gen)
    A0 = 0.1 * torch.randn(N, H, D, generator=gen).abs()
    dkw = torch.randn(B, T, H, D, generator=gen)
    dk = torch.randn(B, T, H, D, generator=gen)
    dA_T = torch.randn(N, H, D, generator=gen)
    return k, g_atk, beta_atk, center, A0, dkw, dk, dA_T


def _run(plan, d, narrow, handoff, kdtype):
    from delta_feedback_experiment_amd import precond as pre

    k, g_atk, beta_atk, center, A0, dkw, dk, dA_T = d
    kf = k.reshape(plan.num_tokens, plan.heads, plan.head_dim)
    st = pre.precond_forward(plan, kf, g_atk, beta_atk, center, 1.5, 1e-6, A0.clone(),
                             want_kw32=kdtype != torch.float32, handoff=handoff)
    shape = (plan.num_tokens, plan.heads, plan.head_dim)
    if narrow:
        dkw_in, dk_in = dkw.reshape(shape).to(kdtype), dk.reshape(shape).to(kdtype)
        dk_final = torch.empty_like(kf)
    else:
        dkw_in, dk_in, dk_final = dkw.reshape(shape).clone(), dk.reshape(shape).clone(), None
    dg_atk, dbeta_atk, dcenter, dA0 = pre.precond_backward(plan, kf, g_atk, beta_atk, center, 1.5, 1e-6, st,
                                                           dkw_in, dk_in, dA_T, True, dk_final=dk_final,
                                                           handoff=handoff)
    out = {"kw": st.kw, "a_chunk": st.a_chunk, "final_A": st.final_A,
           "dk": dk_final if narrow else dk_in, "dg_atk": dg_atk, "dbeta_atk": dbeta_atk,
           "dcenter": dcenter, "dA0": dA0}
    if st.kw32 is not None:
        out["kw32"] = st.kw32
    return out


@pytest.mark.parametrize("case", list(CASES))
def test_decay_handoff_matches_scan_sums_bitwise(dev, case):
    from delta_feedback_experiment_amd.chunk import ChunkPlan

    c = CASES[case]
    B, T, H, D, dtype = c["B"], c["T"], c["H"], c["D"], c["dtype"]
    cu = None if c["cu"] is None else torch.tensor(c["cu"], dtype=torch.int32, device=dev)
    N = B if cu is None else cu.numel() - 1
    print(f"[gpu] preconditioner decay hand-off vs scan sums: {case} (B{B} T{T} H{H} d{D} {dtype})", flush=True)
    d = [x.to(dev) for x in _inputs(B, T, H, D, dtype, N, seed=5 + D)]
    plan = ChunkPlan.make(d[0], cu)
    # a packed launch's bound has empty chunk slots past the documents' chunks:
    # neither form writes their checkpoint rows (nothing reads them)
    real = slice(None) if plan.table is None else plan.table[2:4 * plan.num_chunks:4] > 0
    ref = _run(plan, d, c["narrow"], False, dtype)
    got = _run(plan, d, c["narrow"], True, dtype)
    ref["a_chunk"], got["a_chunk"] = ref["a_chunk"][real], got["a_chunk"][real]
    torch.cuda.synchronize()
    for name, r in ref.items():
        assert torch.isfinite(r).all(), (name, "not finite")
        assert torch.equal(got[name], r), (case, name, (got[name].float() - r.float()).abs().max().item())
    print(f"  {len(ref)} outputs bitwise equal, {plan.num_chunks} chunks", flush=True)


def test_slot_pool_in_place_scans(dev):
    """Slot-indexed prefill updates the A pool in place (start and final A in
    the same rows); with or without the hand-off it gives the same pool, and
    rows of no document (and the empty document's) keep their values."""
    from delta_feedback_experiment_amd import precond as pre
    from delta_feedback_experiment_amd.chunk import ChunkPlan

    print("[gpu] preconditioner scans with and without the hand-off, pool updated in place", flush=True)
    H, D, P = 4, 128, 6
    cu = torch.tensor([0, 1300, 1301, 4000, 4000], dtype=torch.int32, device=dev)
    slot = torch.tensor([4, 0, 2, 5], dtype=torch.int32, device=dev)
    k, g_atk, beta_atk, center, _, _, _, _ = _inputs(1, 4000, H, D, torch.bfloat16, 4, seed=77)
    pool0 = 0.1 * torch.randn(P, H, D, generator=torch.Generator().manual_seed(3)).abs()
    k, g_atk, beta_atk, center, pool0 = (x.to(dev) for x in (k, g_atk, beta_atk, center, pool0))
    plan = ChunkPlan.make(k, cu)
    kf = k.reshape(plan.num_tokens, H, D)
    outs = []
    for handoff in (False, True):
        pool = pool0.clone()
        st = pre.precond_forward(plan, kf, g_atk, beta_atk, center, 1.5, 1e-6, pool, slot_idx=slot,
                                 final_A=pool, handoff=handoff)
        outs.append((pool, st.kw, st.a_chunk))
    torch.cuda.synchronize()
    real = plan.table[2:4 * plan.num_chunks:4] > 0
    for name, a, b in zip(("pool", "kw", "a_chunk"), outs[1], outs[0]):
        if name == "a_chunk":
            a, b = a[real], b[real]
        assert torch.equal(a, b), name
    assert torch.equal(outs[0][0][[1, 3]], pool0[[1, 3]])  # rows of no document untouched
    assert torch.equal(outs[0][0][5], pool0[5])  # the empty document keeps its start A
