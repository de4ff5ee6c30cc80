"""The whole PKDA mixer, composed the way ``PreconditionedKDA.forward``
composes it (``delta_feedback_experiment/pkda.py:477-559``), against the
reference module's own output and gradients (``tests/golden/module_fwd.npz``,
written from the reference's CPU path by ``tests/golden/make_golden.py``).

The composition: the Q/K/V projection GEMM, the fused short convolution +
SiLU + per-head L2 norm (pkda.py:197-220), the packed control projection and
its activations (pkda.py:318-353), the recurrence with the decay expansion and
the preconditioner, the output gate GEMM, RMSNorm with the sigmoid gate
(pkda.py:525-547) and the output projection.  GEMMs are ``F.linear`` in both
(the reference's ``sink_linear`` without sinks is one).

* CPU: the oracle's restatements of each piece composed -- pins them,
  together, to the reference module (FP32, relative L2 <= 1e-6).
* GPU (``gpu``): this package's operators composed -- conv, controls,
  ``chunk_pkda(decay_up=...)``, norm gate -- FP32, relative L2 <= 1e-5 on the
  output, final S and A and the gradients of x and every parameter, the
  decay's own (``A_log``, ``dt_bias``, ``decay_up``) included.  These inputs
  drive the chunk-local cumulative gate to |G| ~ 340 (``A_log`` up to
  log 16): the pair decays e^{G[t]-G[s]} are formed from the gate's FP64
  cumsum carried as two floats, since from the FP32 cumsum alone each
  difference carries ~2e-5 of rounding and ``dA_log`` (a signed sum of the
  gate gradient over a head) ends near 1e-5.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import load_golden, rel_l2

FP32_TOL = 1e-5
H, D = 2, 64


def _params(gd, device):
    return {k[len("param_"):]: torch.from_numpy(v).to(device).clone().requires_grad_()
            for k, v in gd.items() if k.startswith("param_")}


def compose(P, x, conv, controls, recurrence, norm_gate):
    """PreconditionedKDA.forward's dataflow over the given piece
    implementations; returns ``(out, S_T, A_T)``."""
    B, T, _ = x.shape
    HD = H * D
    qkv = F.linear(x, torch.cat([P["q_proj__weight"], P["k_proj__weight"], P["v_proj__weight"]]))
    w = torch.cat([P["q_conv__weight"].squeeze(1), P["k_conv__weight"].squeeze(1), P["v_conv__weight"].squeeze(1)])
    q, k, v = conv(qkv, w, D, 2 * HD, 1e-6)
    packed = F.linear(x, P["control_proj__weight"])
    hidden, beta, pdecay, pbeta, gate_hidden = controls(packed, P["A_log_precond"], P["dt_bias_precond"], D, H)
    shape = (B, T, H, D)
    o, S, A = recurrence(q.reshape(shape), k.reshape(shape), v.reshape(shape), hidden, beta, P["decay_up__weight"],
                         P["A_log"], P["dt_bias"], pdecay, pbeta, P["log_precond_center"])
    gate = F.linear(gate_hidden, P["output_gate_up__weight"], P["output_gate_up__bias"]).reshape(shape)
    mixed, _ = norm_gate(o, gate, P["output_norm"], 1e-6)
    return F.linear(mixed.flatten(-2), P["o_proj__weight"]), S, A


def _check(gd, out, S, A, x, P, tol):
    loss = ((out * torch.from_numpy(gd["cot_o"]).to(out.device)).sum()
            + (S * torch.from_numpy(gd["cot_S"]).to(S.device)).sum()
            + (A * torch.from_numpy(gd["cot_A"]).to(A.device)).sum())
    names = list(P)
    grads = torch.autograd.grad(loss, [x] + [P[n] for n in names])
    res = {"out": rel_l2(out, torch.from_numpy(gd["out_o"])), "S": rel_l2(S, torch.from_numpy(gd["out_S"])),
           "A": rel_l2(A, torch.from_numpy(gd["out_A"])),
           "dx": rel_l2(grads[0], torch.from_numpy(gd["grad_x"]))}
    for n, gval in zip(names, grads[1:]):
        res["d" + n] = rel_l2(gval, torch.from_numpy(gd["grad_" + n]))
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in res.items()), flush=True)
    for name, val in res.items():
        assert val < tol, (name, val)


def test_oracle_composition_matches_the_reference_module():
    from oracle import controls_oracle as co
    from oracle import norm_gate_oracle as no
    from oracle import pkda_oracle as oracle
    from oracle import qkv_conv_oracle as qo

    gd = load_golden("module_fwd")
    P = _params(gd, "cpu")
    x = torch.from_numpy(gd["in_x"]).clone().requires_grad_()

    def recurrence(q, k, v, hidden, beta, up, A_log, dt_bias, pdecay, pbeta, center):
        raw = F.linear(hidden, up).reshape(q.shape)
        return oracle.pkda_reference(q, k, v, raw, beta, A_log=A_log, dt_bias=dt_bias, use_gate_in_kernel=True,
                                     g_atk=pdecay, beta_atk=pbeta, log_atk_scale=center, x=1.5, eps=1e-6,
                                     output_final_state=True)

    out, S, A = compose(P, x, qo.qkv_conv_reference, co.controls_reference, recurrence, no.norm_gate_reference)
    _check(gd, out, S, A, x, P, 1e-6)


@pytest.mark.gpu
def test_gpu_operators_compose_to_the_reference_module():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from delta_feedback_experiment_amd import chunk_pkda, pkda_controls, pkda_norm_gate, pkda_qkv_conv

    print("[gpu] module composition vs the reference module", flush=True)
    dev = torch.device("cuda:0")
    gd = load_golden("module_fwd")
    P = _params(gd, dev)
    x = torch.from_numpy(gd["in_x"]).to(dev).requires_grad_()

    def recurrence(q, k, v, hidden, beta, up, A_log, dt_bias, pdecay, pbeta, center):
        return chunk_pkda(q, k, v, hidden, beta, decay_up=up, A_log=A_log, dt_bias=dt_bias, use_gate_in_kernel=True,
                          g_atk=pdecay, beta_atk=pbeta, log_atk_scale=center, x=1.5, eps=1e-6,
                          output_final_state=True)

    out, S, A = compose(P, x, pkda_qkv_conv, pkda_controls, recurrence, pkda_norm_gate)
    torch.cuda.synchronize()
    _check(gd, out, S, A, x, P, FP32_TOL)
