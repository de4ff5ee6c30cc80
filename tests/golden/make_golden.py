"""Write golden PKDA vectors from the reference's own portable recurrence.

Run in the development container only (``/root/reference`` does not exist on
the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports ``delta_feedback_experiment.pkda.PreconditionedKDA`` from the given
checkout, calls ``_portable_recurrence`` (pkda.py:355-410) on seeded CPU
inputs, and differentiates it with autograd for the gradient cases.  Only the
inputs and outputs are stored (``*.npz``, FP32); nothing of the reference is
copied.  Cases:

* ``c1_fwd``    -- B1 T256 H4 d64, squash_x=1, per-head decay broadcast over
                   channels with A_log=0, dt_bias=0 (so g = -softplus(n)).
* ``c1_grad``   -- B1 T128 H2 d64, the same mapping, with all gradients.
* ``prod_grad`` -- production PKDA (squash_x=1.5, per-channel raw gate,
                   nonzero S0/A0, T=80 not a multiple of 64), all gradients.
* ``decode_t1`` -- B3 T1 H2 d64 production step from nonzero S0/A0.
* ``module_fwd`` -- the whole mixer, ``PreconditionedKDA.forward``
                   (pkda.py:477-559) on its CPU path: B2 T80 hidden 96, H2
                   d64, squash_x=1.5, randomised parameters, the output, the
                   final S and A, and the gradients of x and every parameter.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def l2n(t):
    return t * torch.rsqrt(t.square().sum(-1, keepdim=True) + 1e-6)


def make_module(PreconditionedKDA, H, d, squash_x, A_log, dt_bias, center):
    m = PreconditionedKDA(hidden_size=8, num_heads=H, head_dim=d, squash_x=squash_x, squash_eps=1e-6)
    with torch.no_grad():
        m.A_log.copy_(A_log)
        m.dt_bias.copy_(dt_bias)
        m.log_precond_center.copy_(center)
    return m


def run_case(PreconditionedKDA, name, *, B, T, H, d, squash_x, seed, per_channel, nonzero_state, grads):
    gen = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float32)

    q = l2n(randn(B, T, H, d))
    k = l2n(randn(B, T, H, d))
    v = randn(B, T, H, d)
    beta = torch.sigmoid(randn(B, T, H))
    if per_channel:
        g_raw = randn(B, T, H, d)
        A_log = torch.empty(H).uniform_(1, 16, generator=gen).log()
        dt_bias = 0.1 * randn(H * d)
    else:
        n = randn(B, T, H)
        g_raw = n[..., None].expand(B, T, H, d).contiguous()
        A_log = torch.zeros(H)
        dt_bias = torch.zeros(H * d)
    pA = torch.empty(H).uniform_(1, 16, generator=gen)
    pdt = torch.empty(H).uniform_(math.log(0.001), math.log(0.1), generator=gen).exp()
    pbias = pdt + torch.log(-torch.expm1(-pdt))
    g_atk = -pA * F.softplus(0.2 * randn(B, T, H) + pbias)
    beta_atk = torch.sigmoid(randn(B, T, H))
    center = -0.2 + 0.1 * randn(H)
    if nonzero_state:
        S0 = 0.02 * randn(B, H, d, d)
        A0 = 0.1 * randn(B, H, d).abs()
    else:
        S0 = None
        A0 = None
    m = make_module(PreconditionedKDA, H, d, squash_x, A_log, dt_bias, center)
    leaves = dict(q=q, k=k, v=v, g_raw=g_raw, beta=beta, g_atk=g_atk, beta_atk=beta_atk)
    if S0 is not None:
        leaves.update(S0=S0, A0=A0)
    inputs = {key: val.clone().requires_grad_(grads) for key, val in leaves.items()}
    o, S, A = m._portable_recurrence(
        inputs["q"], inputs["k"], inputs["v"], inputs["g_raw"], inputs["beta"],
        inputs["g_atk"], inputs["beta_atk"], inputs.get("S0"), inputs.get("A0"), True,
    )
    out = {f"in_{key}": val.detach().numpy() for key, val in leaves.items()}
    out.update(
        in_A_log=A_log.numpy(), in_dt_bias=dt_bias.numpy(), in_center=center.numpy(),
        squash_x=np.float64(squash_x), squash_eps=np.float64(1e-6), scale=np.float64(d ** -0.5),
        out_o=o.detach().numpy(), out_S=S.detach().numpy(), out_A=A.detach().numpy(),
    )
    if grads:
        do = randn(*o.shape)
        dS = randn(*S.shape)
        dA = randn(*A.shape)
        loss = (o * do).sum() + (S * dS).sum() + (A * dA).sum()
        params = [m.A_log, m.dt_bias, m.log_precond_center]
        names = list(inputs)
        got = torch.autograd.grad(loss, [inputs[n] for n in names] + params)
        out.update(cot_o=do.numpy(), cot_S=dS.numpy(), cot_A=dA.numpy())
        for n, gval in zip(names + ["A_log", "dt_bias", "center"], got):
            out[f"grad_{n}"] = gval.numpy()
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print(name, {k: v.shape for k, v in out.items() if hasattr(v, "shape") and v.ndim})


def run_module_case(PreconditionedKDA, name, *, B, T, hidden, H, d, seed):
    torch.manual_seed(seed)
    m = PreconditionedKDA(hidden_size=hidden, num_heads=H, head_dim=d, squash_x=1.5, squash_eps=1e-6)
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():  # parameters the default init leaves trivial
        m.output_norm.copy_(1 + 0.3 * torch.randn(m.output_norm.shape, generator=gen))
        m.output_gate_up.bias.copy_(0.3 * torch.randn(m.output_gate_up.bias.shape, generator=gen))
        m.dt_bias.copy_(0.1 * torch.randn(m.dt_bias.shape, generator=gen))
        m.log_precond_center.copy_(-0.2 + 0.1 * torch.randn(H, generator=gen))
    x = torch.randn(B, T, hidden, generator=gen).requires_grad_()
    out, S, A, _conv = m(x, output_final_state=True)
    dout = torch.randn(out.shape, generator=gen)
    dS = torch.randn(S.shape, generator=gen)
    dA = torch.randn(A.shape, generator=gen)
    params = dict(m.named_parameters())
    loss = (out * dout).sum() + (S * dS).sum() + (A * dA).sum()
    got = torch.autograd.grad(loss, [x] + list(params.values()))
    rec = dict(in_x=x.detach().numpy(), out_o=out.detach().numpy(), out_S=S.detach().numpy(),
               out_A=A.detach().numpy(), cot_o=dout.numpy(), cot_S=dS.numpy(), cot_A=dA.numpy(),
               grad_x=got[0].numpy())
    for (n, prm), gval in zip(params.items(), got[1:]):
        key = n.replace(".", "__")
        rec[f"param_{key}"] = prm.detach().numpy()
        rec[f"grad_{key}"] = gval.numpy()
    np.savez_compressed(HERE / f"{name}.npz", **rec)
    print(name, sorted(k for k in rec if k.startswith("param_")))


def main():
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(root))
    from delta_feedback_experiment.pkda import PreconditionedKDA

    torch.set_num_threads(1)
    run_case(PreconditionedKDA, "c1_fwd", B=1, T=256, H=4, d=64, squash_x=1.0, seed=1,
             per_channel=False, nonzero_state=False, grads=False)
    run_case(PreconditionedKDA, "c1_grad", B=1, T=128, H=2, d=64, squash_x=1.0, seed=2,
             per_channel=False, nonzero_state=False, grads=True)
    run_case(PreconditionedKDA, "prod_grad", B=2, T=80, H=2, d=32, squash_x=1.5, seed=3,
             per_channel=True, nonzero_state=True, grads=True)
    run_case(PreconditionedKDA, "decode_t1", B=3, T=1, H=2, d=64, squash_x=1.5, seed=4,
             per_channel=True, nonzero_state=True, grads=False)
    run_module_case(PreconditionedKDA, "module_fwd", B=2, T=80, hidden=96, H=2, d=64, seed=5)


if __name__ == "__main__":
    main()
