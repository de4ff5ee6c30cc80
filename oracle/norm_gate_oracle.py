"""CPU restatement of the RMSNorm sigmoid output gate -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product package never routes through it.

The function is ``delta_feedback::pkda_norm_gate``
(``delta_feedback_experiment/fla_ops.py:572-593``): FLA's fused gated RMSNorm
with a sigmoid activation, whose portable form is
``x * rsqrt(mean(x^2) + eps) * output_norm * sigmoid(gate)``
(``delta_feedback_experiment/pkda.py:542-547``).  The fused path evaluates in
FP32 and rounds once; so does this restatement (the portable form also
rounds the normalised value to the activation dtype before the gate).
``tests/test_norm_gate_oracle.py`` pins it against ``torch.nn.functional.
rms_norm`` and closed forms of the gate.
"""

from __future__ import annotations

import torch
from torch import Tensor


def norm_gate_reference(x: Tensor, gate: Tensor, weight: Tensor, eps: float = 1e-6,
                        dtype: torch.dtype = torch.float32, out_dtype: torch.dtype | None = None,
                        ) -> tuple[Tensor, Tensor]:
    """``(y, rstd)``; differentiable in ``x``, ``gate`` and ``weight``."""
    xf, gf, wf = x.to(dtype), gate.to(dtype), weight.to(dtype)
    rstd = torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    y = xf * rstd * wf * torch.sigmoid(gf)
    return y.to(out_dtype or x.dtype), rstd.reshape(-1).detach().float()
