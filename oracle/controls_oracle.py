"""CPU restatement of the PKDA control path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product package never routes through it.

``PreconditionedKDA._controls`` (``delta_feedback_experiment/pkda.py:318-353``)
after its packed projection: the split into ``control_splits = (d, H, H, H, d)``
(``pkda.py:158-165``), the decay expansion ``raw = decay_hidden decay_up^T``
(``pkda.py:334-339``), ``beta = sigmoid``, ``precond_decay = -exp(A_log_p)
softplus(logit + dt_bias_p)`` evaluated in FP32, ``precond_beta = sigmoid``.
``tests/test_controls_oracle.py`` pins it with closed forms, the split widths
and planted mistakes; its gradients are autograd's.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor


def control_splits(head_dim: int, num_heads: int) -> tuple[int, int, int, int, int]:
    """Widths of the five control slices in packed order (pkda.py:158-164)."""
    return (head_dim, num_heads, num_heads, num_heads, head_dim)


def controls_reference(packed: Tensor, A_log_p: Tensor, dt_bias_p: Tensor, head_dim: int, num_heads: int,
                       decay_up: Tensor | None = None, dtype: torch.dtype | None = None):
    """``(decay, beta, precond_decay, precond_beta, output_gate_hidden)``.

    ``decay`` is the raw decay ``[..., H, d]`` when ``decay_up`` is given,
    else the decay hidden slice.  Arithmetic in ``dtype`` (default: packed's)
    except the preconditioner decay, which the reference evaluates in FP32
    (``pkda.py:344-346``); differentiable.
    """
    p = packed if dtype is None else packed.to(dtype)
    hidden, beta_l, pdecay_l, pbeta_l, gate_hidden = p.split(control_splits(head_dim, num_heads), dim=-1)
    decay = hidden
    if decay_up is not None:
        decay = F.linear(hidden, decay_up.to(hidden.dtype)).reshape(*p.shape[:-1], num_heads, head_dim)
    beta = torch.sigmoid(beta_l)
    precond_decay = -A_log_p.float().exp() * F.softplus(pdecay_l.float() + dt_bias_p.float())
    precond_beta = torch.sigmoid(pbeta_l)
    return decay, beta, precond_decay, precond_beta, gate_hidden
