"""The control-path oracle against what pins it, on the CPU.

* Split widths and order: the module's control_splits = (d, H, H, H, d)
  (delta_feedback_experiment/pkda.py:158-165); each slice is recovered from a
  packed row built with a distinct constant per slice.
* Closed forms: sigmoid(0) = 1/2; with A_log_p = dt_bias_p = logit = 0 the
  preconditioner decay is -ln 2; a large logit makes it -exp(A_log_p) logit
  (softplus's linear tail); a very negative one drives it to 0-.
* The decay expansion equals an explicit per-head product with decay_up's rows.
* Planted mistakes (beta and preconditioner-beta slices swapped, softplus
  without the bias) fail the checks above.
"""

from __future__ import annotations

import math

import torch

from oracle import controls_oracle as co


def _packed(d, H, values, rows=3):
    parts = [torch.full((rows, w), float(v), dtype=torch.float64) for w, v in zip(co.control_splits(d, H), values)]
    return torch.cat(parts, dim=-1)


def test_split_widths_and_order():
    d, H = 8, 3
    packed = _packed(d, H, (1, 2, 3, 4, 5))
    zeros = torch.zeros(H, dtype=torch.float64)
    hidden, beta, pdecay, pbeta, gate = co.controls_reference(packed, zeros, zeros, d, H)
    assert hidden.shape[-1] == d and gate.shape[-1] == d
    assert torch.all(hidden == 1) and torch.all(gate == 5)
    assert torch.allclose(beta, torch.full_like(beta, 1 / (1 + math.exp(-2))))
    assert torch.allclose(pbeta, torch.full_like(pbeta, 1 / (1 + math.exp(-4))))
    assert torch.allclose(pdecay, torch.full_like(pdecay, -math.log1p(math.exp(3))).float())


def test_closed_forms():
    d, H = 4, 2
    zeros = torch.zeros(H, dtype=torch.float64)
    _, beta, pdecay, pbeta, _ = co.controls_reference(_packed(d, H, (0, 0, 0, 0, 0)), zeros, zeros, d, H)
    assert torch.all(beta == 0.5) and torch.all(pbeta == 0.5)
    assert torch.allclose(pdecay.double(), torch.full((3, H), -math.log(2.0), dtype=torch.float64), atol=1e-7)
    A = torch.tensor([0.5, 1.5], dtype=torch.float64)
    _, _, big, _, _ = co.controls_reference(_packed(d, H, (0, 0, 30, 0, 0)), A, zeros, d, H)
    assert torch.allclose(big.double(), (-A.exp() * 30).expand(3, H), rtol=1e-6)
    _, _, small, _, _ = co.controls_reference(_packed(d, H, (0, 0, -40, 0, 0)), A, zeros, d, H)
    assert torch.all(small <= 0) and torch.all(small > -1e-15)


def test_decay_expansion_is_per_head_products():
    gen = torch.Generator().manual_seed(1)
    d, H = 8, 3
    packed = torch.randn(2, 5, 2 * d + 3 * H, generator=gen, dtype=torch.float64)
    up = torch.randn(H * d, d, generator=gen, dtype=torch.float64)
    zeros = torch.zeros(H, dtype=torch.float64)
    raw, *_ = co.controls_reference(packed, zeros, zeros, d, H, decay_up=up)
    hidden = packed[..., :d]
    for h in range(H):
        assert torch.allclose(raw[..., h, :], hidden @ up[h * d:(h + 1) * d].t(), atol=1e-12)


def test_planted_mistakes_fail():
    d, H = 4, 2
    packed = _packed(d, H, (0, 1, 2, 3, 0))
    zeros = torch.zeros(H, dtype=torch.float64)
    _, beta, pdecay, pbeta, _ = co.controls_reference(packed, zeros, zeros, d, H)
    swapped = torch.sigmoid(packed[..., d + 2 * H:d + 3 * H])  # the preconditioner's beta slice
    assert not torch.allclose(beta, swapped)
    dt = torch.full((H,), 0.7, dtype=torch.float64)
    _, _, with_bias, _, _ = co.controls_reference(packed, zeros, dt, d, H)
    assert not torch.allclose(with_bias, pdecay)
