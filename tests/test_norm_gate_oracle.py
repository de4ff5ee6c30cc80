"""The norm-gate oracle against what pins it, on the CPU: the library RMSNorm
(``torch.nn.functional.rms_norm``), the gate's closed forms (saturated gate =
plain RMSNorm, zero logit = half of it), the portable formula of
delta_feedback_experiment/pkda.py:542-547 in FP64, and scale invariance."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle import norm_gate_oracle as ng


def _inputs(seed=0, shape=(3, 5, 2, 64)):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen, dtype=torch.float64)
    g = torch.randn(*shape, generator=gen, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(shape[-1], generator=gen, dtype=torch.float64)
    return x, g, w


def test_matches_library_rms_norm_times_gate():
    x, g, w = _inputs()
    y, rstd = ng.norm_gate_reference(x, g, w, 1e-6, dtype=torch.float64)
    lib = F.rms_norm(x, (x.shape[-1],), w, eps=1e-6) * torch.sigmoid(g)
    assert torch.allclose(y, lib, atol=1e-12)
    assert torch.allclose(rstd.double(), torch.rsqrt(x.square().mean(-1) + 1e-6).reshape(-1), rtol=1e-6)


def test_gate_closed_forms():
    x, _, w = _inputs(1)
    plain = F.rms_norm(x, (x.shape[-1],), w, eps=1e-6)
    y_open, _ = ng.norm_gate_reference(x, torch.full_like(x, 60.0), w, 1e-6, dtype=torch.float64)
    y_half, _ = ng.norm_gate_reference(x, torch.zeros_like(x), w, 1e-6, dtype=torch.float64)
    assert torch.allclose(y_open, plain, atol=1e-12)
    assert torch.allclose(y_half, plain / 2, atol=1e-12)


def test_portable_formula_and_scale_invariance():
    x, g, w = _inputs(2)
    y, _ = ng.norm_gate_reference(x, g, w, 0.0, dtype=torch.float64)
    portable = x * torch.rsqrt(x.square().mean(-1, keepdim=True)) * w * torch.sigmoid(g)
    assert torch.allclose(y, portable, atol=1e-12)
    y3, _ = ng.norm_gate_reference(3.0 * x, g, w, 0.0, dtype=torch.float64)
    assert torch.allclose(y3, y, atol=1e-12)
