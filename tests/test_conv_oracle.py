"""The Q/K/V convolution oracle against what pins it, on the CPU.

* The reference's own formulation (delta_feedback_experiment/pkda.py:197-220):
  history-padded ``F.conv1d`` with ``groups = channels`` on ``[B, C, T]``,
  then SiLU -- a library routine; the oracle's explicit shifted sums must
  agree, which fixes the tap order and the causal offset.
* A single last tap is the identity: ``y = silu(w x[t])``.
* A single first tap is a pure delay by ``W - 1`` tokens.
* The normalised slabs have unit L2 norm per head (up to eps), the value slab
  is left unnormalised.
* Planted mistakes (taps reversed, a non-causal offset) fail the first check.
* Cached rows (a stored history in front of the projections): the reference's
  formulation with its conv state concatenated (pkda.py:205-219), and
  splitting a row anywhere -- the second piece continuing from the history the
  first one leaves -- reproduces the unsplit row exactly.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import qkv_conv_oracle as co


def _reference_formulation(x, weight):
    """pkda.py:203-220 restated with the library convolution: [B, T, C] -> silu(conv)."""
    C, W = weight.shape
    x_t = x.transpose(1, 2)
    combined = torch.cat((x_t.new_zeros(x.shape[0], C, W - 1), x_t), dim=-1)
    out = F.conv1d(combined, weight.unsqueeze(1), bias=None, groups=C).transpose(1, 2)
    return F.silu(out)


@pytest.mark.parametrize("W", [1, 2, 3, 4])
def test_shifted_sums_equal_the_grouped_convolution(W):
    gen = torch.Generator().manual_seed(W)
    x = torch.randn(2, 37, 24, generator=gen, dtype=torch.float64)
    w = torch.randn(24, W, generator=gen, dtype=torch.float64)
    got = co.causal_conv_silu(x, w, torch.float64)
    assert torch.allclose(got, _reference_formulation(x, w), atol=1e-12, rtol=0)


def test_single_taps_are_identity_and_delay():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 20, 8, generator=gen, dtype=torch.float64)
    last = torch.zeros(8, 4, dtype=torch.float64)
    last[:, 3] = 2.0
    assert torch.allclose(co.causal_conv_silu(x, last, torch.float64), F.silu(2.0 * x), atol=1e-14)
    first = torch.zeros(8, 4, dtype=torch.float64)
    first[:, 0] = 1.0
    delayed = torch.cat((x.new_zeros(1, 3, 8), x[:, :-3]), dim=1)
    assert torch.allclose(co.causal_conv_silu(x, first, torch.float64), F.silu(delayed), atol=1e-14)


def test_norm_slabs_are_unit_per_head_and_v_is_not_normalised():
    gen = torch.Generator().manual_seed(4)
    B, T, H, d = 2, 33, 3, 32
    P = H * d
    x = torch.randn(B, T, 3 * P, generator=gen, dtype=torch.float64)
    w = torch.randn(3 * P, 4, generator=gen, dtype=torch.float64)
    q, k, v = co.qkv_conv_reference(x, w, d, 2 * P, eps=0.0, dtype=torch.float64)
    for t in (q, k):
        norms = t.reshape(B, T, H, d).norm(dim=-1)
        assert torch.allclose(norms, torch.ones_like(norms), atol=1e-12)
    y = co.causal_conv_silu(x, w, torch.float64)
    assert torch.equal(v, y[..., 2 * P:])


@pytest.mark.parametrize("mistake", ["reversed_taps", "non_causal"])
def test_planted_mistakes_fail(mistake):
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(1, 16, 8, generator=gen, dtype=torch.float64)
    w = torch.randn(8, 4, generator=gen, dtype=torch.float64)
    if mistake == "reversed_taps":
        got = co.causal_conv_silu(x, w.flip(1), torch.float64)
    else:
        padded = torch.cat((x, x.new_zeros(1, 3, 8)), dim=1)  # future instead of history
        got = F.silu(sum(w[:, i] * padded[:, i:i + 16] for i in range(4)))
    assert not torch.allclose(got, _reference_formulation(x, w), atol=1e-6)


def _reference_with_state(x, weight, state):
    """pkda.py:203-219 with a conv state [B, C, W - 1]: cat(state, x_t), then conv1d."""
    C, W = weight.shape
    combined = torch.cat((state, x.transpose(1, 2)), dim=-1)
    out = F.conv1d(combined, weight.unsqueeze(1), bias=None, groups=C).transpose(1, 2)
    return F.silu(out), combined[..., -(W - 1):]


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("T", [1, 2, 9])
def test_history_matches_the_reference_conv_state(W, T):
    gen = torch.Generator().manual_seed(10 * W + T)
    x = torch.randn(2, T, 12, generator=gen, dtype=torch.float64)
    w = torch.randn(12, W, generator=gen, dtype=torch.float64)
    hist = torch.randn(2, W - 1, 12, generator=gen, dtype=torch.float64)
    want, state = _reference_with_state(x, w, hist.transpose(1, 2))
    assert torch.allclose(co.causal_conv_silu(x, w, torch.float64, hist), want, atol=1e-12, rtol=0)
    assert torch.equal(co.history_after(x, hist, W), state.transpose(1, 2))


@pytest.mark.parametrize("split", [1, 2, 3, 17, 39])
def test_split_rows_continue_from_the_history(split):
    gen = torch.Generator().manual_seed(split)
    B, T, H, d, W = 2, 40, 2, 8, 4
    x = torch.randn(B, T, 3 * H * d, generator=gen, dtype=torch.float64)
    w = torch.randn(3 * H * d, W, generator=gen, dtype=torch.float64)
    whole = co.qkv_conv_reference(x, w, d, 2 * H * d, dtype=torch.float64)
    first = co.qkv_conv_reference(x[:, :split], w, d, 2 * H * d, dtype=torch.float64)
    hist = co.history_after(x[:, :split], None, W)
    second = co.qkv_conv_reference(x[:, split:], w, d, 2 * H * d, dtype=torch.float64, history=hist)
    for a, b, c in zip(whole, first, second):
        assert torch.equal(a, torch.cat((b, c), dim=1))
    assert torch.equal(co.history_after(x[:, split:], hist, W), x[:, -(W - 1):])


def test_planted_history_mistake_fails():
    """Oldest-last history order would still convolve, but not the same rows."""
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(1, 5, 6, generator=gen, dtype=torch.float64)
    w = torch.randn(6, 4, generator=gen, dtype=torch.float64)
    hist = torch.randn(1, 3, 6, generator=gen, dtype=torch.float64)
    want, _ = _reference_with_state(x, w, hist.transpose(1, 2))
    assert not torch.allclose(co.causal_conv_silu(x, w, torch.float64, hist.flip(1)), want, atol=1e-6)
