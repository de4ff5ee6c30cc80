"""Host-side argument checks that need no device."""

from __future__ import annotations

import pytest
import torch


@pytest.mark.parametrize("cu,ok", [
    ([0, 17, 17, 100, 164], True),
    ([0], False),                        # no documents but tokens
    ([0, 17, 9, 100, 164], False),       # a decrease
    ([5, 17, 40, 100, 164], False),      # cu[0] != 0
    ([0, 17, 40, 100, 150], False),      # ends before the packed length
    ([0, 17, 40, 100, 900], False),      # ends past it
    ([0, -30, 40, 2000, 90], False),     # negative and huge values
])
def test_validate_cu_seqlens(cu, ok):
    """The opt-in check behind ``check_cu_seqlens=True`` of ``chunk_pkda``,
    ``fused_recurrent_pkda`` and ``pkda_prefill_``: the same cases the chunk
    table flags on the device (tests/test_gpu_chunk.py)."""
    from delta_feedback_experiment_amd.chunk import validate_cu_seqlens

    cu_t = torch.tensor(cu, dtype=torch.int32)
    if ok:
        validate_cu_seqlens(cu_t, 164)
    else:
        with pytest.raises(ValueError, match="cu_seqlens"):
            validate_cu_seqlens(cu_t, 164)


def test_validate_cu_seqlens_empty_packing():
    from delta_feedback_experiment_amd.chunk import validate_cu_seqlens

    validate_cu_seqlens(torch.tensor([0], dtype=torch.int32), 0)
    validate_cu_seqlens(torch.tensor([0, 0, 0], dtype=torch.int32), 0)
