"""The C ABI library loads, exports every declared entry point and agrees
with its ctypes mirror -- no compute, so this runs without a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "pkda_gfx950.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(pkda_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = _declared_functions()
    for required in ("pkda_abi_version", "pkda_last_error", "pkda_recurrent_fwd", "pkda_decode_step"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from delta_feedback_experiment_amd import _lib

    path = _lib.library_path()
    if not path.exists():
        pytest.fail(f"{path} missing: build it with python -m delta_feedback_experiment_amd.build")
    handle = ctypes.CDLL(str(path))
    for name in _declared_functions():
        assert hasattr(handle, name), name


def test_binding_structs_match_library():
    from delta_feedback_experiment_amd import _lib

    handle = _lib.lib()  # checks ABI version and every struct size it knows
    assert handle.pkda_abi_version() == _lib.ABI_VERSION
    assert handle.pkda_args_size(0) == ctypes.sizeof(_lib.RecurrentArgs)


def test_rejected_arguments_raise_before_any_launch():
    from delta_feedback_experiment_amd import _lib

    args = _lib.RecurrentArgs(dtype=0, num_seqs=1, seqlen=1, heads=1, head_dim=48)
    with pytest.raises(ValueError, match="head_dim 48"):
        _lib.call("pkda_recurrent_fwd", args, 0)
    args = _lib.RecurrentArgs(dtype=7, num_seqs=1, seqlen=1, heads=1, head_dim=64)
    with pytest.raises(ValueError, match="dtype"):
        _lib.call("pkda_recurrent_fwd", args, 0)
    args = _lib.RecurrentArgs(dtype=0, num_seqs=1, seqlen=2, heads=1, head_dim=64)
    with pytest.raises(ValueError, match="seqlen == 1"):
        _lib.call("pkda_decode_step", args, 0)
    # key gradients narrower than dq, dv: not a supported combination
    args = _lib.ChunkBwdArgs(dtype=_lib.PKDA_BF16, num_seqs=1, seqlen=64, heads=1, head_dim=64,
                             grad_dtype=_lib.PKDA_F32, key_grad_dtype=_lib.PKDA_BF16)
    with pytest.raises(ValueError, match="key_grad_dtype"):
        _lib.call("pkda_chunk_bwd", args, 0)


def test_operators_refuse_cpu_tensors():
    import torch

    from delta_feedback_experiment_amd import fused_recurrent_pkda

    q = torch.randn(1, 4, 1, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fused_recurrent_pkda(q, q, q, torch.zeros(1, 4, 1), torch.ones(1, 4, 1))


def test_noalloc_gate_backward_refuses_past_its_scratch():
    """pkda_gate_bwd_noalloc checks its size bound before any HIP call, so the
    refusal runs here, without a device; the pointers are never read."""
    from delta_feedback_experiment_amd import _lib

    H, D = 64, 128
    chunks = (1 << 22) // (H * (D + 1)) + 1  # one chunk past the 16 MiB array
    args = _lib.GateArgs(num_seqs=chunks, seqlen=64, heads=H, head_dim=D, gate_kind=_lib.GATE_RAW_CHANNEL,
                         g_dtype=_lib.PKDA_BF16, g=1, A_log=1, dt_bias=1, dgcum=1, dg=1, dA_log=1, ddt_bias=1,
                         num_chunks=chunks, dg_dtype=_lib.PKDA_F32)
    with pytest.raises(ValueError, match="exceeds its scratch"):
        _lib.call("pkda_gate_bwd_noalloc", args, 0)


def test_packed_triangular_refused_outside_its_configuration():
    """``tri_packed`` (Aqk and T as each chunk's ten lower blocks) is built for
    BF16 with a per-head gate and kw == k; both chunk entry points refuse any
    other combination before any HIP call, so this runs without a device
    (the pointers, nonzero stand-ins, are never read)."""
    from delta_feedback_experiment_amd import _lib

    geo = dict(num_seqs=1, seqlen=64, heads=1, head_dim=64, num_chunks=1)
    fake = dict(q=16, k=16, v=32, gcum=48, beta=64, u=96, aqk=112, akk=128, w=144, h=160)
    for dtype, kw in ((_lib.PKDA_F32, 16), (_lib.PKDA_BF16, 176)):  # FP32; a separate write key
        args = _lib.ChunkFwdArgs(dtype=dtype, **geo, kw=kw, o=80, tri_packed=1, **fake)
        with pytest.raises(ValueError, match="tri_packed"):
            _lib.call("pkda_chunk_fwd", args, 0)
    grads = dict(do=192, dh=208, du=224, dq=240, dk=256, dkw=272, dv=288, dbeta=304, dgcum=320)
    for dtype, kw in ((_lib.PKDA_F32, 16), (_lib.PKDA_BF16, 176)):
        args = _lib.ChunkBwdArgs(dtype=dtype, **geo, kw=kw, tri_packed=1, **fake, **grads)
        with pytest.raises(ValueError, match="tri_packed"):
            _lib.call("pkda_chunk_bwd", args, 0)
