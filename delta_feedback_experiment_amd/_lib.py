"""ctypes binding of ``libpkda_gfx950.so`` (the C ABI in ``include/pkda_gfx950.h``).

The structs below mirror the header field for field; ``check_abi`` compares
their sizes with the library's own ``pkda_args_size`` so a drifted mirror
fails at load time instead of passing garbage to a kernel.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_int64, c_void_p
from pathlib import Path

from .build import library_path

PKDA_F32 = 0
PKDA_BF16 = 1
GATE_LOG_HEAD = 0
GATE_LOG_CHANNEL = 1
GATE_RAW_CHANNEL = 2
GATE_LOW_RANK = 3
STAGE_FWD_INTRA = 1
STAGE_FWD_STATE = 2
STAGE_BWD_STATE = 1
STAGE_BWD_CHUNK = 2
ABI_VERSION = 13


class RecurrentArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("dtype", c_int32),
        ("num_seqs", c_int32), ("seqlen", c_int32), ("heads", c_int32), ("head_dim", c_int32),
        ("cu_seqlens", c_void_p),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("g", c_void_p),
        ("gate_kind", c_int32), ("g_dtype", c_int32),
        ("A_log", c_void_p), ("dt_bias", c_void_p), ("beta", c_void_p),
        ("scale", c_float),
        ("g_atk", c_void_p), ("beta_atk", c_void_p), ("center", c_void_p),
        ("squash_x", c_float), ("squash_eps", c_float),
        ("state_pool", c_void_p), ("a_pool", c_void_p), ("pool_size", c_int64),
        ("slot_idx", c_void_p), ("slot_idx_host", c_void_p), ("check_slots", c_int32),
        ("initial_state", c_void_p), ("initial_A_state", c_void_p),
        ("final_state", c_void_p), ("final_A_state", c_void_p),
        ("o", c_void_p),
    ]


class GateArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("num_seqs", c_int32), ("seqlen", c_int32),
        ("heads", c_int32), ("head_dim", c_int32), ("gate_kind", c_int32), ("g_dtype", c_int32),
        ("cu_seqlens", c_void_p), ("g", c_void_p), ("A_log", c_void_p), ("dt_bias", c_void_p),
        ("gcum", c_void_p), ("dgcum", c_void_p), ("dg", c_void_p), ("dA_log_part", c_void_p),
        ("ddt_bias_part", c_void_p), ("dA_log", c_void_p), ("ddt_bias", c_void_p),
        ("num_chunks", c_int32), ("table", c_void_p),
        ("up_weight", c_void_p), ("rank", c_int32), ("g_stride", c_int32), ("dg_dtype", c_int32),
        ("gcum_lo", c_void_p),
    ]


class PrecondArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("dtype", c_int32), ("num_seqs", c_int32), ("seqlen", c_int32),
        ("heads", c_int32), ("head_dim", c_int32), ("cu_seqlens", c_void_p),
        ("k", c_void_p), ("g_atk", c_void_p), ("beta_atk", c_void_p), ("center", c_void_p),
        ("squash_x", c_float), ("squash_eps", c_float),
        ("initial_A_state", c_void_p), ("final_A_state", c_void_p),
        ("kw", c_void_p), ("a_chunk", c_void_p), ("num_chunks", c_int32),
        ("dkw", c_void_p), ("dk", c_void_p), ("dg_atk", c_void_p), ("dbeta_atk", c_void_p),
        ("dcenter_part", c_void_p), ("dcenter", c_void_p), ("dA0", c_void_p), ("dA_T", c_void_p),
        ("table", c_void_p), ("slot_idx", c_void_p), ("pool_size", c_int64), ("lam_chunk", c_void_p),
        ("dk_final", c_void_p), ("kw32", c_void_p), ("grad_dtype", c_int32), ("chunk_decay", c_void_p),
    ]


_CHUNK_COMMON = [
    ("struct_size", c_int32), ("dtype", c_int32), ("num_seqs", c_int32), ("seqlen", c_int32),
    ("heads", c_int32), ("head_dim", c_int32), ("cu_seqlens", c_void_p), ("num_chunks", c_int32),
    ("table", c_void_p),
    ("q", c_void_p), ("k", c_void_p), ("kw", c_void_p), ("v", c_void_p),
    ("gcum", c_void_p), ("gate_per_channel", c_int32), ("beta", c_void_p), ("scale", c_float),
    ("initial_state", c_void_p),
]


class ChunkFwdArgs(ctypes.Structure):
    _fields_ = _CHUNK_COMMON + [
        ("final_state", c_void_p), ("o", c_void_p),
        ("w", c_void_p), ("u", c_void_p), ("aqk", c_void_p), ("akk", c_void_p), ("h", c_void_p),
        ("stages", c_int32), ("qg", c_void_p), ("kg", c_void_p),
        ("slot_idx", c_void_p), ("pool_size", c_int64), ("gcum_lo", c_void_p), ("tri_packed", c_int32),
    ]


class ChunkBwdArgs(ctypes.Structure):
    _fields_ = _CHUNK_COMMON + [
        ("w", c_void_p), ("u", c_void_p), ("aqk", c_void_p), ("akk", c_void_p), ("h", c_void_p),
        ("do", c_void_p), ("dht", c_void_p), ("dh", c_void_p), ("du", c_void_p),
        ("dq", c_void_p), ("dk", c_void_p), ("dkw", c_void_p), ("dv", c_void_p),
        ("dbeta", c_void_p), ("dgcum", c_void_p), ("dh0", c_void_p),
        ("stages", c_int32), ("qg", c_void_p), ("kg", c_void_p), ("grad_dtype", c_int32),
        ("key_grad_dtype", c_int32), ("kw32", c_void_p), ("gcum_lo", c_void_p), ("tri_packed", c_int32),
    ]


class QkvConvArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("dtype", c_int32), ("w_dtype", c_int32),
        ("batch", c_int32), ("seqlen", c_int32), ("width", c_int32), ("head_dim", c_int32),
        ("norm_channels", c_int32), ("conv_size", c_int32), ("eps", c_float),
        ("x", c_void_p), ("weight", c_void_p), ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("dq", c_void_p), ("dk", c_void_p), ("dv", c_void_p), ("dx", c_void_p), ("dw", c_void_p),
        ("dw_part", c_void_p), ("slot_idx", c_void_p), ("history_in", c_void_p), ("history_out", c_void_p),
        ("pool_size", c_int64),
    ]


class NormGateArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("dtype", c_int32), ("w_dtype", c_int32), ("dim", c_int32),
        ("rows", c_int64), ("eps", c_float),
        ("x", c_void_p), ("gate", c_void_p), ("weight", c_void_p), ("y", c_void_p), ("rstd", c_void_p),
        ("dy", c_void_p), ("dx", c_void_p), ("dgate", c_void_p), ("dw", c_void_p), ("dw_part", c_void_p),
    ]


class ControlsArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_int32), ("dtype", c_int32), ("rows", c_int64),
        ("heads", c_int32), ("rank", c_int32), ("gate_width", c_int32), ("row_stride", c_int32),
        ("packed", c_void_p), ("A_log_p", c_void_p), ("dt_bias_p", c_void_p),
        ("beta", c_void_p), ("precond_decay", c_void_p), ("precond_beta", c_void_p),
        ("d_decay_hidden", c_void_p), ("dbeta", c_void_p), ("dprecond_decay", c_void_p),
        ("dprecond_beta", c_void_p), ("d_gate_hidden", c_void_p),
        ("dpacked", c_void_p), ("part", c_void_p), ("dA_log_p", c_void_p), ("ddt_bias_p", c_void_p),
    ]


_ARG_KINDS = {0: RecurrentArgs, 1: GateArgs, 2: PrecondArgs, 3: ChunkFwdArgs, 4: ChunkBwdArgs, 5: QkvConvArgs,
              6: NormGateArgs, 7: ControlsArgs}
_LIB: ctypes.CDLL | None = None


class PkdaError(RuntimeError):
    """A call into the PKDA library failed; carries the library's status code."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} failed with status {status}: {message}")
        self.status = status


def _hip_runtimes_loaded() -> set[str]:
    found = set()
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                if "libamdhip64" in line:
                    found.add(line.split()[-1])
    except OSError:
        pass
    return found


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or mismatched."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path: Path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built; run `python -m delta_feedback_experiment_amd.build` "
            "(or __graft_entry__.build()). There is no CPU fallback."
        )
    import torch  # noqa: F401  -- the HIP runtime must be torch's, loaded first

    handle = ctypes.CDLL(str(path))
    handle.pkda_abi_version.restype = c_int32
    handle.pkda_last_error.restype = ctypes.c_char_p
    handle.pkda_args_size.restype = c_int64
    handle.pkda_args_size.argtypes = [c_int32]
    for name in ("pkda_recurrent_fwd", "pkda_decode_step"):
        fn = getattr(handle, name)
        fn.restype = c_int32
        fn.argtypes = [POINTER(RecurrentArgs), c_void_p]
    for name, struct in (
        ("pkda_gate_fwd", GateArgs), ("pkda_gate_bwd", GateArgs), ("pkda_gate_bwd_noalloc", GateArgs),
        ("pkda_precond_fwd", PrecondArgs), ("pkda_precond_bwd", PrecondArgs),
        ("pkda_chunk_fwd", ChunkFwdArgs), ("pkda_chunk_bwd", ChunkBwdArgs),
        ("pkda_qkv_conv_fwd", QkvConvArgs), ("pkda_qkv_conv_bwd", QkvConvArgs),
        ("pkda_norm_gate_fwd", NormGateArgs), ("pkda_norm_gate_bwd", NormGateArgs),
        ("pkda_controls_fwd", ControlsArgs), ("pkda_controls_bwd", ControlsArgs),
    ):
        fn = getattr(handle, name, None)
        if fn is not None:
            fn.restype = c_int32
            fn.argtypes = [POINTER(struct), c_void_p]
    handle.pkda_qkv_conv_workspace.restype = c_int64
    handle.pkda_qkv_conv_workspace.argtypes = [c_int32, c_int32, c_int32, c_int32]
    handle.pkda_norm_gate_workspace.restype = c_int64
    handle.pkda_norm_gate_workspace.argtypes = [c_int64, c_int32]
    handle.pkda_controls_workspace.restype = c_int64
    handle.pkda_controls_workspace.argtypes = [c_int64, c_int32]
    handle.pkda_chunk_table.restype = c_int32
    handle.pkda_chunk_table.argtypes = [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]
    if handle.pkda_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libpkda ABI {handle.pkda_abi_version()} != binding ABI {ABI_VERSION}")
    for kind, struct in _ARG_KINDS.items():
        size = handle.pkda_args_size(kind)
        if size >= 0 and size != ctypes.sizeof(struct):
            raise RuntimeError(f"{struct.__name__}: binding size {ctypes.sizeof(struct)} != library {size}")
    runtimes = _hip_runtimes_loaded()
    if len(runtimes) > 1:
        raise RuntimeError(f"more than one HIP runtime mapped: {sorted(runtimes)}")
    _LIB = handle
    return handle


def call(name: str, args: ctypes.Structure, stream: int) -> None:
    args.struct_size = ctypes.sizeof(args)
    status = getattr(lib(), name)(ctypes.byref(args), c_void_p(stream))
    if status != 0:
        msg = lib().pkda_last_error().decode(errors="replace")
        if status < 0:
            raise ValueError(f"{name}: {msg} (status {status})")
        raise PkdaError(name, status, msg)
