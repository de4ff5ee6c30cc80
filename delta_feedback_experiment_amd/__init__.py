"""MI355X (gfx950) PKDA recurrence: hand-written HIP kernels behind a C ABI.

A drop-in for the PKDA recurrence path of a9lim/delta-feedback-experiment
(``delta_feedback_experiment/pkda.py:412-475`` and
``delta_feedback_experiment/fla_ops.py:252-569``).  The compute lives in
``libpkda_gfx950.so`` (``csrc/*.hip``, C ABI in ``include/pkda_gfx950.h``);
this package is the PyTorch-facing host side.  It also carries the
recurrence's producer, the fused Q/K/V short convolution + SiLU + L2 norm
(``delta_feedback_experiment/fla_ops.py:134-249``), and its consumer, the
RMSNorm with a sigmoid output gate (``fla_ops.py:572-657``), the control
activations with their packed gradient (:mod:`.controls`; the decay
expansion runs inside the gate kernel, ``chunk_pkda(..., decay_up=...)``), and
the slot-pool serving path that connects a cached prefill to the decode step
(:mod:`.serve`).  Nothing here falls back to the CPU: without a HIP device and
the built library every operator raises.
"""

from .chunk import chunk_pkda
from .controls import pkda_controls
from .conv import pkda_qkv_conv
from .norm_gate import pkda_norm_gate
from .ops import pkda_recurrence
from .pkda import fused_recurrent_pkda, pkda_decode_step_
from .serve import DecodePool, pkda_prefill_, pkda_qkv_conv_cached_

__all__ = ["DecodePool", "chunk_pkda", "fused_recurrent_pkda", "pkda_controls", "pkda_decode_step_",
           "pkda_norm_gate", "pkda_prefill_", "pkda_qkv_conv", "pkda_qkv_conv_cached_", "pkda_recurrence"]
