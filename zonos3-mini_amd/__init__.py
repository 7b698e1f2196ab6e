"""MI355X-native (gfx950) gated-DeltaNet token mixer of ZONOS3-Mini.

Hand-written HIP kernels behind a C ABI (``include/zonos3_gdn.h``, ``libzonos3_gdn.so``), driven from
PyTorch-ROCm. Public surface:

* ``ops``: direct ops (``recurrent_fwd``, ``decode_step``, ``chunk_fwd``, ``fused_decode_step``).
* ``torch_ops``: the same kernels registered as ``torch.ops.zgdn.*`` (with fake implementations for tracing).
"""

from . import ops  # noqa: F401
from . import torch_ops  # noqa: F401  (registers torch.ops.zgdn.*)
from .ops import chunk_fwd, decode_step, fused_decode_step, recurrent_fwd  # noqa: F401

__all__ = ["ops", "torch_ops", "recurrent_fwd", "decode_step", "chunk_fwd", "fused_decode_step"]
