"""dsk_moe -- MI355X (gfx950) MoE-layer forward of DeepSeeker, as a drop-in.

Host side in Python/torch; all compute in ``libdsk_moe.so`` (hand-written
HIP kernels behind the C ABI of ``include/dsk_moe.h``), called through
ctypes on the current HIP stream.

    from dsk_moe import moe_layer, ResidentBank, SharedExpert

``moe_layer`` has the reference's signature
(``src/deepseeker/mlx_forward.py:257-263``).
"""

from ._lib import DskError, load as load_library
from .bank import ResidentBank, SharedExpert
from .checkpoint import Checkpoint, build_manifest, fp8_block_dequant
from .layer import MoELayer, moe_layer
from .pinned import expert_rows, gather_pinned_contributions
from .stack import MoEStack, rmsnorm
from .trace import Geometry, Trace, TraceSink
from .ops import (align_block_size, dispatch, fp4_dequant, fp4_quantize, q3_dequant,
                  q3_quantize, q3_repack, route, workspace_size)

__all__ = ["Checkpoint", "DskError", "MoELayer", "MoEStack", "ResidentBank", "SharedExpert", "TraceSink", "align_block_size",
           "build_manifest", "dispatch", "expert_rows", "gather_pinned_contributions", "fp4_dequant", "fp8_block_dequant", "fp4_quantize", "load_library", "moe_layer",
           "q3_dequant", "q3_quantize", "q3_repack", "rmsnorm", "route", "workspace_size", "Geometry", "Trace"]
