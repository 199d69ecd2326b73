"""MI355X-native SSD scan: the import surface of r2/dhammic-ai/src/kernels/__init__.py:7,18
for this path (``FusedSSDScan``, ``fused_ssd_scan``), plus the extended
``ssd_scan_combined``, ``fused_trapezoidal_ssd_scan`` (the caller's two SSD calls,
r2/dhammic-ai/src/mamba_base_engine.py:167-191, as one scan) and the block front end that
feeds it (``fused_trapezoidal``, ``fused_rope``, ``fused_inproj_split``; the reference's
src/kernels/trapezoidal.py, rope.py, inproj_split.py), and the loss head
(``fused_lmhead_xent``, ``ChunkedLMHeadXent``; src/kernels/lmhead_xent.py,
src/runtime/chunked_lmhead.py). Put ``dhammic-ai_amd/`` on
sys.path and import ``kernels`` (the reference puts ``src/`` on sys.path, r2/dhammic-ai/train.py:20).
"""
from .frontend import (FusedInProjSplit, FusedInProjSplitModule, FusedRoPE, FusedTrapezoidal, fused_inproj_split,
                       fused_rope, fused_trapezoidal)
from .lmhead import ChunkedLMHeadXent, FusedLMHeadXent, FusedLMHeadXentModule, fused_lmhead_xent
from .ssd_scan import FusedSSDScan, fused_ssd_scan, ssd_scan_combined
from .trapezoidal_ssd import fused_trapezoidal_ssd_scan

__all__ = ["FusedSSDScan", "fused_ssd_scan", "ssd_scan_combined", "fused_trapezoidal_ssd_scan",
           "fused_trapezoidal", "FusedTrapezoidal", "fused_rope", "FusedRoPE", "fused_inproj_split",
           "FusedInProjSplit", "FusedInProjSplitModule", "fused_lmhead_xent", "FusedLMHeadXent",
           "FusedLMHeadXentModule", "ChunkedLMHeadXent"]
