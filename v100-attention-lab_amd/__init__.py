"""MI355X-native fused chunked Gated DeltaNet forward.

The hot path of ``v100-attention-lab`` (``gdn_chunk_fwd``,
gdn_triton.py:113-140) as a hand-written gfx950 HIP kernel behind a C ABI
(``include/gdn_mi355x.h``), called from PyTorch-ROCm through ctypes.

The directory name is not a Python identifier; import it with
``importlib.import_module("v100-attention-lab_amd")`` -- it also registers
itself as ``v100_attention_lab_amd``.
"""

import sys as _sys

from ._lib import load_library, status_string, LIB_PATH  # noqa: F401
from .ops import (gdn_fwd, gdn_chunk_fwd, auto_block_v, gdn_prep, l2norm,  # noqa: F401
                  chunk_gated_delta_rule, gdn_bwd)

_sys.modules.setdefault("v100_attention_lab_amd", _sys.modules[__name__])

__all__ = ["gdn_fwd", "gdn_chunk_fwd", "chunk_gated_delta_rule", "gdn_prep", "l2norm",
           "gdn_bwd", "auto_block_v", "load_library", "status_string"]
