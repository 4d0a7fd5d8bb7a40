"""MI355X (gfx950) Mamba-2 SSD hot path behind the ``ascend_kernel`` API.

Drop-in for the reference package's public entry points
(mamba_ascendc/python/ascend_kernel/ascend_kernel/__init__.py):
``mamba2_ssd_fwd`` and its alias ``mamba_chunk_scan_combined``, plus the
decode step ``selective_state_update`` of the reference's Triton port.  Importing the
package loads the HIP library (no GPU work) and registers the
``torch.ops.mamba_ascend`` operators.
"""

from ._runtime import LIBRARY_PATH, load_library
from .mamba2 import (TrainingPolicy, get_training_policy, mamba2_ssd_fwd, mamba_chunk_scan_combined,
                     register_ops, set_training_policy, training_policy)
from .modules import SsdCore
from .selective_state_update import selective_state_update

load_library()
register_ops()

__all__ = ["mamba2_ssd_fwd", "mamba_chunk_scan_combined", "selective_state_update", "SsdCore",
           "TrainingPolicy", "get_training_policy", "set_training_policy", "training_policy",
           "load_library", "LIBRARY_PATH"]
