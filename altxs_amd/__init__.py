"""altxs_amd -- MI355X (gfx950) implementation of the altxs per-symbol model step.

Host side in Python/PyTorch-ROCm; compute in libaltxs_hip.so (hand-written HIP
kernels for CDNA4) behind the C-ABI declared in include/altxs.h.
"""

from .config import AltxsConfig, make_config, slot_itinerary  # noqa: F401

__version__ = "0.1.0"
