"""MI355X (gfx950) implementation of LightDelta's fused Gated DeltaNet decode path.

Importing the package registers the `torch.ops.lightdelta` ops (decode, gather_state,
scatter_state and the additive copy_state / gather_slots / scatter_slots).  The HIP
library is loaded on first use and its absence raises; there is no CPU fallback.
"""

from . import ops  # noqa: F401
from .backend import GDNBackend
from .config import BackendConfig

__version__ = "0.1.0"
__all__ = ["GDNBackend", "BackendConfig", "ops"]
