"""MI355X-native CRESSO5: the reference optimizer's per-step coordinate-field
hot path on hand-written gfx950 HIP kernels (libcresso_hip.so)."""

from .optimizer import CRESSO, CRESSO5, count_optimizer_state_elements, theoretical_state_elements

__all__ = ["CRESSO5", "CRESSO", "count_optimizer_state_elements", "theoretical_state_elements"]
