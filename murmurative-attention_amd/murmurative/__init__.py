"""Murmurative Attention for AMD Instinct MI355X (gfx950).

Same public names as the reference package (src/murmurative/__init__.py):
six ops on hand-written HIP kernels and the five eager ``*_reference``
functions.
"""

from .ops import (
    slot_select,
    slot_attend,
    slot_select_attend,
    slot_update,
    slot_diffusion,
    slot_murmurate,
)

from .reference import (
    slot_select_reference,
    slot_attend_reference,
    slot_update_reference,
    slot_diffusion_reference,
    slot_murmurate_reference,
)

__version__ = "0.1.0"
__all__ = [
    "slot_select",
    "slot_attend",
    "slot_select_attend",
    "slot_update",
    "slot_diffusion",
    "slot_murmurate",
    "slot_select_reference",
    "slot_attend_reference",
    "slot_update_reference",
    "slot_diffusion_reference",
    "slot_murmurate_reference",
]
