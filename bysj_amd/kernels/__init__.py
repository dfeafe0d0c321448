"""MI355X (gfx950) operators of the DPA4/SeZM slice: the reference's ``kernels`` package."""

from .gie import gie_available, gie_zonal_scatter, zonal_scatter
from .rmsnorm import rmsnorm, rmsnorm_available
from .segment import (
    force_assembly,
    group_by_source,
    segment_available,
    segment_offsets,
    segment_softmax,
    segment_sum,
)

__all__ = [
    "force_assembly",
    "gie_available",
    "gie_zonal_scatter",
    "group_by_source",
    "rmsnorm",
    "rmsnorm_available",
    "segment_available",
    "segment_offsets",
    "segment_softmax",
    "segment_sum",
    "zonal_scatter",
]
