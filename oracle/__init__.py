"""CPU oracle of the DPA4/SeZM operator slice -- TEST INFRASTRUCTURE ONLY.

A restatement, in torch on the CPU, of the reference's executable
specification (lipengfei1409/bysj ``python/reference/*.py`` and the CSR
helpers of ``python/kernels/segment.py``), following the same ATen op order
so that sequential fp32 results can be compared bit for bit.  Plus
independent brute-force loops (``oracle.loops``) used to pin it.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only as the checker.  The product
(``bysj_amd``) never imports it and has no CPU fallback.

Pinning status of each function (tests/test_oracle_pinning.py; every
function below has a check of its own, so none is parity unpinned):

=============================  ==============================================
segment_offsets                known answers of the reference tests, brute force
group_by_source                known answers (stable order), brute force
segment_sum_reference          reference known-answer loop, sequential fp32
                               loop (bit-exact), fp64 brute force
segment_sum_backward           autograd of the chain vs closed form
segment_softmax_reference      per-segment brute force, sum-to-one, masking,
                               no-null normalisation, all-masked -> zeros
segment_softmax_backward       autograd of the chain vs closed form
force_assembly_reference       reference loop, Newton's third law, exact
                               (math.fsum) fp64 brute force
zonal_scatter_reference        loop oracle, exact normalise-after-sum known
                               answer, zero row 0, 1-D == 3-D inverse, empty
zonal_scatter backward         fp64 closed form with exact sums (shared and
                               unreferenced slots, both inverse shapes), the
                               golden fixture of the reference's GIE test,
                               four planted mistakes
rmsnorm                        closed formula, fp64 brute force, zeros
rmsnorm backward               autograd of the chain vs closed form
edge_stream_combine_reference  float64 element loop, closed values, the
                               float32 rounding order, planted mistakes
=============================  ==============================================
"""

from .edge_stream import edge_stream_combine_reference
from .gie import gie_zonal_scatter_reference, zonal_scatter_backward_reference, zonal_scatter_reference
from .rmsnorm import rmsnorm, rmsnorm_backward_reference
from .segment import (
    force_assembly_reference,
    group_by_source,
    segment_offsets,
    segment_softmax_backward_reference,
    segment_softmax_reference,
    segment_sum_backward_reference,
    segment_sum_reference,
)

__all__ = [
    "edge_stream_combine_reference",
    "force_assembly_reference",
    "gie_zonal_scatter_reference",
    "group_by_source",
    "rmsnorm",
    "rmsnorm_backward_reference",
    "segment_offsets",
    "segment_softmax_backward_reference",
    "segment_softmax_reference",
    "segment_sum_backward_reference",
    "segment_sum_reference",
    "zonal_scatter_backward_reference",
    "zonal_scatter_reference",
]
