"""GPU forms of the vector-search engine's distance functions.

The reference engine (engine/src/index) computes L2SquaredDistance,
InnerProduct, SquaredNorm, PqAdcDistance and ProductQuantizer::
ComputeDistanceTable one call at a time on the CPU.  vectra_amd.index.scan
computes whole batches of those calls on the GPU through
libvectra_scan.so (include/vectra_scan.h), each result bit-identical to the
reference function's.
"""

from vectra_amd.index.scan import (  # noqa: F401
    ScanError,
    inner_products,
    l2_squared_distances,
    pq_adc_distances,
    pq_distance_tables,
    squared_norms,
)
