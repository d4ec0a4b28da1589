"""The shared-weight qmv for the aligned reduction lengths K = 4096 and 15360.

Mirrors ironmule/qmv_fast_shared.py (`SUPPORTED_K`, `KERNELS`, `shape_array`,
`run_fast`).  In the reference this is a separate Metal transcription (MLX's
`qmv_fast_impl`: 16 values per thread, 512-value blocks, no tail); on gfx950 both shapes
run the same library kernel, registered under the reference's kernel names so callers
and identifiers carry over.  Widths 1 and 2 are pre-registered; up to 32 are served.
"""

from __future__ import annotations

import torch

from . import kernel_registry
from .qmv_k3840 import NUM_SIMDGROUPS, SIMD_SIZE, SOURCE

SUPPORTED_K = (4096, 15360)
MAX_WIDTH = 32
VALUES_PER_THREAD = 16
BLOCK_SIZE = VALUES_PER_THREAD * SIMD_SIZE  # 512


def _kernel(k: int, width: int):
    inputs = ["w", "scales", "biases"] + [f"x{v}" for v in range(width)] + ["shape"]
    return kernel_registry.build(
        f"qmv_fast_k{k}_x{width}",
        input_names=inputs,
        output_names=[f"out{v}" for v in range(width)],
        source=SOURCE,
        ensure_row_contiguous=True,
        template={"width": width, "k": k},
    )


KERNELS = {(k, width): _kernel(k, width) for k in SUPPORTED_K for width in (1, 2)}
shape_array = kernel_registry.shape_tensor


def run_fast(w, scales, biases, vectors, out_features: int, in_features: int):
    """One weight sweep for `len(vectors)` requests on an aligned reduction length."""
    if in_features not in SUPPORTED_K:
        raise ValueError(f"K={in_features} is not one of {SUPPORTED_K}")
    width = len(vectors)
    if not 1 <= width <= MAX_WIDTH:
        raise ValueError(f"1 to {MAX_WIDTH} vectors share one sweep, got {width}")
    kernel = KERNELS.get((in_features, width))
    if kernel is None:
        kernel = KERNELS[(in_features, width)] = _kernel(in_features, width)
    groups = (out_features + 7) // 8
    return kernel(
        inputs=[w, scales, biases, *vectors, shape_array(in_features, out_features)],
        output_shapes=[(1, out_features)] * width,
        output_dtypes=[vectors[0].dtype] * width,
        grid=(SIMD_SIZE, NUM_SIMDGROUPS * groups, 1),
        threadgroup=(SIMD_SIZE, NUM_SIMDGROUPS, 1),
    )
