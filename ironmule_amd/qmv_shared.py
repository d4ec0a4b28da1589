"""The shared-weight qmv at K=3840: one weight sweep serves several activation vectors.

Mirrors ironmule/qmv_shared.py (`SHARED`, `shape_array`, `run_shared`).  The reference
shares one weight load between 1 or 2 vectors ("shares the load, not the arithmetic").
The gfx950 library serves up to 32 vectors per sweep (imq_qmv_multi); the reference's
widths 1 and 2 are pre-registered in `SHARED` and any other width up to 32 is registered
on first use.  Each vector's result depends only on that vector and the weight.
"""

from __future__ import annotations

import torch

from . import kernel_registry
from .qmv_k3840 import NUM_SIMDGROUPS, SIMD_SIZE, SOURCE

TARGET_K = 3840
MAX_WIDTH = 32


def _kernel(width: int):
    inputs = ["w", "scales", "biases"] + [f"x{v}" for v in range(width)] + ["shape"]
    outputs = [f"out{v}" for v in range(width)]
    return kernel_registry.build(
        f"qmv_k3840_shared_x{width}",
        input_names=inputs,
        output_names=outputs,
        source=SOURCE,
        ensure_row_contiguous=True,
        template={"width": width, "k": TARGET_K},
    )


SHARED = {width: _kernel(width) for width in (1, 2)}
shape_array = kernel_registry.shape_tensor


def run_shared(w, scales, biases, vectors, out_features: int):
    """One weight sweep, `len(vectors)` independent (1, N) results."""
    width = len(vectors)
    if not 1 <= width <= MAX_WIDTH:
        raise ValueError(f"1 to {MAX_WIDTH} vectors share one sweep, got {width}")
    kernel = SHARED.get(width)
    if kernel is None:
        kernel = SHARED[width] = _kernel(width)
    groups = (out_features + 7) // 8
    return kernel(
        inputs=[w, scales, biases, *vectors, shape_array(TARGET_K, out_features)],
        output_shapes=[(1, out_features)] * width,
        output_dtypes=[vectors[0].dtype] * width,
        grid=(SIMD_SIZE, NUM_SIMDGROUPS * groups, 1),
        threadgroup=(SIMD_SIZE, NUM_SIMDGROUPS, 1),
    )
