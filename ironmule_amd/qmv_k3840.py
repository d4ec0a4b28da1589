"""The fixed-K (3840) decode qmv behind an admission gate, on the gfx950 kernels.

Mirrors ironmule/qmv_k3840.py.  The reference ships MLX 0.32.0's `qmv_impl` transcribed
to Metal at K=3840 (`K3840`) and at runtime K (`PORT`), dispatched as MLX does, and swaps
admitted projections for `K3840QuantizedLinear` after a narrow, fail-closed admission.
Here the kernels are the gfx950 library's (libironmule_qmv.so, `imq_qmv`); the Python
surface, the admission rules, the module swap and its restore are the reference's:

* `run(kernel, w, scales, biases, x, out_features, in_features)` dispatches with the
  reference's geometry arguments (grid (32, 2*ceil(N/8), 1), threadgroup (32, 2, 1)),
  which are validated and recorded; the library picks the HIP launch;
* `K3840QuantizedLinear` runs the kernel for single-token decode (x of shape (1, 1, K))
  and calls the original module for everything else;
* `enable` admits or raises `K3840Unsupported` before mutating anything; `disable`
  restores the original module objects.

Admission differs in what it pins.  The reference pins one Apple machine fingerprint,
MLX/mlx_lm versions and one model revision digest, because its kernel was qualified as
byte-identical to MLX on that stack.  These kernels are qualified by the parity tests
against the oracle over any weights of the admitted format, so admission pins the
device architecture (gfx950), requires a model identity (architecture and a sha256
digest, as the reference's identity object carries) and checks every projection's
format exactly as the reference does.
"""

from __future__ import annotations

import re
from typing import Any

import torch

from . import _native, kernel_registry
from .quantized import QuantizedLinear


class K3840Unsupported(RuntimeError):
    """The candidate is not admitted here. The library path stays in charge."""


VERIFIED_DEVICE_ARCH = "gfx950"
VERIFIED_ARCHITECTURES = ("gemma3", "qwen3")
VERIFIED_BITS = 4
VERIFIED_GROUP_SIZE = 64
VERIFIED_DTYPE = torch.bfloat16
TARGET_K = 3840

# The reference's Metal dispatch vocabulary (ironmule/qmv_k3840.py:44-52): the geometry
# arguments callers pass are checked against it.
SIMD_SIZE = 32
VALUES_PER_THREAD = 8
BLOCK_SIZE = VALUES_PER_THREAD * SIMD_SIZE  # 256
NUM_SIMDGROUPS = 2
RESULTS_PER_SIMDGROUP = 4
BYTES_PER_PACK = 4
PACK_FACTOR = 8
GROUP_SIZE = 64

SOURCE = ("imq_qmv (libironmule_qmv.so): y = x @ dequantize(w, scales, biases).T, 4-bit "
          "affine, group 64, bf16 activations, fp32 accumulation, bf16 output")


def _kernel(name: str, fixed_k: int | None):
    if fixed_k is not None and fixed_k % BLOCK_SIZE:
        raise ValueError(f"{fixed_k} is not a whole number of {BLOCK_SIZE}-value blocks")
    return kernel_registry.build(
        name,
        input_names=["w", "scales", "biases", "x", "shape"],
        output_names=["out"],
        source=SOURCE,
        ensure_row_contiguous=True,
        template={"fixed_k": fixed_k},
    )


PORT = _kernel("qmv_port", None)
K3840 = _kernel("qmv_k3840", TARGET_K)

_SHAPES: dict[tuple[int, int], torch.Tensor] = {}


def shape_array(in_features: int, out_features: int) -> torch.Tensor:
    """One shared constant per geometry (K, N); building it per call would be measured work."""
    key = (in_features, out_features)
    cached = _SHAPES.get(key)
    if cached is None:
        cached = torch.tensor([in_features, out_features], dtype=torch.int32)
        _SHAPES[key] = cached
    return cached


def run(kernel, w, scales, biases, x, out_features: int, in_features: int):
    """Dispatch with the reference's arguments: (32, 2, 1) threads, ceil(N/8) groups in y."""
    groups = (out_features + 7) // 8
    return kernel(
        inputs=[w, scales, biases, x, shape_array(in_features, out_features)],
        output_shapes=[(1, out_features)],
        output_dtypes=[x.dtype],
        grid=(SIMD_SIZE, NUM_SIMDGROUPS * groups, 1),
        threadgroup=(SIMD_SIZE, NUM_SIMDGROUPS, 1),
    )[0]


class K3840QuantizedLinear(torch.nn.Module):
    """The admitted projection with its matmul replaced. Same buffers, same bytes.

    Decode reaches the kernel; anything else calls the original module on the very same
    buffers, so a shape this module was not admitted for costs one comparison.
    """

    def __init__(self, source: QuantizedLinear) -> None:
        super().__init__()
        # Kept outside the module tree, so a walk never mistakes it for a live projection.
        object.__setattr__(self, "_source", source)
        self.weight = source.weight
        self.scales = source.scales
        self.biases = source.biases
        self.group_size = source.group_size
        self.bits = source.bits
        self.out_features = int(source.weight.shape[0])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        # Single-token decode only. Prefill and every wider input keep the library path.
        if len(shape) != 3 or shape[0] != 1 or shape[1] != 1:
            return self._source(x)
        out = run(K3840, self.weight, self.scales, self.biases, x[0], self.out_features,
                  TARGET_K)
        return out[None]


_SHA256 = re.compile(r"^[0-9a-f]{64}$")


def _admit_environment(identity: Any) -> None:
    """Everything expensive happens here, once, and never per token."""
    if identity is None:
        raise K3840Unsupported("no model identity available; the candidate fails closed")
    digest = getattr(identity, "identity_sha256", None)
    if not isinstance(digest, str) or not _SHA256.match(digest):
        raise K3840Unsupported(f"model identity digest missing or malformed: {str(digest)[:16]}")
    architecture = getattr(identity, "architecture", None)
    if architecture not in VERIFIED_ARCHITECTURES:
        raise K3840Unsupported(
            f"admitted architectures are {VERIFIED_ARCHITECTURES}, found {architecture}")
    try:
        code, arch, _ = _native.device_check()
    except Exception as exc:  # no library, no HIP runtime
        raise K3840Unsupported(f"the gfx950 library is unavailable: {exc}") from exc
    if code != 0 or not arch.startswith(VERIFIED_DEVICE_ARCH):
        raise K3840Unsupported(f"qualified on {VERIFIED_DEVICE_ARCH}, found {arch or 'no device'}")


def _admit_projection(module: QuantizedLinear) -> bool:
    """K alone is not enough: bits, group size, dtype, width and layout all decide
    (the reference's checks, ironmule/qmv_k3840.py:379-408)."""
    if int(module.bits) != VERIFIED_BITS or int(module.group_size) != VERIFIED_GROUP_SIZE:
        return False
    columns = int(module.weight.shape[1]) * 32 // int(module.bits)
    if columns != TARGET_K:
        return False
    out_features = int(module.weight.shape[0])
    if out_features % (NUM_SIMDGROUPS * RESULTS_PER_SIMDGROUP):
        return False  # the reference's kernel writes eight rows per threadgroup
    for array in (module.scales, module.biases):
        if array.dtype != VERIFIED_DTYPE:
            return False
    if module.weight.dtype not in (torch.int32, torch.uint32):
        return False
    if int(module.scales.shape[1]) != TARGET_K // VERIFIED_GROUP_SIZE:
        return False
    if module.scales.shape != module.biases.shape:
        return False
    expected = (
        (module.weight, out_features * (TARGET_K * VERIFIED_BITS // 32) * 4),
        (module.scales, out_features * (TARGET_K // VERIFIED_GROUP_SIZE) * 2),
        (module.biases, out_features * (TARGET_K // VERIFIED_GROUP_SIZE) * 2),
    )
    return all(array.is_contiguous() and array.numel() * array.element_size() == size
               for array, size in expected)


def _replace(module: torch.nn.Module, admitted: list[str], skipped: list[str],
             prefix: str = "") -> None:
    for name, child in list(module.named_children()):
        path = f"{prefix}.{name}" if prefix else name
        if isinstance(child, QuantizedLinear):
            columns = int(child.weight.shape[1]) * 32 // int(child.bits)
            if columns != TARGET_K:
                continue
            if _admit_projection(child):
                setattr(module, name, K3840QuantizedLinear(child))
                admitted.append(path)
            else:
                skipped.append(path)
        elif not isinstance(child, K3840QuantizedLinear):
            _replace(child, admitted, skipped, path)


def _restore(module: torch.nn.Module, restored: list[str], prefix: str = "") -> None:
    for name, child in list(module.named_children()):
        path = f"{prefix}.{name}" if prefix else name
        if isinstance(child, K3840QuantizedLinear):
            setattr(module, name, child._source)
            restored.append(path)
        else:
            _restore(child, restored, path)


def disable(model: torch.nn.Module) -> int:
    """Put every admitted projection back on the library path. Returns how many."""
    restored: list[str] = []
    _restore(model, restored)
    return len(restored)


def enable(model: torch.nn.Module, identity: Any) -> dict[str, Any]:
    """Admit the candidate on this model, or raise and leave it untouched."""
    _admit_environment(identity)
    admitted: list[str] = []
    skipped: list[str] = []
    _replace(model, admitted, skipped)
    if not admitted:
        raise K3840Unsupported("no projection met the admission conditions")
    return {
        "admitted": len(admitted),
        "declined": len(skipped),
        "admitted_paths": admitted,
        "declined_paths": skipped,
        "device_arch": VERIFIED_DEVICE_ARCH,
        "identity_sha256": getattr(identity, "identity_sha256", None),
    }
