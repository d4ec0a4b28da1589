"""The K=3840 decode qmv as a drop-in for a model's projections, on the gfx950 kernels.

Mirrors the call surface of ironmule/qmv_k3840.py: the kernels `K3840` (fixed K) and
`PORT` (runtime K), `run`, `shape_array`, `K3840QuantizedLinear`, `enable`/`disable`, the
admission helpers `_admit_environment`/`_admit_projection` and `K3840Unsupported`.  The
reference runs a Metal transcription of MLX's qmv; here both kernels are the library's
`imq_qmv` (libironmule_qmv.so), reached through `kernel_registry.HipKernel`.

How a model is changed:

* `enable(model, identity)` first checks the caller and the machine (a model identity
  with an architecture this path is qualified for and a sha256 digest; a gfx950 device
  with the library loaded), then lists every `QuantizedLinear` whose reduction length is
  3840, sorts them into admitted and declined by their format, and only then swaps the
  admitted ones.  Any refusal raises `K3840Unsupported` with the model unchanged.
* A swapped projection is a `K3840QuantizedLinear`: a (1, 1, 3840) activation runs the
  kernel, anything else (prefill, batches) runs the original module on the same tensors.
* `disable(model)` puts the original module objects back.

What admission pins differs from the reference.  The reference qualified its kernel as
byte-identical to MLX on one Apple machine, one MLX/mlx_lm version pair and one model
revision, and pins those.  These kernels are qualified by parity tests against the oracle
over any weights of the admitted format, so admission pins the device architecture and
the format (4-bit, group 64, bf16 scales and biases, contiguous, N a multiple of 8) and
asks for a model identity in the same shape as the reference's.
"""

from __future__ import annotations

import re
from typing import Any

import torch

from . import _native, kernel_registry
from .module_swap import DecodeOverride, find_sites, in_features, replace, restore
from .quantized import QuantizedLinear


class K3840Unsupported(RuntimeError):
    """Raised by `enable` when this machine, this model or none of its projections
    qualifies; the model is left as it was."""


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

ROWS_PER_THREADGROUP = NUM_SIMDGROUPS * RESULTS_PER_SIMDGROUP  # 8

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

shape_array = kernel_registry.shape_tensor


def run(kernel, w, scales, biases, x, out_features: int, in_features: int):
    """`x @ dequantize(w).T` for one (1, K) row through `kernel`, with the dispatch a Metal
    caller passes: threadgroups of two 32-lane simdgroups, each simdgroup owning four
    output rows, enough threadgroups to cover N."""
    threadgroups = -(-out_features // ROWS_PER_THREADGROUP)
    (y,) = kernel(inputs=[w, scales, biases, x, shape_array(in_features, out_features)],
                  output_shapes=[(1, out_features)], output_dtypes=[x.dtype],
                  grid=(SIMD_SIZE, NUM_SIMDGROUPS * threadgroups, 1),
                  threadgroup=(SIMD_SIZE, NUM_SIMDGROUPS, 1))
    return y


class K3840QuantizedLinear(DecodeOverride):
    """An admitted projection: (1, 1, 3840) activations run `K3840`; every other input
    runs the original module, whose tensors this one shares."""

    def __init__(self, source: QuantizedLinear) -> None:
        super().__init__(source)

    def decode(self, row: torch.Tensor) -> torch.Tensor:
        return run(K3840, self.weight, self.scales, self.biases, row, self.out_features,
                   TARGET_K)


# ------------------------------------------------------------------ admission

_HEX_DIGEST = re.compile(r"[0-9a-f]{64}")


def _identity_problem(identity: Any) -> str | None:
    if identity is None:
        return "enable() needs the model's identity (architecture, sha256 digest); got None"
    digest = getattr(identity, "identity_sha256", None)
    if not isinstance(digest, str) or not _HEX_DIGEST.fullmatch(digest):
        return f"identity_sha256 is not 64 lowercase hex digits: {str(digest)[:16]!r}"
    architecture = getattr(identity, "architecture", None)
    if architecture not in VERIFIED_ARCHITECTURES:
        return f"architecture {architecture!r} is not one of {VERIFIED_ARCHITECTURES}"
    return None


def _device_problem() -> str | None:
    try:
        code, arch, _ = _native.device_check()
    except Exception as exc:  # the library or the HIP runtime is missing
        return f"libironmule_qmv.so cannot run here: {exc}"
    if code != 0 or not arch.startswith(VERIFIED_DEVICE_ARCH):
        return f"the device is {arch or 'absent'}; these kernels are qualified on {VERIFIED_DEVICE_ARCH}"
    return None


def _admit_environment(identity: Any) -> None:
    """Raise K3840Unsupported unless the identity qualifies and the device is gfx950.
    Called once per `enable`, never per token."""
    problem = _identity_problem(identity) or _device_problem()
    if problem is not None:
        raise K3840Unsupported(problem)


def _format_problems(module: QuantizedLinear) -> list[str]:
    """Every way this projection differs from the admitted format (empty: admitted).

    The format: 4-bit codes in groups of 64 over K=3840, N a multiple of the eight rows a
    Metal threadgroup writes, packed int32 (or uint32) words of shape (N, 480) and bf16
    scales and biases of shape (N, 60), all contiguous
    (the conditions of ironmule/qmv_k3840.py:379-408)."""
    problems = []
    if int(module.bits) != VERIFIED_BITS:
        problems.append(f"bits={module.bits}")
    if int(module.group_size) != VERIFIED_GROUP_SIZE:
        problems.append(f"group_size={module.group_size}")
    if in_features(module) != TARGET_K:
        problems.append(f"K={in_features(module)}")
    n = int(module.weight.shape[0])
    if n % ROWS_PER_THREADGROUP:
        problems.append(f"N={n} is not a multiple of {ROWS_PER_THREADGROUP}")
    groups = TARGET_K // VERIFIED_GROUP_SIZE
    expected = {
        "weight": ((n, TARGET_K * VERIFIED_BITS // 32), (torch.int32, torch.uint32)),
        "scales": ((n, groups), (VERIFIED_DTYPE,)),
        "biases": ((n, groups), (VERIFIED_DTYPE,)),
    }
    for name, (shape, dtypes) in expected.items():
        tensor = getattr(module, name, None)
        if tensor is None:
            problems.append(f"no {name}")
        elif tuple(tensor.shape) != shape or tensor.dtype not in dtypes:
            problems.append(f"{name} {tuple(tensor.shape)} {tensor.dtype}")
        elif not tensor.is_contiguous():
            problems.append(f"{name} not contiguous")
    return problems


def _admit_projection(module: QuantizedLinear) -> bool:
    """True when the projection is exactly in the admitted format."""
    return not _format_problems(module)


def _candidates(model: torch.nn.Module):
    """The sites of every QuantizedLinear with K=3840, admitted or not; installed
    replacements are not looked into."""
    return find_sites(model, lambda m: isinstance(m, QuantizedLinear)
                      and in_features(m) == TARGET_K, opaque=(DecodeOverride,))


def _replace(module: torch.nn.Module, admitted: list[str], skipped: list[str],
             prefix: str = "") -> None:
    """Swap every admitted K=3840 projection under `module` for a K3840QuantizedLinear;
    append the dotted paths (under `prefix`) of the swapped ones to `admitted` and of the
    refused ones to `skipped`."""
    take, leave = [], []
    for site in _candidates(module):
        (take if _admit_projection(site.module) else leave).append(site)
    replace(take, K3840QuantizedLinear)
    head = f"{prefix}." if prefix else ""
    admitted.extend(head + site.path for site in take)
    skipped.extend(head + site.path for site in leave)


def _restore(module: torch.nn.Module, restored: list[str], prefix: str = "") -> None:
    """Put back the original of every K3840QuantizedLinear under `module`; append their
    dotted paths to `restored`."""
    head = f"{prefix}." if prefix else ""
    restored.extend(head + path for path in restore(module, K3840QuantizedLinear))


def enable(model: torch.nn.Module, identity: Any) -> dict[str, Any]:
    """Swap the model's admitted K=3840 projections, or raise K3840Unsupported and change
    nothing.  Returns what was done: counts and dotted paths of the admitted and declined
    projections, the device architecture and the identity digest."""
    _admit_environment(identity)
    candidates = _candidates(model)
    if not any(_admit_projection(site.module) for site in candidates):
        raise K3840Unsupported(
            f"none of the model's {len(candidates)} K={TARGET_K} projections is in the "
            "admitted format")
    admitted: list[str] = []
    declined: list[str] = []
    _replace(model, admitted, declined)
    return {
        "admitted": len(admitted),
        "declined": len(declined),
        "admitted_paths": admitted,
        "declined_paths": declined,
        "device_arch": VERIFIED_DEVICE_ARCH,
        "identity_sha256": identity.identity_sha256,
    }


def disable(model: torch.nn.Module) -> int:
    """Undo `enable`: the original modules go back in place. Returns how many."""
    restored: list[str] = []
    _restore(model, restored)
    return len(restored)
