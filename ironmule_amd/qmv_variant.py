"""A second dispatch geometry of the K=3840 qmv, installed per model and switched at run time.

Mirrors the call surface of ironmule/qmv_variant.py: `QUALIFIED_GEOMETRY`,
`QUALIFIED_ACTION_ID`, `CORRECTNESS_CONTRACT`, `VariantUnsupported`, `VariantGate`,
`kernel_for`, `GatedVariantLinear`, `_identical`, `install` and `uninstall`.

A geometry is (simdgroups per threadgroup, output rows per simdgroup), the dispatch a
Metal caller describes.  On gfx950 it does not choose the HIP launch (the library does);
it is part of the kernel's specification, so each geometry is registered under its own
name, and every call is checked to cover all N rows with it.

`install` works in three passes over the model and changes it only in the last: it checks
the environment as `qmv_k3840.enable` does; it qualifies every K=3840 projection (format,
N a multiple of the geometry's rows per threadgroup, then `_identical` on the projection's
own weights); and only if no projection failed `_identical` does it swap the qualified
ones for `GatedVariantLinear`s that share one `VariantGate`.  The gate starts shut: while
it is shut, or for any input but a single decode row, the original module runs.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from . import _native, kernel_registry
from . import qmv_k3840 as qmv
from .module_swap import DecodeOverride, replace, restore
from .quantized import QuantizedLinear

#: The geometry the reference qualified, and the identifier its evidence names it by.
QUALIFIED_GEOMETRY = (4, 8)
QUALIFIED_ACTION_ID = "k3840_geometry_sg4_r8"

#: `_identical`'s bound: the bf16 rounding of the output (2^-8 of |ref|) plus an
#: allowance for fp32 summation order of 2^-14 of sum(|w|*|x|) over the row.
ROUNDING = 2.0 ** -8
SUMMATION = 2.0 ** -14
#: Rows of the float64 reference computed at a time (at K=3840: 126 MB per chunk).
REFERENCE_CHUNK = 4096

CORRECTNESS_CONTRACT = (
    "before it is installed, every admitted projection's decode output on its own weights "
    "and a seeded probe row is within 2^-8 |ref| + 2^-14 sum|w*x| of ref, a float64 product "
    "of the weight dequantised by imq_dequant; if any projection misses that bound nothing "
    "is installed")


class VariantUnsupported(RuntimeError):
    """Raised by `install` when the variant cannot be installed on this model; the model
    is left as it was."""


@dataclass
class VariantGate:
    """The switch every projection of one `install` consults on each call.

    `open` and `close` flip it with a reason the caller can log; `kill` shuts it for the
    rest of the process, after which `open` is ignored."""

    active: bool = False
    killed: bool = False
    reason: str = "not activated"

    def open(self, reason: str) -> None:
        if not self.killed:
            self.active, self.reason = True, reason

    def close(self, reason: str) -> None:
        self.active, self.reason = False, reason

    def kill(self, reason: str) -> None:
        self.active, self.killed, self.reason = False, True, reason


def kernel_for(geometry: tuple[int, int], fixed_k: int = qmv.TARGET_K):
    """The registered kernel for this geometry at K=`fixed_k`."""
    simdgroups, results = geometry
    if simdgroups < 1 or results < 1:
        raise ValueError(f"geometry {geometry} must be positive")
    return kernel_registry.build(
        f"qmv_k{fixed_k}_sg{simdgroups}_r{results}",
        input_names=["w", "scales", "biases", "x", "shape"], output_names=["out"],
        source=qmv.SOURCE, ensure_row_contiguous=True,
        template={"fixed_k": fixed_k, "num_simdgroups": simdgroups,
                  "results_per_simdgroup": results})


class GatedVariantLinear(DecodeOverride):
    """A qualified projection that runs the variant for a single decode row while `gate`
    is open, and the original module otherwise."""

    def __init__(self, source: QuantizedLinear, kernel, geometry: tuple[int, int],
                 gate: VariantGate) -> None:
        super().__init__(source)
        self._kernel = kernel
        self._gate = gate
        simdgroups, results = geometry
        threadgroups = self.out_features // (simdgroups * results)
        self._grid = (qmv.SIMD_SIZE, simdgroups * threadgroups, 1)
        self._threadgroup = (qmv.SIMD_SIZE, simdgroups, 1)
        self._shape = qmv.shape_array(qmv.TARGET_K, self.out_features)

    def serves(self, x: torch.Tensor) -> bool:
        return self._gate.active and super().serves(x)

    def decode(self, row: torch.Tensor) -> torch.Tensor:
        (y,) = self._kernel(inputs=[self.weight, self.scales, self.biases, row, self._shape],
                            output_shapes=[(1, self.out_features)], output_dtypes=[row.dtype],
                            grid=self._grid, threadgroup=self._threadgroup)
        return y


def _reference(module: QuantizedLinear, probe: torch.Tensor):
    """(ref, sum|w*x|) per output row in float64, from imq_dequant's fp32 weight."""
    x = probe.reshape(-1).to(torch.float64)
    ref, mag = [], []
    for start in range(0, module.out_features, REFERENCE_CHUNK):
        rows = slice(start, start + REFERENCE_CHUNK)
        dense = _native.dequant(module.weight[rows].contiguous(), module.scales[rows].contiguous(),
                                module.biases[rows].contiguous(), torch.float32).to(torch.float64)
        ref.append(dense @ x)
        mag.append(dense.abs() @ x.abs())
    ref, mag = torch.cat(ref), torch.cat(mag)
    bias = getattr(module, "bias", None)
    if bias is not None:
        ref = ref + bias.to(torch.float64).reshape(-1)
        mag = mag + bias.to(torch.float64).abs().reshape(-1)
    return ref, mag


def _identical(module: QuantizedLinear, kernel, geometry: tuple[int, int],
               probe_seed: int = 0) -> bool:
    """Whether the variant meets the correctness contract on this projection: one seeded
    bf16 probe row through the variant, against an independent float64 reference."""
    gen = torch.Generator(device=module.weight.device)
    gen.manual_seed(probe_seed)
    probe = torch.randn((1, 1, qmv.TARGET_K), generator=gen,
                        device=module.weight.device).to(torch.bfloat16)
    variant = GatedVariantLinear(module, kernel, geometry, VariantGate(active=True))
    got = variant(probe).reshape(-1).to(torch.float64)
    ref, mag = _reference(module, probe)
    return bool(torch.all((got - ref).abs() <= ROUNDING * ref.abs() + SUMMATION * mag))


def install(model: torch.nn.Module, identity: Any,
            geometry: tuple[int, int] = QUALIFIED_GEOMETRY) -> tuple[VariantGate, dict[str, Any]]:
    """Qualify the variant on every K=3840 projection of `model` and install it on those
    that qualify, or raise (K3840Unsupported for the environment, VariantUnsupported
    otherwise) with the model unchanged.  Returns the shut gate and a record."""
    qmv._admit_environment(identity)
    kernel = kernel_for(geometry)
    simdgroups, results = geometry
    qualified, declined, mismatched = [], [], []
    for site in qmv._candidates(model):
        fits = qmv._admit_projection(site.module) and \
            site.module.out_features % (simdgroups * results) == 0
        if not fits:
            declined.append(site.path)
        elif _identical(site.module, kernel, geometry):
            qualified.append(site)
        else:
            mismatched.append(site.path)
    if mismatched:
        raise VariantUnsupported(
            f"the variant missed its bound on {len(mismatched)} projection(s), first "
            f"{mismatched[0]}; the model is unchanged")
    if not qualified:
        raise VariantUnsupported(
            f"no K={qmv.TARGET_K} projection has the admitted format with N a multiple of "
            f"{simdgroups * results}")
    gate = VariantGate()
    replace(qualified, lambda module: GatedVariantLinear(module, kernel, geometry, gate))
    return gate, {"admitted": len(qualified), "declined": len(declined),
                  "mismatched": len(mismatched),
                  "admitted_paths": [site.path for site in qualified],
                  "declined_paths": declined,
                  "geometry": {"num_simdgroups": simdgroups, "results_per_simdgroup": results},
                  "action_id": QUALIFIED_ACTION_ID,
                  "correctness_contract": CORRECTNESS_CONTRACT}


def uninstall(model: torch.nn.Module) -> int:
    """Undo `install`: the original modules go back in place. Returns how many."""
    return len(restore(model, GatedVariantLinear))
