"""The opt-in `native` plan on MI355X: every eligible 4-bit module runs the gfx950 kernels.

Mirrors ironmule/cuda_native.py (`matmul`, `gather_matmul`, `NativeQuantizedLinear`,
`NativeQuantizedEmbedding.as_linear`, `NativeQuantizedSwitchLinear`, `_eligible`,
`_probe`, `install`, `head_skip_needed`).  The reference's plan exists for pre-Ampere CUDA GPUs; this one for
gfx950.  The routing is the reference's, with the row limit raised from 8 to 32 because
the gfx950 library serves up to 32 activation rows with one weight sweep:

* bf16 activations with at most MAX_ROWS rows: the qmv kernel (imq_qmv);
* more rows (prefill): dequantise to fp16 (imq_dequant) and one GEMM, as the reference;
* MoE experts (QuantizedSwitchLinear): the gather kernel (imq_gather_qmv) for single-row
  activations and at most GATHER_MAX (token, expert) rows, the library path beyond;
* anything else (non-bf16 activations): the module's library path.

Installation is scoped to one model, probes one module per (type, weight shape) class
against an fp32 dequantise-then-matmul reference (tolerance 1e-2, as the reference), and
swaps classes only after every probe passes.
"""

from __future__ import annotations

import time
from typing import Any

import torch

from . import _native
from .quantized import (QuantizedEmbedding, QuantizedLinear, QuantizedSwitchLinear,
                        library_gather_matmul, library_matmul)

GROUP_SIZE = 64
BITS = 4
MAX_ROWS = _native.MAX_ROWS
#: (token, expert) rows the gather kernel serves (ironmule/cuda_native.py:40).
GATHER_MAX = 64
PROBE_TOLERANCE = 1e-2
#: Rows of a tall weight (an output head) the probe uses: the full K, a bounded N.
PROBE_ROWS = 8192
#: The fraction of device memory a prefill may plan to fill (weights + fp16 head copy).
PREFILL_HEADROOM = 0.9


def _qmv(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
         out_dtype: torch.dtype | None = None) -> torch.Tensor:
    k = int(w.shape[1]) * 8
    rows = x.reshape(-1, k)
    y = _native.qmv(w, scales, biases, rows.contiguous(), out_dtype=out_dtype or x.dtype)
    return y.reshape(*x.shape[:-1], int(w.shape[0]))


def matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
           biases: torch.Tensor) -> torch.Tensor:
    """`x @ dequantize(w).T` for a 4-bit, group-64 affine weight with bf16 scales."""
    if x.dtype != torch.bfloat16:
        return library_matmul(x, w, scales, biases)
    k = int(w.shape[1]) * 8
    if x.numel() <= MAX_ROWS * k:
        return _qmv(x, w, scales, biases)
    dense = _native.dequant(w, scales, biases, torch.float16)
    return (x.to(torch.float16) @ dense.T).to(x.dtype)


class NativeQuantizedLinear(QuantizedLinear):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = matmul(x, self.weight, self.scales, self.biases)
        return y + self.bias if self.bias is not None else y


class NativeQuantizedEmbedding(QuantizedEmbedding):
    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        return matmul(x, self.weight, self.scales, self.biases)


def gather_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                  indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
    """`x @ dequantize(w[indices]).T` over experts (mlx's gather_qmm with rhs_indices), the
    reference's routing (ironmule/cuda_native.py:199-218): single-row bf16 activations
    with at most GATHER_MAX (token, expert) rows take the gather kernel; a down
    projection has one activation row per pair, a gate/up projection one row per token
    shared by its experts (rows_per_x); anything else the library path."""
    if x.dtype != torch.bfloat16:
        return library_gather_matmul(x, w, scales, biases, indices)
    batch = tuple(torch.broadcast_shapes(x.shape[:-2], indices.shape))
    pairs = 1
    for d in batch:
        pairs *= int(d)
    if x.shape[-2] == 1 and pairs <= GATHER_MAX:
        if tuple(x.shape[:-2]) == batch:  # down: one activation row per pair
            xs = 1
        elif tuple(x.shape[:-2]) == batch[:-1] + (1,):  # gate/up: a token's row for its experts
            xs = batch[-1]
        else:
            x, xs = x.expand(*batch, *x.shape[-2:]), 1
        idx = indices.expand(batch).reshape(-1).to(torch.int32).contiguous()
        out = _native.gather_qmv(w, scales, biases, x.reshape(-1, x.shape[-1]).contiguous(), idx,
                                 rows_per_x=xs)
        return out.reshape(*batch, 1, int(w.shape[1]))
    return library_gather_matmul(x, w, scales, biases, indices)


class NativeQuantizedSwitchLinear(QuantizedSwitchLinear):
    def forward(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        y = gather_matmul(x, self.weight, self.scales, self.biases, indices, sorted_indices)
        return y + self.bias[indices].unsqueeze(-2) if self.bias is not None else y


def _eligible(module: torch.nn.Module) -> bool:
    if not isinstance(module, (QuantizedLinear, QuantizedEmbedding, QuantizedSwitchLinear)):
        return False
    if module.bits != BITS or module.group_size != GROUP_SIZE or module.biases is None:
        return False
    return module.scales.dtype == torch.bfloat16 and (int(module.weight.shape[-1]) * 8) % 32 == 0


def _probe(module: torch.nn.Module) -> float:
    """Relative error of the kernel on the module's own weight against an fp32 reference:
    max|y - ref| / max|ref| (ironmule/cuda_native.py:253-268)."""
    w, scales, biases = module.weight, module.scales, module.biases
    switch = isinstance(module, QuantizedSwitchLinear)
    if not switch and w.shape[0] > PROBE_ROWS:
        w, scales, biases = w[:PROBE_ROWS], scales[:PROBE_ROWS], biases[:PROBE_ROWS]
    gen = torch.Generator(device=w.device)
    gen.manual_seed(0)
    x = torch.randn((1, int(w.shape[-1]) * 8), generator=gen, device=w.device).to(torch.bfloat16)
    if switch:  # one token against its first eight experts
        experts = torch.arange(min(8, int(w.shape[0])), dtype=torch.int32, device=w.device)
        y = gather_matmul(x.reshape(1, 1, -1), w, scales, biases, experts).reshape(experts.numel(), -1)
        sel = experts.to(torch.long)
        dense = _native.dequant(w[sel].reshape(-1, w.shape[-1]).contiguous(),
                                scales[sel].reshape(-1, scales.shape[-1]).contiguous(),
                                biases[sel].reshape(-1, biases.shape[-1]).contiguous(), torch.float32)
        reference = (x.float() @ dense.T).reshape(experts.numel(), -1)
    else:
        y = _qmv(x, w, scales, biases)
        reference = (x.float() @ _native.dequant(w, scales, biases, torch.float32).T).squeeze(0)
        y = y.squeeze(0)
    error = (y.float() - reference).abs().max()
    return float(error / reference.abs().max().clamp_min(1e-6))


def device_class(device_info: dict[str, Any] | None) -> str | None:
    """The architecture family the plan keys on (gfx950 for MI355X), or None."""
    arch = (device_info or {}).get("gcnArchName") or (device_info or {}).get("arch")
    if isinstance(arch, str) and arch.startswith("gfx950"):
        return "gfx950"
    return None


def head_skip_needed(model: torch.nn.Module, device_info: dict[str, Any] | None) -> str | None:
    """Why the prefill must compute the head for the last position only (its fp16 dequantised
    copy would not fit beside the weights), or None when it fits or nothing is known."""
    info = device_info or {}
    total = next((info[key] for key in ("total_memory", "memory_size", "total_memory_bytes",
                                         "memory_bytes")
                  if isinstance(info.get(key), int) and info[key] > 0), None)
    heads = [m for name, m in model.named_modules()
             if name.rsplit(".", 1)[-1] in ("lm_head", "embed_tokens")
             and isinstance(m, (QuantizedLinear, QuantizedEmbedding)) and m.bits == BITS]
    if total is None or not heads:
        return None
    weights = sum(t.numel() * t.element_size() for t in model.buffers())
    weights += sum(p.numel() * p.element_size() for p in model.parameters())
    copy = max(int(m.weight.shape[0]) * int(m.weight.shape[1]) * 8 * 2 for m in heads)
    if weights + copy <= PREFILL_HEADROOM * total:
        return None
    return (f"the head's float16 prefill copy ({copy / 1e9:.2f} GB) does not fit beside "
            f"{weights / 1e9:.2f} GB of weights in {PREFILL_HEADROOM:.0%} of this card's "
            f"{total / 1e9:.2f} GB, so the head is computed for the last position only")


def install(model: torch.nn.Module, device_info: dict[str, Any] | None) -> dict[str, Any]:
    """Swap every eligible quantised module of `model` to the native kernels, or refuse."""
    if device_class(device_info) != "gfx950":
        raise ValueError("the native plan exists for gfx950 (MI355X) GPUs only")
    modules = [m for _, m in model.named_modules() if _eligible(m)]
    if not modules:
        raise ValueError("the native plan found no 4-bit group-64 affine bfloat16 weights")
    shapes: dict[tuple, torch.nn.Module] = {}
    for module in modules:
        shapes.setdefault((type(module).__name__, tuple(module.weight.shape)), module)
    started = time.perf_counter()
    error = max(_probe(m) for m in shapes.values())
    probe_seconds = time.perf_counter() - started
    if not error <= PROBE_TOLERANCE:
        raise ValueError(f"the native kernel disagrees with the float32 reference ({error:.3g})")
    for module in modules:
        module.__class__ = (NativeQuantizedEmbedding if isinstance(module, QuantizedEmbedding)
                            else NativeQuantizedSwitchLinear if isinstance(module, QuantizedSwitchLinear)
                            else NativeQuantizedLinear)
    return {"modules": len(modules), "probed_shapes": len(shapes), "probe_rel_error": error,
            "probe_seconds": round(probe_seconds, 3)}
