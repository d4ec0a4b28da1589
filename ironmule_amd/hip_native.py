"""The opt-in `native` plan on MI355X: a model's eligible 4-bit modules switch to the
gfx950 kernels after a probe on their own weights.

Call surface of ironmule/cuda_native.py (`matmul`, `gather_matmul`,
`NativeQuantizedLinear`, `NativeQuantizedEmbedding.as_linear`,
`NativeQuantizedSwitchLinear`, `_eligible`, `_probe`, `install`, `head_skip_needed`, and
the thresholds `GATHER_MAX`, `PROBE_ROWS`, `PROBE_TOLERANCE`, `PREFILL_HEADROOM`).  The
reference's plan serves CUDA GPUs below compute capability 8; this one serves gfx950.

Which path a call takes (`_route`, `_gather_route`):

====================================================  =====================================
call                                                  path
====================================================  =====================================
bf16 x with at most MAX_ROWS (32) rows                imq_qmv, one weight sweep for all rows
bf16 x with more rows (prefill)                       imq_dequant to fp16, one GEMM
expert call, one bf16 row per (token, expert) pair,   imq_gather_qmv
at most GATHER_MAX pairs
anything else (fp32 x, larger expert batches)         the module's library path
====================================================  =====================================

The reference's qmv route stops at 8 rows; the gfx950 kernel sweeps the weight once for
up to 32 rows, so the limit here is 32.

`install` keeps everything on one model: it refuses off gfx950 or when nothing is
eligible, probes one module of each (type, weight shape) class against a float32
dequantise-then-matmul reference, and changes module classes only when every probe is
within PROBE_TOLERANCE.
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
#: Largest number of (token, expert) rows the gather kernel takes (ironmule/cuda_native.py:40).
GATHER_MAX = 64
#: Largest max|y - ref| / max|ref| a probe may show (the reference's value).
PROBE_TOLERANCE = 1e-2
#: A probe of a weight taller than this uses its first PROBE_ROWS rows (all of K).
PROBE_ROWS = 8192
#: Share of device memory that weights plus the head's fp16 prefill copy may take.
PREFILL_HEADROOM = 0.9

_HEAD_NAMES = ("lm_head", "embed_tokens")
_MEMORY_KEYS = ("total_memory", "memory_size", "total_memory_bytes", "memory_bytes")


# ------------------------------------------------------------------ routing

def _route(x: torch.Tensor, k: int) -> str:
    if x.dtype != torch.bfloat16:
        return "library"
    return "qmv" if x.numel() // k <= MAX_ROWS else "dequant_gemm"


def _qmv(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
         out_dtype: torch.dtype | None = None) -> torch.Tensor:
    n, k = int(w.shape[0]), int(w.shape[1]) * 8
    y = _native.qmv(w, scales, biases, x.reshape(-1, k).contiguous(),
                    out_dtype=out_dtype or x.dtype)
    return y.reshape(*x.shape[:-1], n)


def matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
           biases: torch.Tensor) -> torch.Tensor:
    """`x @ dequantize(w).T` for a 4-bit, group-64 affine weight with bf16 scales."""
    route = _route(x, int(w.shape[1]) * 8)
    if route == "qmv":
        return _qmv(x, w, scales, biases)
    if route == "dequant_gemm":
        weight16 = _native.dequant(w, scales, biases, torch.float16)
        return torch.matmul(x.to(torch.float16), weight16.T).to(x.dtype)
    return library_matmul(x, w, scales, biases)


def _gather_route(x: torch.Tensor, indices: torch.Tensor):
    """(pairs shape, activation rows per pair group) for the gather kernel, or None.

    The kernel reads activation row `p // rows_per_x` for pair p.  A down projection
    brings one row per pair (rows_per_x = 1); a gate/up projection one row per token,
    shared by its experts along the last index axis (rows_per_x = experts per token).
    Any other broadcast is expanded to one row per pair first."""
    if x.dtype != torch.bfloat16 or x.shape[-2] != 1:
        return None
    pairs = tuple(torch.broadcast_shapes(x.shape[:-2], indices.shape))
    if torch.Size(pairs).numel() > GATHER_MAX:
        return None
    lead = tuple(x.shape[:-2])
    if lead == pairs:
        return pairs, 1
    if pairs and lead == pairs[:-1] + (1,):
        return pairs, pairs[-1]
    return pairs, 0  # 0: expand to one row per pair


def gather_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                  indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
    """`x @ dequantize(w[indices]).T` over stacked experts (mlx's gather_qmm with
    rhs_indices; routing of ironmule/cuda_native.py:199-218).  x is (..., 1, K) per
    token or per pair, w (E, N, K/8); the result is (*pairs, 1, N)."""
    route = _gather_route(x, indices)
    if route is None:
        return library_gather_matmul(x, w, scales, biases, indices)
    pairs, rows_per_x = route
    if rows_per_x == 0:
        x, rows_per_x = x.expand(*pairs, *x.shape[-2:]), 1
    experts = indices.expand(pairs).reshape(-1).to(torch.int32).contiguous()
    rows = x.reshape(-1, x.shape[-1]).contiguous()
    y = _native.gather_qmv(w, scales, biases, rows, experts, rows_per_x=rows_per_x)
    return y.reshape(*pairs, 1, int(w.shape[1]))


class NativeQuantizedLinear(QuantizedLinear):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = matmul(x, self.weight, self.scales, self.biases)
        return y if self.bias is None else y + self.bias


class NativeQuantizedEmbedding(QuantizedEmbedding):
    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        return matmul(x, self.weight, self.scales, self.biases)


class NativeQuantizedSwitchLinear(QuantizedSwitchLinear):
    def forward(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        y = gather_matmul(x, self.weight, self.scales, self.biases, indices, sorted_indices)
        return y if self.bias is None else y + self.bias[indices].unsqueeze(-2)


#: Library class -> native class; a native instance maps to itself.
_NATIVE = {QuantizedLinear: NativeQuantizedLinear,
           QuantizedEmbedding: NativeQuantizedEmbedding,
           QuantizedSwitchLinear: NativeQuantizedSwitchLinear}


def _native_class(module: torch.nn.Module) -> type | None:
    for base in type(module).__mro__:
        if base in _NATIVE:
            return _NATIVE[base]
    return None


# ------------------------------------------------------------------ installation

def _eligible(module: torch.nn.Module) -> bool:
    """A quantised module in the format the kernels take: 4-bit, group 64, affine with
    biases, bf16 scales, K a multiple of 32."""
    if _native_class(module) is None:
        return False
    return (module.bits == BITS and module.group_size == GROUP_SIZE
            and module.biases is not None and module.scales.dtype == torch.bfloat16
            and int(module.weight.shape[-1]) * 8 % 32 == 0)


def _probe_input(k: int, device: torch.device) -> torch.Tensor:
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    return torch.randn((1, k), generator=gen, device=device).to(torch.bfloat16)


def _probe(module: torch.nn.Module) -> float:
    """The kernel's max|y - ref| / max|ref| on one seeded bf16 row and the module's own
    weight, ref = the row in fp32 times imq_dequant's fp32 weight (the measure of
    ironmule/cuda_native.py:253-268).  An expert stack is probed as one token routed to
    its first eight experts; a weight taller than PROBE_ROWS by its first PROBE_ROWS rows."""
    w, scales, biases = module.weight, module.scales, module.biases
    x = _probe_input(int(w.shape[-1]) * 8, w.device)
    if isinstance(module, QuantizedSwitchLinear):
        chosen = torch.arange(min(8, int(w.shape[0])), device=w.device)
        got = gather_matmul(x.reshape(1, 1, -1), w, scales, biases, chosen.to(torch.int32))
        w, scales, biases = (t[chosen].flatten(0, 1).contiguous() for t in (w, scales, biases))
    else:
        w, scales, biases = w[:PROBE_ROWS], scales[:PROBE_ROWS], biases[:PROBE_ROWS]
        got = _qmv(x, w, scales, biases)
    ref = x.float() @ _native.dequant(w, scales, biases, torch.float32).T
    scale = ref.abs().max().clamp_min(1e-6)
    return float((got.float().reshape(ref.shape) - ref).abs().max() / scale)


def device_class(device_info: dict[str, Any] | None) -> str | None:
    """"gfx950" when the device description names that architecture, else None."""
    info = device_info or {}
    arch = info.get("gcnArchName") or info.get("arch")
    return "gfx950" if isinstance(arch, str) and arch.startswith("gfx950") else None


def install(model: torch.nn.Module, device_info: dict[str, Any] | None) -> dict[str, Any]:
    """Switch `model`'s eligible modules to the native kernels, or raise ValueError and
    leave them as they are.  Returns the module count, the probed shape classes, the
    worst probe error and the probing time."""
    if device_class(device_info) != "gfx950":
        raise ValueError("the native plan needs a gfx950 (MI355X) device")
    modules = [m for m in model.modules() if _eligible(m)]
    if not modules:
        raise ValueError("the native plan found no 4-bit group-64 affine bfloat16 weights")
    classes = {(type(m).__name__, tuple(m.weight.shape)): m for m in reversed(modules)}
    started = time.perf_counter()
    worst = max(_probe(m) for m in classes.values())
    elapsed = time.perf_counter() - started
    if not worst <= PROBE_TOLERANCE:
        raise ValueError(f"the native kernel disagrees with the float32 reference by "
                         f"{worst:.3g} (tolerance {PROBE_TOLERANCE:g})")
    for module in modules:
        module.__class__ = _native_class(module)
    return {"modules": len(modules), "probed_shapes": len(classes), "probe_rel_error": worst,
            "probe_seconds": round(elapsed, 3)}


# ------------------------------------------------------------------ prefill memory

def _device_memory(info: dict[str, Any]) -> int | None:
    for key in _MEMORY_KEYS:
        value = info.get(key)
        if isinstance(value, int) and value > 0:
            return value
    return None


def head_skip_needed(model: torch.nn.Module, device_info: dict[str, Any] | None) -> str | None:
    """A reason to compute the prefill's output head for the last position only, or None.

    The prefill route dequantises a weight to fp16 for its GEMM; for the head (lm_head or
    a tied embed_tokens) that copy is N*K*2 bytes.  When the model's tensors plus the
    largest such copy exceed PREFILL_HEADROOM of device memory, the reason says so.
    Nothing is decided (None) when the device reports no memory size or the model has
    no 4-bit head."""
    total = _device_memory(device_info or {})
    heads = [m for name, m in model.named_modules()
             if name.rsplit(".", 1)[-1] in _HEAD_NAMES
             and isinstance(m, (QuantizedLinear, QuantizedEmbedding)) and m.bits == BITS]
    if total is None or not heads:
        return None
    tensors = [*model.parameters(), *model.buffers()]
    resident = sum(t.numel() * t.element_size() for t in tensors)
    head_copy = max(int(m.weight.shape[0]) * int(m.weight.shape[1]) * 8 * 2 for m in heads)
    budget = PREFILL_HEADROOM * total
    if resident + head_copy <= budget:
        return None
    return (f"{resident / 1e9:.2f} GB of weights and the head's {head_copy / 1e9:.2f} GB fp16 "
            f"prefill copy exceed {budget / 1e9:.2f} GB ({PREFILL_HEADROOM:.0%} of "
            f"{total / 1e9:.2f} GB), so the prefill computes the head at the last position only")
