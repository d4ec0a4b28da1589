"""Torch stand-ins for the library's quantised modules, on the reference's weight format.

The reference's hot path swaps MLX modules (`nn.QuantizedLinear`, `nn.QuantizedEmbedding`)
for kernel-backed ones and falls back to the *original* module whenever a call is not
one it admits (ironmule/qmv_k3840.py:313-342, ironmule/qmv_variant.py:99-129).  These
classes are that original module here: same buffers (packed uint32 words as int32,
bf16 scales and biases, group size, bits), and a library path that runs on the GPU:

* up to 32 activation rows: the qmv kernel (libironmule_qmv.so, imq_qmv), as MLX's own
  `quantized_matmul` runs its qmv kernel for few rows;
* more rows (prefill): the weight dequantised by imq_dequant, then a torch GEMM
  (hipBLASLt), as the reference's prefill does (ironmule/cuda_native.py:177-179).

There is no CPU path: the forward fails loudly without a GPU and the HIP library.

`quantize` is this build's own affine quantiser (per group of 64: scale = (max-min)/15,
bias = min, both rounded to bf16, q = round((w - bias) / scale) clamped to 0..15).  MLX's
quantiser is not reproduced (it is third-party and not needed: the benchmark weights are
synthesised directly in the packed format).
"""

from __future__ import annotations

import torch

from . import _native

GROUP_SIZE = 64
BITS = 4


def quantize(weight: torch.Tensor, group_size: int = GROUP_SIZE, bits: int = BITS):
    """Dense (N, K) weight -> (packed int32 (N, K/8), bf16 scales, bf16 biases)."""
    if bits != BITS or group_size != GROUP_SIZE:
        raise ValueError("only 4-bit, group-64 affine quantisation is supported")
    n, k = weight.shape
    if k % group_size:
        raise ValueError(f"K={k} is not a multiple of {group_size}")
    w = weight.detach().to(torch.float32).reshape(n, k // group_size, group_size)
    lo = w.amin(dim=-1)
    hi = w.amax(dim=-1)
    scale = ((hi - lo) / 15.0).clamp_min(1e-8).to(torch.bfloat16)
    bias = lo.to(torch.bfloat16)
    q = torch.round((w - bias.float()[..., None]) / scale.float()[..., None]).clamp(0, 15)
    q = q.to(torch.int64).reshape(n, k // 8, 8)
    shifts = (4 * torch.arange(8, device=q.device, dtype=torch.int64))
    words = (q << shifts).sum(dim=-1)  # low nibble first
    packed = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return packed, scale, bias


def unpack(w: torch.Tensor) -> torch.Tensor:
    """Packed (N, K/8) words -> (N, K) uint8 nibbles, low nibble first (host helper)."""
    u = w.to(torch.int64) & 0xFFFFFFFF
    shifts = 4 * torch.arange(8, device=w.device, dtype=torch.int64)
    return ((u[..., None] >> shifts) & 0xF).reshape(*w.shape[:-1], w.shape[-1] * 8).to(torch.uint8)


class QuantizedLinear(torch.nn.Module):
    """A 4-bit, group-64 affine linear layer: y = x @ (scales*q + biases).T (+ bias)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = GROUP_SIZE,
                 bits: int = BITS) -> None:
        super().__init__()
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None
        self.group_size = int(group_size)
        self.bits = int(bits)

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear, group_size: int = GROUP_SIZE,
                    bits: int = BITS) -> "QuantizedLinear":
        w, s, b = quantize(linear.weight, group_size, bits)
        bias = linear.bias.detach().to(torch.bfloat16) if linear.bias is not None else None
        return cls(w, s, b, bias, group_size, bits)

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[1]) * 32 // self.bits

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = library_matmul(x, self.weight, self.scales, self.biases, self.group_size, self.bits)
        return y + self.bias if self.bias is not None else y


class QuantizedEmbedding(torch.nn.Module):
    """A 4-bit embedding table that can also serve as a tied output head (as_linear)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = GROUP_SIZE, bits: int = BITS) -> None:
        super().__init__()
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.group_size = int(group_size)
        self.bits = int(bits)

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        rows = tokens.reshape(-1)
        w, s, b = self.weight[rows].contiguous(), self.scales[rows].contiguous(), \
            self.biases[rows].contiguous()
        dense = _native.dequant(w, s, b, torch.float32)
        return dense.to(torch.bfloat16).reshape(*tokens.shape, -1)

    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        return library_matmul(x, self.weight, self.scales, self.biases, self.group_size, self.bits)


def library_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                   group_size: int = GROUP_SIZE, bits: int = BITS) -> torch.Tensor:
    """The library path: qmv for up to 32 bf16 rows, dequantise + GEMM beyond."""
    if group_size != GROUP_SIZE or bits != BITS:
        raise ValueError("only 4-bit, group-64 weights are supported")
    if not x.is_cuda:
        raise _native.NativeUnavailable("the quantised layers run on the GPU only")
    k = int(w.shape[1]) * 8
    lead = x.shape[:-1]
    rows = x.reshape(-1, k)
    if x.dtype == torch.bfloat16 and rows.shape[0] <= _native.MAX_ROWS:
        y = _native.qmv(w, scales, biases, rows.contiguous())
    else:
        dense = _native.dequant(w, scales, biases, torch.float32)
        y = (rows.to(torch.float32) @ dense.T).to(x.dtype)
    return y.reshape(*lead, int(w.shape[0]))


class QuantizedSwitchLinear(torch.nn.Module):
    """A stack of `experts` 4-bit group-64 affine weights, (E, N, K/8) packed words with
    (E, N, K/64) bf16 scales and biases (mlx-lm's QuantizedSwitchLinear layout); the call
    takes activations and each row's expert indices."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = GROUP_SIZE,
                 bits: int = BITS) -> None:
        super().__init__()
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)
        self.group_size = int(group_size)
        self.bits = int(bits)

    @property
    def num_experts(self) -> int:
        return int(self.weight.shape[0])

    def forward(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        y = library_gather_matmul(x, self.weight, self.scales, self.biases, indices,
                                  self.group_size, self.bits)
        return y + self.bias[indices].unsqueeze(-2) if self.bias is not None else y


def library_gather_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                          biases: torch.Tensor, indices: torch.Tensor,
                          group_size: int = GROUP_SIZE, bits: int = BITS) -> torch.Tensor:
    """The library gather path: every selected expert dequantised to fp32 and one batched
    product, (*batch, M, K) x experts -> (*batch, M, N), batch = broadcast(x.shape[:-2],
    indices.shape)."""
    if group_size != GROUP_SIZE or bits != BITS:
        raise ValueError("only 4-bit, group-64 weights are supported")
    if not x.is_cuda:
        raise _native.NativeUnavailable("the quantised layers run on the GPU only")
    batch = torch.broadcast_shapes(x.shape[:-2], indices.shape)
    xb = x.expand(*batch, *x.shape[-2:]).reshape(-1, x.shape[-2], x.shape[-1])
    idx = indices.expand(batch).reshape(-1).to(torch.long)
    dense = _native.dequant(w[idx].reshape(-1, w.shape[-1]).contiguous(),
                            scales[idx].reshape(-1, scales.shape[-1]).contiguous(),
                            biases[idx].reshape(-1, biases.shape[-1]).contiguous(), torch.float32)
    dense = dense.reshape(idx.numel(), int(w.shape[1]), -1)
    y = torch.bmm(xb.to(torch.float32), dense.transpose(1, 2).contiguous())
    return y.to(x.dtype).reshape(*batch, x.shape[-2], int(w.shape[1]))
