"""Helpers shared by the GPU tests: numpy bit patterns <-> torch device tensors."""

from __future__ import annotations

import numpy as np
import torch


def to_device(pr, device: str = "cuda"):
    """(w int32, s bf16, b bf16, x bf16) device tensors holding the problem's bits."""
    w = torch.from_numpy(np.ascontiguousarray(pr.w).view(np.int32)).to(device)
    s = torch.from_numpy(np.ascontiguousarray(pr.s)).view(torch.bfloat16).to(device)
    b = torch.from_numpy(np.ascontiguousarray(pr.b)).view(torch.bfloat16).to(device)
    x = torch.from_numpy(np.ascontiguousarray(pr.x)).view(torch.bfloat16).to(device)
    return w, s, b, x


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def announce(*parts) -> None:
    """Name the case before a GPU step, flushed, so a failure can be placed."""
    print("[gpu case]", *parts, flush=True)
