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


def oracle_decoder(do, orc, weights, lazy: bool = False):
    """The decode oracle's Model for a `decode.DecoderWeights` on the GPU: every projection
    and the tied embedding dequantised to float64 by the oracle, norms widened from bf16.
    With `lazy` the layers are dequantised one at a time as the oracle walks them (a
    36-layer Qwen3-4B in float64 would take 32 GB at once)."""
    import numpy as np

    def vals(t):
        return t.float().cpu().numpy().astype(np.float64)

    def deq(q):
        w, s, b = (t.cpu() for t in q)
        return orc.dequant_f32(w.numpy().view(np.uint32), s.view(torch.int16).numpy().view(np.uint16),
                               b.view(torch.int16).numpy().view(np.uint16)).astype(np.float64)

    def layer(L):
        return do.Layer(wq=deq(L["q"]), wk=deq(L["k"]), wv=deq(L["v"]), wo=deq(L["o"]),
                        wg=deq(L["gate"]), wu=deq(L["up"]), wd=deq(L["down"]),
                        input_norm=vals(L["input_norm"]), post_norm=vals(L["post_norm"]),
                        q_norm=vals(L["q_norm"]), k_norm=vals(L["k_norm"]))

    class _Layers:
        def __len__(self):
            return len(weights.layers)

        def __iter__(self):
            for L in weights.layers:
                yield layer(L)

    c = weights.config
    layers = _Layers() if lazy else [layer(L) for L in weights.layers]
    return do.Model(layers=layers, embed=deq(weights.embed), norm=vals(weights.norm),
                    heads=c.heads, kv_heads=c.kv_heads, eps=c.eps, theta=c.theta)


def logit_error(got, ref):
    """max|got - ref| / max|ref| over one request's logits."""
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / np.abs(ref).max())


def oracle_gemma3(do, orc, weights):
    """The decode oracle's Gemma3Model for a `gemma3.Gemma3Weights` on the GPU: every
    projection and the tied embedding dequantised to float64 by the oracle (the layers one
    at a time as the oracle walks them), norm weights widened from bf16."""
    import numpy as np

    def vals(t):
        return t.float().cpu().numpy().astype(np.float64)

    def deq(q):
        w, s, b = (t.cpu() for t in q)
        return orc.dequant_f32(w.numpy().view(np.uint32), s.view(torch.int16).numpy().view(np.uint16),
                               b.view(torch.int16).numpy().view(np.uint16)).astype(np.float64)

    def layer(L):
        return do.Gemma3Layer(wq=deq(L["q"]), wk=deq(L["k"]), wv=deq(L["v"]), wo=deq(L["o"]),
                              wg=deq(L["gate"]), wu=deq(L["up"]), wd=deq(L["down"]),
                              input_norm=vals(L["input_norm"]), post_attn_norm=vals(L["post_attn_norm"]),
                              pre_ff_norm=vals(L["pre_ff_norm"]), post_ff_norm=vals(L["post_ff_norm"]),
                              q_norm=vals(L["q_norm"]), k_norm=vals(L["k_norm"]))

    class _Layers:
        def __iter__(self):
            for L in weights.layers:
                yield layer(L)

    c = weights.config
    return do.Gemma3Model(layers=_Layers(), embed=deq(weights.embed), norm=vals(weights.norm),
                          heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim, eps=c.eps,
                          theta_global=c.theta_global, theta_local=c.theta_local, window=c.window,
                          pattern=c.pattern, query_scalar=c.query_scalar)

