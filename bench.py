"""Benchmark of the 4-bit affine group-64 qmv on one MI355X.

Default workload (the headline): one Qwen3-4B-shaped decoder layer, all seven
projections as 4-bit qmv at batch 1 (q 2560->4096, k/v 2560->1024, o 4096->2560,
gate/up 2560->9728, down 9728->2560), seeded random weights, bf16 activations.
A step is one pass over one layer's seven projections; consecutive steps rotate over
36 distinct layer copies (2.05 GB, one Qwen3-4B's worth), so every step streams its
weights from HBM rather than the 256 MB last-level cache.  The streaming engine runs the
36 layers' projections in one persistent launch (independent stages in decode order),
captured in a HIP graph; inputs are resident in HBM.

Prints one JSON line.  `value` = algorithmic bytes moved per step (packed weights +
bf16 scales/biases + x + y) / GPU time per step, in GB/s.  `roofline` is the streaming
kernel (the only kernel of the timed steps): algorithmic bytes per launch over its mean
launch time from HIP events on its own stream.  The layer breakdown times the same
layers as per-kernel launches, as one grouped launch per layer, and through the
streaming engine with decode-order dependencies.  `decode` times the full synthetic
Qwen3-4B decode step at batch 1 and 32.  `cpu_baseline` times the oracle's restatement of
the reference row kernel on the host cores (rank 0, N=1 only).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
LAYER = [("q", 4096, 2560), ("k", 1024, 2560), ("v", 1024, 2560), ("o", 2560, 4096),
         ("gate", 9728, 2560), ("up", 9728, 2560), ("down", 2560, 9728)]
LAYERS = 36
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
SEED = 20261201


def qmv_bytes(n: int, k: int, m: int, y_bytes: int = 2) -> int:
    """Algorithmic bytes of one call: packed w, bf16 scales and biases, x, y."""
    return n * k // 2 + n * (k // 64) * 4 + m * k * 2 + m * n * y_bytes


def weight_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * (k // 64) * 4


def make_weight(torch, n, k, gen, device):
    w = torch.randint(0, 2**32, (n, k // 8), dtype=torch.int64, device=device,
                      generator=gen).to(torch.int32)
    s = torch.empty((n, k // 64), device=device).uniform_(0.005, 0.02, generator=gen)
    b = torch.empty((n, k // 64), device=device).uniform_(-0.1, 0.1, generator=gen)
    return w, s.to(torch.bfloat16), b.to(torch.bfloat16)


def make_x(torch, m, k, gen, device):
    return torch.randn((m, k), device=device, generator=gen).to(torch.bfloat16)


class GraphRunner:
    """Captures a list of launch closures into one HIP graph on a side stream."""

    def __init__(self, torch, launches, stream):
        self.torch = torch
        self.stream = stream
        with torch.cuda.stream(stream):
            for fn in launches:  # eager warm-up (first-use device set-up happens here)
                fn()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            for fn in launches:
                fn()
        torch.cuda.synchronize()

    def replay(self):
        with self.torch.cuda.stream(self.stream):
            self.graph.replay()


class DirectRunner:
    """The same launch closures issued straight onto the stream, no graph: a graph replay
    in the timed position measured about 8 us more per replay than the same kernel
    launched directly behind the work ahead of it (20-layer streaming program: 188.2 against
    180.5 us on one MI355X), the graph launch's own cost rather than the kernel's."""

    def __init__(self, torch, launches, stream):
        self.torch = torch
        self.stream = stream
        self.launches = launches

    def replay(self):
        with self.torch.cuda.stream(self.stream):
            for fn in self.launches:
                fn()


def time_graph(torch, runner, repeats, stream):
    """Seconds per replay: events on the graph's own stream around `repeats` replays,
    queued behind one untimed replay so the GPU never waits on the host inside them."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    runner.replay()
    start.record(stream)
    for _ in range(repeats):
        runner.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / repeats


def warm_up(torch, runner, stream, min_seconds=0.2, max_seconds=3.0, tol=0.01, batch=4):
    """Replays `runner` until at least `min_seconds` have passed and two successive timed
    batches of `batch` replays agree within `tol`: the GPU's clocks ramp over tens of
    milliseconds, so a fixed count of short replays would time the ramp (the reference's
    GEMV probe also warms up before it takes the median of repeats, ironmule/hw.py:421-438).
    Returns what was done, for the result line."""
    t0 = time.perf_counter()
    prev, replays = None, 0
    while True:
        sec = time_graph(torch, runner, batch, stream)
        replays += batch
        elapsed = time.perf_counter() - t0
        settled = prev is not None and abs(sec - prev) <= tol * prev
        if (elapsed >= min_seconds and settled) or elapsed >= max_seconds:
            return {"replays": replays, "seconds": round(elapsed, 3), "settled": settled,
                    "last_replay_us": round(sec * 1e6, 3)}
        prev = sec


# The layer in decode order: launches that read the same activation share one launch.
LAUNCHES = [("qkv", ["q", "k", "v"], 2560), ("o", ["o"], 4096), ("gate_up", ["gate", "up"], 2560),
            ("down", ["down"], 9728)]


def _layer_stages(layers, xs, ys, index, chained=False):
    """The stages of `layers` in decode order (q/k/v, o, gate/up, down) for the streaming
    engine.  Independent: every stage reads the fixed x of its K.  Chained: every stage
    waits for the one before it and reads its output, as a decode step does (o reads q,
    gate/up read o, down reads gate, the next layer's q/k/v read down)."""
    stages = []
    if not chained:
        for L in layers:
            for (_, names, k) in LAUNCHES:
                stages.append(([L[index[nm]] for nm in names], xs[k], [ys[nm] for nm in names],
                               False))
        return stages
    import torch
    h = xs[2560]
    for li, L in enumerate(layers):
        dev = h.device
        yq = [torch.empty(n, dtype=torch.bfloat16, device=dev) for n in (4096, 1024, 1024)]
        yo = [torch.empty(2560, dtype=torch.bfloat16, device=dev)]
        yg = [torch.empty(9728, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        yd = [torch.empty(2560, dtype=torch.bfloat16, device=dev)]
        stages += [([L[index["q"]], L[index["k"]], L[index["v"]]], h.reshape(-1), yq, li > 0),
                   ([L[index["o"]]], yq[0], yo, True),
                   ([L[index["gate"]], L[index["up"]]], yo[0], yg, True),
                   ([L[index["down"]]], yg[0], yd, True)]
        h = yd[0]
    return stages


STAGE_NAMES = ("q/k/v", "o", "gate/up", "down")


def chain_trace(torch, native, device, layers_n=LAYERS, repeats=3):
    """Where a chained streaming launch (the layer breakdown's `stream_chained`: the
    decode-order stages of `layers_n` Qwen3-4B layers at batch 1, each waiting for the one
    before it) spends its time, from the kernel's per-(stage, wavefront) stamps
    (imq_stream_trace, a 100 MHz clock): for each stage kind, medians over the layers after
    the first of
      signal   a wavefront's last tile of the previous stage -> this stage's start (its
               workgroup's barrier, the stores' acknowledgement and the counter add);
      wait     start -> input ready (every workgroup of the previous stage counted);
      x        input ready -> x staged in LDS (sc1 loads of the previous stage's output);
      compute  x staged -> last tile done (the stage's tiles, dealt in turn);
      tail     the stage's slowest wavefront done - its median wavefront done;
      period   median input ready of this stage -> of the next stage."""
    gen = torch.Generator(device=device)
    gen.manual_seed(SEED + 1)
    index = {name: i for i, (name, _, _) in enumerate(LAYER)}
    layers = [[make_weight(torch, n, k, gen, device) for (_, n, k) in LAYER]
              for _ in range(layers_n)]
    xs = {k: make_x(torch, 1, k, gen, device) for k in {k for (_, _, k) in LAYER}}
    xrow = {k: v.reshape(-1) for k, v in xs.items()}
    stream = torch.cuda.Stream(device=device)
    prog = native.stream_program(_layer_stages(layers, xrow, None, index, chained=True))
    info = prog.info()
    waves = info["workgroups"] * 12
    nst = info["stages"]
    buf = torch.zeros(nst * waves * 4, dtype=torch.int64, device=device)
    for _ in range(20):
        prog.launch(stream)
    torch.cuda.synchronize()
    runs = []
    for _ in range(repeats):
        buf.zero_()
        prog.trace(buf)
        prog.launch(stream)
        torch.cuda.synchronize()
        prog.trace(None)
        if prog.failed():
            raise SystemExit("the chained launch stopped on a bounded wait")
        runs.append(buf.view(nst, waves, 4).cpu().numpy().astype("float64") * 0.01)  # us
    import numpy as np
    kinds = {name: {"signal": [], "wait": [], "x": [], "compute": [], "tail": [], "period": []}
             for name in STAGE_NAMES}
    launch_us = []
    for t in runs:
        launch_us.append(float(t[:, :, 3].max() - t[0, :, 0].min()))
        for s in range(4, nst - 1):  # the layers after the first, up to the last stage
            d = kinds[STAGE_NAMES[s % 4]]
            d["signal"].append(float(np.median(t[s, :, 0] - t[s - 1, :, 3])))
            d["wait"].append(float(np.median(t[s, :, 1] - t[s, :, 0])))
            d["x"].append(float(np.median(t[s, :, 2] - t[s, :, 1])))
            d["compute"].append(float(np.median(t[s, :, 3] - t[s, :, 2])))
            d["tail"].append(float(t[s, :, 3].max() - np.median(t[s, :, 3])))
            d["period"].append(float(np.median(t[s + 1, :, 1]) - np.median(t[s, :, 1])))
    summary = {name: {k: round(float(np.median(v)), 2) for k, v in d.items()}
               for name, d in kinds.items()}
    per_layer = sum(v["period"] for v in summary.values())
    prog.close()
    del layers
    torch.cuda.empty_cache()
    return {"metric": "chained streaming launch, per-stage time (us, medians)",
            "layers": layers_n, "workgroups": info["workgroups"], "stages": nst,
            "launch_us": round(float(np.median(launch_us)), 1),
            "per_layer_us": round(per_layer, 2), "by_stage": summary}


def bench_layer(torch, native, steps, warmup, device, breakdown=True):
    """The headline: K steps of one layer's seven projections, rotating over 36 distinct
    layers, streamed by the streaming engine: one launch runs 36 layers' projections as
    independent stages (as in the reference's bandwidth measurement over chained distinct
    weights, ironmule/hw.py:441-473).  The breakdown times the same layers as per-kernel
    launches in decode order, all seven projections in one grouped launch, and the
    streaming engine with decode-order dependencies."""
    gen = torch.Generator(device=device)
    gen.manual_seed(SEED + 1)
    index = {name: i for i, (name, _, _) in enumerate(LAYER)}
    layers = [[make_weight(torch, n, k, gen, device) for (_, n, k) in LAYER]
              for _ in range(LAYERS)]
    xs = {k: make_x(torch, 1, k, gen, device) for k in {k for (_, _, k) in LAYER}}
    ys = {name: torch.empty((1, n), dtype=torch.bfloat16, device=device)
          for (name, n, _) in LAYER}
    stream = torch.cuda.Stream(device=device)
    xrow = {k: v.reshape(-1) for k, v in xs.items()}
    yrow = {k: v.reshape(-1) for k, v in ys.items()}

    full_prog = native.stream_program(_layer_stages(layers, xrow, yrow, index))
    full = DirectRunner(torch, [lambda: full_prog.launch(stream)], stream)
    part_n = steps % LAYERS
    part_prog = native.stream_program(_layer_stages(layers[:part_n], xrow, yrow, index)) if part_n else None
    part = DirectRunner(torch, [lambda: part_prog.launch(stream)], stream) if part_n else None
    # at least `warmup` layers, and in any case until the launch time has settled
    for _ in range(warmup // LAYERS + (1 if warmup % LAYERS else 0)):
        full.replay()
    warm = warm_up(torch, full, stream)
    if part is not None:
        part.replay()  # the first launch of the partial program is not timed
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # One untimed launch ahead of the start event keeps the GPU busy while the host queues
    # the event and the timed launches behind it, so the timed region holds GPU work only
    # (not the host's submission latency).
    full.replay()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps // LAYERS):
        full.replay()
    if part is not None:
        part.replay()
    end.record(stream)
    end.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = start.elapsed_time(end) / 1e3
    step_bytes = sum(qmv_bytes(n, k, 1) for (_, n, k) in LAYER)
    launches = steps // LAYERS + (1 if part_n else 0)
    info = full_prog.info()
    out = {"gpu_s": gpu_s, "wall_s": wall, "step_bytes": step_bytes, "launches": launches,
           "workgroups": info["workgroups"], "launch_bytes": step_bytes * LAYERS,
           "avg_launch_s": gpu_s / launches if not part_n else None, "warm_up": warm}
    if part_n == 0:
        out["avg_launch_s"] = gpu_s / launches
    else:  # the full-program launches alone, for the per-launch figure
        out["avg_launch_s"] = time_graph(torch, full, 10, stream)
    if not breakdown:
        del full, part, full_prog, part_prog, layers
        torch.cuda.empty_cache()
        return out

    # each launch type alone: 36 back-to-back per-kernel launches over distinct weights
    def launch(i, names, k):
        weights = [layers[i][index[nm]] for nm in names]
        outs = [ys[nm] for nm in names]
        return lambda: native.qmv_grouped(weights, [xs[k]] * len(names), outs=outs, stream=stream)

    per_launch = {}
    for (lname, names, k) in LAUNCHES:
        runner = GraphRunner(torch, [launch(i, names, k) for i in range(LAYERS)], stream)
        runner.replay()
        sec = time_graph(torch, runner, 20, stream) / LAYERS
        nbytes = sum(qmv_bytes(n, kk, 1) for (nm, n, kk) in LAYER if nm in names)
        per_launch[lname] = {"us": sec * 1e6, "gbs": nbytes / sec / 1e9, "bytes": nbytes}
        del runner
    runner = GraphRunner(torch, [fn for i in range(LAYERS)
                                 for fn in (launch(i, names, k) for (_, names, k) in LAUNCHES)], stream)
    runner.replay()
    sec = time_graph(torch, runner, 20, stream) / LAYERS
    decode_order = {"us": sec * 1e6, "gbs": step_bytes / sec / 1e9}
    del runner

    # all seven projections of a layer in one launch (they are independent here)
    runner = GraphRunner(torch, [
        (lambda i=i: native.qmv_grouped(layers[i], [xs[k] for (_, _, k) in LAYER],
                                        outs=[ys[nm] for (nm, _, _) in LAYER], stream=stream))
        for i in range(LAYERS)], stream)
    runner.replay()
    sec = time_graph(torch, runner, 20, stream) / LAYERS
    one_launch = {"us": sec * 1e6, "gbs": step_bytes / sec / 1e9}
    del runner

    # the streaming engine with decode-order dependencies between the stages
    chain_prog = native.stream_program(_layer_stages(layers, xrow, yrow, index, chained=True))
    runner = GraphRunner(torch, [lambda: chain_prog.launch(stream)], stream)
    runner.replay()
    sec = time_graph(torch, runner, 10, stream) / LAYERS
    chained = {"us": sec * 1e6, "gbs": step_bytes / sec / 1e9, "stalled": chain_prog.failed()}
    del runner, chain_prog, full, part, full_prog, part_prog, layers
    torch.cuda.empty_cache()
    out.update({"per_launch": per_launch, "decode_order": decode_order, "one_launch": one_launch,
                "chained": chained})
    return out


def bench_config(torch, native, n, k, ms, y_dtype, copies, device, seed, repeats=10):
    """Rotating copies (>= 1 GiB total) of one (N, K) weight, one graph per M."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    ws = [make_weight(torch, n, k, gen, device) for _ in range(copies)]
    stream = torch.cuda.Stream(device=device)
    out = {}
    ybytes = 4 if y_dtype == torch.float32 else 2
    for m in ms:
        x = make_x(torch, m, k, gen, device)
        y = torch.empty((m, n), dtype=y_dtype, device=device)
        runner = GraphRunner(torch, [
            (lambda w=w, s=s, b=b: native.qmv(w, s, b, x, out=y, stream=stream))
            for (w, s, b) in ws], stream)
        warm_up(torch, runner, stream, min_seconds=0.05, batch=2)
        sec = time_graph(torch, runner, repeats, stream) / copies
        out[str(m)] = {"us": sec * 1e6, "gbs": qmv_bytes(n, k, m, ybytes) / sec / 1e9,
                       "weight_gbs": weight_bytes(n, k) / sec / 1e9}
        if m >= 3:  # the MFMA path: algorithmic 2 M N K flops against the dense bf16 peak
            tflops = 2.0 * m * n * k / sec / 1e12
            out[str(m)].update({"tflops": tflops, "mfma_frac": tflops / MFMA_BF16_PEAK_TFLOPS})
        del runner
    del ws
    torch.cuda.empty_cache()
    return out


CONTEXT = 512  # tokens already in every request's KV slot


def bench_prefill(torch, weights, device, gen, count: int = CONTEXT, repeats: int = 3):
    """Wall time of `decode.prefill` over a `count`-token prompt (one request), median of
    `repeats` runs after one untimed run; the host-side prompt upload is included, as in
    a serving engine's time to first token."""
    from ironmule_amd.decode import DecodeState, prefill

    cfg = weights.config
    state = DecodeState(cfg, batch=1, slots=1, capacity=count + 8, max_len=count + 8,
                        device=device)
    tokens = torch.randint(0, cfg.vocab, (count,), generator=gen, device=device).tolist()
    times = []
    for trial in range(repeats + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prefill(weights, state, tokens, 0)
        torch.cuda.synchronize()
        if trial:
            times.append(time.perf_counter() - t0)
    del state
    torch.cuda.empty_cache()
    sec = sorted(times)[len(times) // 2]
    return {"tokens": count, "ms": round(sec * 1e3, 3), "ns": int(sec * 1e9),
            "tokens_per_s": round(count / sec, 1),
            "path": "imq_dequant to fp16 + GEMM per projection, fp32 causal attention, "
                    "head at the last position only"}


def _epilogue_launches(weights, batch: int) -> int:
    """Residual-epilogue launches per layer of the fused-norm step at `batch` rows: one after
    each of o and down where it splits K (decode._residual_projection)."""
    import torch

    from ironmule_amd import _native
    from ironmule_amd.decode import RESIDUAL_BANDS_MAX_K
    layer = weights.layers[0]
    count = 0
    c = weights.config
    for name, k in (("o", c.heads * c.head_dim), ("down", c.intermediate)):
        if k % 256 == 0 and k <= RESIDUAL_BANDS_MAX_K:
            continue  # over bands of rows and the whole K: one launch
        x = torch.empty((batch, k), dtype=torch.bfloat16, device=layer[name][0].device)
        if 2 <= _native.residual_split_planes(layer[name], x) <= _native.RESIDUAL_MAX_PLANES:
            count += 1
    return count


def bench_decode(torch, batches=(1, 32), steps: int = 30, warmup: int = 5, device="cuda:0",
                 seed: int = SEED + 4, prefill_tokens: bool = True):
    """Full synthetic Qwen3-4B decode step (36 layers of 4-bit projections + the 151,936-
    token tied head, GQA attention over a 512-token KV context per request), as one HIP
    graph per batch size; returns tokens/s and the weight + KV bytes per step."""
    from ironmule_amd.decode import (FUSED_NORM_ROWS, DecodeState, DecoderConfig, PersistentDecode,
                                     decode_step, random_weights)

    cfg = DecoderConfig()
    weights = random_weights(cfg, device, seed=seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed + 1)
    out = {"prefill": bench_prefill(torch, weights, device, gen)} if prefill_tokens else {}
    for b in batches:
        state = DecodeState(cfg, batch=b, slots=b, capacity=CONTEXT + 8, max_len=CONTEXT + 8,
                            device=device)
        for pool in state.k_pool + state.v_pool:
            pool.copy_(torch.randn(pool.shape, device=device, generator=gen).to(torch.bfloat16))
        state.set_requests(torch.randint(0, cfg.vocab, (b,), generator=gen, device=device).tolist(),
                           list(range(b)), [CONTEXT] * b)
        stream = torch.cuda.Stream(device=device)
        # launches per step: the embedding, the layers, the final norm and the head; from
        # FUSED_NORM_ROWS requests the RMSNorms run inside the projections (five launches per
        # layer, the residual epilogues of o and down as two more where those projections
        # split K, and one more for the first layer's input norm), below it eight per layer
        # (seven from 5 requests, where gate/up and SiLU * up are one launch)
        per_layer = (5 + _epilogue_launches(weights, b)) if b >= FUSED_NORM_ROWS else (7 if b >= 5 else 8)
        extra = 4 if b >= FUSED_NORM_ROWS else 3
        paths = {"per_kernel": (lambda: decode_step(weights, state, stream=stream),
                                extra + cfg.layers * per_layer)}
        if b == 1:
            staged = PersistentDecode(weights, state, staged=True)
            paths["staged_program"] = (lambda: staged.step(stream), 2 + cfg.layers * 5)
        kv_bytes = cfg.layers * b * cfg.kv_heads * (CONTEXT + 1) * cfg.head_dim * 2 * 2
        times = {}
        for name, (fn, launches) in paths.items():
            runner = GraphRunner(torch, [fn], stream)
            for _ in range(warmup):
                runner.replay()
            warm_up(torch, runner, stream, min_seconds=0.1)
            times[name] = (time_graph(torch, runner, steps, stream), launches)
            del runner
        best = min(times, key=lambda k: times[k][0])
        sec, launches = times[best]
        out[str(b)] = {"ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(b / sec, 1),
                       "timed_steps": steps, "seconds_per_step": sec,
                       "weight_gbs": round(cfg.weight_bytes() / sec / 1e9, 1),
                       "weight_plus_kv_gbs": round((cfg.weight_bytes() + kv_bytes) / sec / 1e9, 1),
                       "path": best, "launches_per_step": launches,
                       "paths_ms": {k: round(v[0] * 1e3, 4) for k, v in times.items()}}
        del state
        torch.cuda.empty_cache()
    del weights
    torch.cuda.empty_cache()
    return out


def decode_traffic(cfg, batch: int) -> dict:
    """Bytes per generated token of the synthetic decode step at `batch` requests: the
    weights (shared by the batch), each request's K and V rows over CONTEXT + 1 positions,
    its new K and V rows, and its fp32 logits plus embedding row."""
    row = cfg.layers * cfg.kv_heads * cfg.head_dim * 2 * 2  # K and V, bf16, every layer
    return {"active_weight_bytes_per_token": cfg.weight_bytes() / batch,
            "kv_read_bytes_per_token": row * (CONTEXT + 1),
            "kv_write_bytes_per_token": row,
            "extra_bytes_per_token": cfg.vocab * 4 + cfg.hidden // 2 + cfg.hidden // 64 * 4}


def phase_rooflines(dec: dict, probe: dict) -> dict:
    """The reference's phase roofline diagnostic for each decode batch, fed with the
    measured prefill and decode times and the GEMV probe's large-matrix bandwidth."""
    from ironmule_amd.decode import DecoderConfig
    from ironmule_amd.measure import phase_roofline_diagnostic

    cfg = DecoderConfig()
    prefill_ns = dec.get("prefill", {}).get("ns")
    out = {}
    for key, entry in dec.items():
        if key == "prefill":
            continue
        b = int(key)
        out[f"batch_{b}"] = phase_roofline_diagnostic(
            prefill_ns=prefill_ns,
            decode_ns=entry["seconds_per_step"] * entry["timed_steps"] * 1e9,
            decode_steps=entry["timed_steps"] * b,
            effective_bandwidth_gbps=probe.get("gemv_gbps_large"),
            bandwidth_source="measure.gemv_gbps(262144, 1 GiB): streaming engine, "
                             f"{probe.get('gemv_chain', {}).get('large')} distinct K=2560 "
                             "weights per launch, cache flushed",
            bandwidth_source_kind="measured_effective", **decode_traffic(cfg, b))
    return out


def host_cpu() -> dict:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo) and counts."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((line.split(":", 1)[1].strip() for line in f
                          if line.lower().startswith("model name")), None)
    except OSError:
        pass
    if model is None:
        import subprocess
        try:
            text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            model = next((line.split(":", 1)[1].strip() for line in text.splitlines()
                          if line.lower().startswith("model name")), None)
        except (OSError, subprocess.SubprocessError):
            pass
    return {"model": model, "logical_cpus": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0))}


def cpu_dequantized_gemv(seconds: float):
    """The reference's `dequantize` plan on the host (ironmule/numeric_plans.py:449-497):
    every weight expanded once to dense fp32 (untimed, as at model load), then each
    decode projection is an fp32 GEMV (numpy over OpenBLAS).  Rate in the metric's unit:
    the same 4-bit bytes per layer as the qmv rows, over the time the fp32 GEMVs take."""
    import numpy as np
    import threadpoolctl

    from oracle import oracle as orc

    copies = []
    for c in range(4):
        layer = []
        for i, (_, n, k) in enumerate(LAYER):
            pr = orc.synthetic(n, k, 1, seed=SEED + 7 + c * 10 + i)
            layer.append((orc.dequant_f32(pr.w, pr.s, pr.b),
                          orc.bf16_to_f32(pr.x).reshape(-1).astype(np.float32)))
        copies.append(layer)
    step_bytes = sum(qmv_bytes(n, k, 1) for (_, n, k) in LAYER)
    dense_bytes = sum(n * k * 4 for (_, n, k) in LAYER)
    info = threadpoolctl.threadpool_info()
    threads = max((p.get("num_threads", 1) for p in info if p.get("user_api") == "blas"),
                  default=1)
    for w, x in copies[0]:
        w @ x
    done, t0 = 0, time.perf_counter()
    while True:
        for w, x in copies[done % 4]:
            w @ x
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done * step_bytes / el / 1e9, 3), "unit": "GB/s",
            "fp32_weight_gbs": round(done * dense_bytes / el / 1e9, 3), "cores": threads,
            "sample": (f"{done} passes over one layer's 7 projections at batch 1, weights "
                       f"pre-expanded to fp32 ({dense_bytes / 1e6:.0f} MB per layer, 4 "
                       f"rotating copies), {el:.1f} s, numpy fp32 GEMV on OpenBLAS "
                       f"({threads} threads); value counts the 4-bit bytes of the same work")}


def cpu_baseline(seconds: float = 10.0):
    """The oracle's restatement of the reference CUDA row kernel (ironmule/cuda_native.py:
    57-128) on the host cores, over the same layer shapes, rotating 4 layer copies."""
    import numpy as np

    from oracle import oracle as orc

    threads = orc.max_threads()
    copies = [[orc.synthetic(n, k, 1, seed=SEED + 7 + c * 10 + i) for i, (_, n, k) in enumerate(LAYER)]
              for c in range(4)]
    step_bytes = sum(qmv_bytes(n, k, 1) for (_, n, k) in LAYER)

    def run(nthreads, budget):
        for pr in copies[0]:  # warm
            orc.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x, threads=nthreads)
        done, t0 = 0, time.perf_counter()
        while True:
            for pr in copies[done % 4]:
                orc.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x, threads=nthreads)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return done * step_bytes / el / 1e9, done, el

    gbs, layers_done, el = run(threads, seconds)
    gbs1, layers1, el1 = run(1, seconds / 2)
    del np
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"{layers_done} passes over one layer's 7 projections at batch 1 "
                   f"({step_bytes / 1e6:.1f} MB each, 4 rotating copies), {el:.1f} s, "
                   f"oracle restatement of the reference row kernel, {threads} OpenMP threads"),
        "single_thread_gbs": round(gbs1, 3),
        "single_thread_sample": f"{layers1} passes, {el1:.1f} s, 1 thread",
        "host_cpu": host_cpu(),
        "dequantize_fp32_gemv": cpu_dequantized_gemv(seconds / 2),
    }


COPY_READ = 1 << 30   # the calibration copy: 2^27 int64 values read ...
COPY_WRITTEN = 1 << 29  # ... and written back as int32
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "stream_kernel_layer_m1_hbm_traffic.md")
# the only kernel of the timed layer steps: the streaming engine's independent-stage kernel
DOMINANT = "stream_kernel"


def copy_calibration(torch, device) -> None:
    """One plain elementwise copy of known size (int64 -> int32, COPY_READ bytes in,
    COPY_WRITTEN out): the yardstick that scales a profiling pass's FETCH_SIZE /
    WRITE_SIZE counters to bytes."""
    src = torch.ones(COPY_READ // 8, dtype=torch.int64, device=device)
    dst = src.to(torch.int32)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def _short(name: str) -> str:
    for marker in ("qmv_pair_rows_kernel", "qmv_rowband_kernel", "stream_chain_kernel", "stream_kernel", "qmv_stage_kernel", "attention_stage_kernel",
                   "step_kernel", "reset_kernel", "qmv_gather_kernel", "qmv_m1c_kernel", "qmv_m1_kernel", "qmv_rows_kernel",
                   "qmv_mma_staged_kernel", "qmv_mma_kernel", "qmv_dma_kernel", "qmv_band_kernel", "xprep_kernel",
                   "qmv_xs_kernel", "qmv_mr_kernel", "clear_words_kernel",
                   "dequant_kernel", "embed_kernel", "add_rmsnorm_kernel", "qk_norm_rope_kernel",
                   "attention_partial_kernel", "attention_combine_kernel", "silu_mul_kernel",
                   "residual_planes_kernel"):
        if marker in name:
            return name[name.index(marker):].split("(")[0]
    if "direct_copy_kernel" in name:
        return "torch copy kernel"
    return name.split("(")[0][:60]


def profile_summary(directories: list[str]) -> str:
    """Reduces rocprofv3 CSV output (kernel trace and --pmc passes) under `directories` to
    short text tables per (kernel, workgroups): dispatch count and mean duration from the
    trace; mean counters per dispatch from each pass.  FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch) are scaled to bytes by the calibration copy found in the same pass (the
    largest torch copy kernel, COPY_READ bytes read and COPY_WRITTEN written)."""
    import csv
    import glob
    from collections import defaultdict

    lines, traffic = [], defaultdict(dict)
    paths = lambda pattern: sorted(p for d in directories
                                   for p in glob.glob(os.path.join(d, "**", pattern), recursive=True))
    for path in paths("*kernel_trace.csv"):
        agg = defaultdict(list)
        for r in csv.DictReader(open(path)):
            key = (_short(r["Kernel_Name"]), int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]),
                   r.get("VGPR_Count", "?"), r.get("LDS_Block_Size", "?"))
            agg[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        lines += [f"kernel trace ({os.path.basename(path)}), this library's kernels:", "",
                  "| kernel | workgroups | vgpr | lds bytes | dispatches | mean us | median us |",
                  "|---|---|---|---|---|---|---|"]
        for key, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            if "at::native" in key[0] or "rocclr" in key[0]:
                continue
            v.sort()
            lines.append(f"| {key[0]} | {key[1]} | {key[2]} | {key[3]} | {len(v)} | "
                         f"{sum(v) / len(v) / 1e3:.3f} | {v[len(v) // 2] / 1e3:.3f} |")
        lines.append("")
    for path in paths("*counter_collection.csv"):
        agg = defaultdict(lambda: defaultdict(list))
        for r in csv.DictReader(open(path)):
            grid = int(r.get("Grid_Size", r.get("Grid_Size_X", 0)))
            wg = int(r.get("Workgroup_Size", r.get("Workgroup_Size_X", 1)) or 1)
            agg[(_short(r["Kernel_Name"]), grid // wg)][r["Counter_Name"]].append(float(r["Counter_Value"]))
        copies = [k for k in agg if k[0] == "torch copy kernel"]
        copy = agg[max(copies, key=lambda k: k[1])] if copies else None
        lines += [f"counters ({os.path.basename(path)}), mean per dispatch:", ""]
        for key, cs in sorted(agg.items()):
            if "at::native" in key[0] or "rocclr" in key[0] or key[0] == "torch copy kernel":
                continue
            vals = ", ".join(f"{c}={sum(v) / len(v):.1f}" for c, v in sorted(cs.items()))
            lines.append(f"* {key[0]}, {key[1]} workgroups, {len(next(iter(cs.values())))} "
                         f"dispatches: {vals}")
        if copy is not None:
            for c, known in (("FETCH_SIZE", COPY_READ), ("WRITE_SIZE", COPY_WRITTEN)):
                if c not in copy:
                    continue
                kib = sum(copy[c]) / len(copy[c])
                factor = known / 1024 / kib
                lines.append(f"* calibration: the copy moves {known} B; {c} reads {kib:.1f} KiB "
                             f"-> factor {factor:.4f}")
                for key, cs in agg.items():
                    if "at::native" not in key[0] and key[0] != "torch copy kernel" and c in cs:
                        traffic[key][c] = sum(cs[c]) / len(cs[c]) * 1024 * factor
        lines.append("")
    if traffic:
        lines += ["HBM traffic per dispatch (calibrated bytes):", "",
                  "| kernel | workgroups | fetch bytes | write bytes | traffic bytes |",
                  "|---|---|---|---|---|"]
        for key, t in sorted(traffic.items()):
            if "FETCH_SIZE" in t and "WRITE_SIZE" in t:
                lines.append(f"| {key[0]} | {key[1]} | {t['FETCH_SIZE']:.0f} | "
                             f"{t['WRITE_SIZE']:.0f} | {t['FETCH_SIZE'] + t['WRITE_SIZE']:.0f} |")
    return "\n".join(lines)


def profiled_traffic(kernel: str, workgroups: int):
    """Calibrated HBM bytes per dispatch of (kernel, workgroups) from the committed
    counter summary, or None when it holds no such row."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    for row in text.splitlines():
        cells = [c.strip() for c in row.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == kernel and cells[1] == str(workgroups):
            return int(cells[4])
    return None


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3600)
    ap.add_argument("--warmup", type=int, default=3600)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary configs")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-decode", action="store_true", help="skip the full decode step")
    ap.add_argument("--no-probe", action="store_true",
                    help="skip the GEMV bandwidth probe (and with it the phase roofline)")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the full decode step and exit (a short program for profilers)")
    ap.add_argument("--decode-batches", default="1,32", metavar="B[,B...]",
                    help="with --decode-only: the batch sizes to time (and no prefill unless 1 is one)")
    ap.add_argument("--no-breakdown", action="store_true",
                    help="time only the headline layer steps (a short program for profilers)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 1 GiB device copies (the yardstick for --pmc byte counters)")
    ap.add_argument("--profile-summary", nargs="+", default=None, metavar="DIR",
                    help="print a text summary of rocprofv3 CSV output under DIR... and exit")
    ap.add_argument("--chain-trace", action="store_true",
                    help="time the stages of the chained streaming launch from its per-stage "
                         "stamps (imq_stream_trace) and exit")
    ap.add_argument("--only", default=None, metavar="N,K,M[,f32]",
                    help="time one qmv shape over rotating weights (>= 1 GiB) and exit; "
                         "a short program for profilers")
    args = ap.parse_args()
    if args.profile_summary:
        print(profile_summary(args.profile_summary))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU runs "
                          "are not part of this build", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from ironmule_amd import _native

    device = "cuda:0"
    torch.cuda.set_device(0)
    code, arch, cus = _native.device_check()
    if code != 0:
        raise SystemExit(f"unsupported device {arch!r}")
    if args.copy_calibration:
        copy_calibration(torch, device)
    if args.chain_trace:
        print(json.dumps(chain_trace(torch, _native, device)), flush=True)
        return
    if args.decode_only:
        batches = tuple(int(b) for b in args.decode_batches.split(","))
        print(json.dumps({"metric": "decode tokens/s (profiling run)",
                          **bench_decode(torch, batches=batches, device=device,
                                         prefill_tokens=1 in batches)}), flush=True)
        return
    if args.only:
        parts = args.only.split(",")
        n, k, m = (int(v) for v in parts[:3])
        y_dtype = torch.float32 if len(parts) > 3 and parts[3] == "f32" else torch.bfloat16
        copies = max(2, -(-(1 << 30) // weight_bytes(n, k)))
        res = bench_config(torch, _native, n, k, [m], y_dtype, copies, device, SEED + 9)
        print(json.dumps({"metric": "qmv GB/s (profiling run)", "shape": [n, k, m],
                          "copies": copies, **res[str(m)]}), flush=True)
        return
    print(f"[bench] device {arch} with {cus} CUs; layer workload, {args.steps} steps",
          file=sys.stderr, flush=True)
    res = bench_layer(torch, _native, args.steps, args.warmup, device,
                      breakdown=not args.no_breakdown)
    if args.no_breakdown:
        value = res["step_bytes"] * args.steps / res["gpu_s"] / 1e9
        print(json.dumps({"metric": "layer GB/s (profiling run)", "value": round(value, 2),
                          "unit": "GB/s", "steps": args.steps, "workgroups": res["workgroups"],
                          "avg_launch_us": round(res["avg_launch_s"] * 1e6, 3)}), flush=True)
        return
    ms_per_step = res["gpu_s"] / args.steps * 1e3
    value = res["step_bytes"] * args.steps / res["gpu_s"] / 1e9
    launch_us = res["avg_launch_s"] * 1e6
    achieved = res["launch_bytes"] / res["avg_launch_s"] / 1e9
    line = {
        "metric": "4-bit qmv HBM GB/s (% of peak) + synthetic decode tokens/s at batch 1 and 32",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic: seeded random 4-bit weights, bf16 scales/biases, bf16 x ~ N(0,1)",
        "config": {"workload": "qwen3-4b decoder layer, 7 projections as 4-bit qmv, batch 1",
                   "projections": {name: [k, n] for (name, n, k) in LAYER},
                   "group_size": 64, "batch": 1, "rotating_layers": LAYERS,
                   "launch": "streaming engine: one persistent launch per 36 layers, each "
                             "layer's projections as 4 independent stages in decode order "
                             "(q/k/v, o, gate/up, down), launched directly on one stream; "
                             "steps % 36 layers as one more launch of that many layers",
                   "warm_up": res["warm_up"]},
        "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic(DOMINANT, res["workgroups"]),
                     "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                     "kernel": f"{DOMINANT} x {res['workgroups']} workgroups: 36 layers' "
                               "7 projections (144 stages), M=1",
                     "bytes_per_launch": res["launch_bytes"],
                     "avg_launch_us": round(launch_us, 3)},
        "layer_breakdown": {
            "per_kernel_launches": {k: {"us": round(v["us"], 3), "gbs": round(v["gbs"], 1)}
                                    for k, v in res["per_launch"].items()},
            "per_kernel_decode_order": {"us": round(res["decode_order"]["us"], 3),
                                        "gbs": round(res["decode_order"]["gbs"], 1),
                                        "note": "4 per-kernel launches per layer"},
            "one_grouped_launch": {"us": round(res["one_launch"]["us"], 3),
                                   "gbs": round(res["one_launch"]["gbs"], 1),
                                   "note": "all 7 projections of a layer in one launch"},
            "stream_chained": {"us": round(res["chained"]["us"], 3),
                               "gbs": round(res["chained"]["gbs"], 1),
                               "stalled": res["chained"]["stalled"],
                               "note": "streaming engine, each stage waits for and reads the "
                                       "previous one's output (decode-order dependencies)"},
        },
    }
    if not args.no_decode:
        print("[bench] decode step", file=sys.stderr, flush=True)
        dec = bench_decode(torch, device=device)
        line["decode_tokens_per_s"] = {"batch_1": dec["1"]["tokens_per_s"],
                                       "batch_32": dec["32"]["tokens_per_s"]}
        line["decode"] = {"workload": "synthetic qwen3-4b decode step: 36 layers + tied "
                                      "151936-token head, 4-bit group-64 weights, GQA 32/8 "
                                      f"heads, {CONTEXT}-token KV context per request, one "
                                      "hip graph per step", **dec}
    if not args.no_probe:
        from ironmule_amd import measure
        print("[bench] gemv bandwidth probe", file=sys.stderr, flush=True)
        probe = measure.measure(repeats=5)
        line["hardware"] = {k: probe[k] for k in (
            "device_name", "peak_bandwidth_gbps", "dispatch_us", "gemv_gbps_small",
            "gemv_gbps_large", "gemv_size_sensitivity", "gemv_frac_of_peak", "gemv_chain",
            "cache_flushed", "repeats")}
        line["hardware"]["gemv_gbps_small_warm"] = measure.gemv_gbps(
            *measure.GEMV_SMALL, 5, flush=False)
        if "decode" in line:
            line["decode"]["phase_roofline"] = phase_rooflines(dec, probe)
    if not args.no_extra:
        print("[bench] secondary configs", file=sys.stderr, flush=True)
        line["configs"] = {
            "c1_2560x2560": bench_config(torch, _native, 2560, 2560, [1], torch.bfloat16, 300,
                                         device, SEED),
            "c3_k3840_n15360": bench_config(torch, _native, 15360, 3840, [1, 2, 4, 8, 16, 32],
                                            torch.bfloat16, 36, device, SEED + 2),
            "c4_lm_head_fp32": bench_config(torch, _native, 151936, 2560, [1, 32],
                                            torch.float32, 5, device, SEED + 3, repeats=4),
        }
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
