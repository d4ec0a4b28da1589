"""What the decode path can expect of this machine, and how close a run came to it.

Call surface of the reference's measurement pieces, on MI355X:

* `BANDWIDTH_GB_S` and `bandwidth_gb_s(name)`: published peak memory bandwidth by device
  name (ironmule_product/hardware_profile.py:20-52).  The table here lists AMD Instinct
  parts; gfx950 (MI350X and MI355X) is 8,000 GB/s.
* `gemv_bytes(out_features, target_bytes)` and `gemv_gbps(out_features, target_bytes,
  repeats)`: the 4-bit GEMV bandwidth probe (ironmule/hw.py:401-404, 441-473).  K=2560,
  group 64; `target_bytes // bytes-per-weight` distinct weights, at least 2 and at most 48,
  one activation row; the rate is (weights x bytes-per-weight) / median time.  The weights
  are run by the streaming engine (imq_stream_*) as independent stages of one launch,
  where the reference chains its library GEMV calls inside one evaluation.
* `measure(repeats)`: the reference's probe set (ironmule/hw.py:477-511): the per-launch
  cost of a chain of 512 dependent one-element additions, the probe at N=1024 (512 MiB
  target, a per-layer matrix) and at N=262144 (1 GiB target, an output head).
* `phase_roofline_diagnostic(...)`: the per-run prefill/decode roofline calculation
  (ironmule/benchmark.py:272-479).  It only computes over what it is given, and says
  "inconclusive" rather than assume a missing term is zero.

Differences that follow from the hardware: MI355X has a 256 MB memory-side cache, larger
than the 48 weights of the N=1024 probe (70.8 MB), so `gemv_gbps` by default reads a
1 GiB buffer before each timed launch (a read, so that no dirty lines are written back
during the timed launch); each sample then reads its weights from HBM, as decode does
with a model several times the cache.  `flush=False` gives the warm figure.
Each sample is one launch timed with HIP events on the launching stream.
"""

from __future__ import annotations

import math
import re
import statistics
import time
from typing import Any

import torch

from . import _native

#: Published peak memory bandwidth (GB/s), matched in order against the device name.
BANDWIDTH_GB_S: tuple[tuple[str, float], ...] = (
    (r"MI355X", 8000.0),
    (r"MI350X", 8000.0),
    (r"\bgfx950\b", 8000.0),
    (r"MI325X", 6000.0),
    (r"MI300X", 5300.0),
    (r"MI300A", 5300.0),
    (r"MI250X?\b", 3276.8),
    (r"MI210", 1638.4),
    (r"MI100", 1228.8),
)

GEMV_IN_FEATURES = 2560
GEMV_GROUP = 64
GEMV_BITS = 4
GEMV_MIN_CHAIN, GEMV_MAX_CHAIN = 2, 48
#: (out_features, target bytes) of the two probes `measure` runs.
GEMV_SMALL = (1024, 512 * 2**20)
GEMV_LARGE = (262144, 1024 * 2**20)
DISPATCH_CHAIN = 512
FLUSH_BYTES = 1 << 30
PROBE_SEED = 20260321
PROBE_VERSION = 1
MAX_REPEATS = 32

ROOFLINE_SCHEMA = "ironmule.phase_roofline.v1"
BANDWIDTH_KINDS = ("measured_effective", "nominal_peak")


def bandwidth_gb_s(name: str | None) -> float | None:
    """The published peak bandwidth of the device `name` describes, or None."""
    if not name:
        return None
    return next((gbs for pattern, gbs in BANDWIDTH_GB_S if re.search(pattern, name)), None)


def device_name(index: int = 0) -> str | None:
    """The device's marketing name and architecture ("AMD Instinct MI355X (gfx950)")."""
    if not torch.cuda.is_available():
        return None
    props = torch.cuda.get_device_properties(index)
    arch = getattr(props, "gcnArchName", "") or ""
    return f"{props.name} ({arch.split(':')[0]})" if arch else props.name


# ------------------------------------------------------------------ the GEMV probe

def _weight_bytes(out_features: int) -> int:
    k = GEMV_IN_FEATURES
    return out_features * k * GEMV_BITS // 8 + out_features * (k // GEMV_GROUP) * 4


def _chain(out_features: int, target_bytes: int) -> int:
    return min(GEMV_MAX_CHAIN, max(GEMV_MIN_CHAIN, target_bytes // _weight_bytes(out_features)))


def gemv_bytes(out_features: int, target_bytes: int) -> int:
    """Weight bytes the probe streams per timed launch: distinct weights x bytes each
    (packed 4-bit codes plus a bf16 scale and bias per group of 64)."""
    return _chain(out_features, target_bytes) * _weight_bytes(out_features)


def _check_repeats(repeats: int) -> int:
    if type(repeats) is not int or not 1 <= repeats <= MAX_REPEATS:
        raise ValueError(f"repeats must be an integer in [1, {MAX_REPEATS}]")
    return repeats


def gemv_gbps(out_features: int, target_bytes: int, repeats: int = 5, *,
              raw_samples: list[float] | None = None, flush: bool = True,
              device: str = "cuda:0") -> float:
    """Achieved GB/s of one streaming-engine launch over `gemv_bytes(...)` of distinct
    4-bit weights (K=2560, one bf16 row): bytes / median of `repeats` event-timed
    launches after two untimed ones.  Seconds per sample are appended to `raw_samples`."""
    _check_repeats(repeats)
    k, chain = GEMV_IN_FEATURES, _chain(out_features, target_bytes)
    gen = torch.Generator(device=device)
    gen.manual_seed(PROBE_SEED + out_features)
    weights = []
    for _ in range(chain):
        w = torch.randint(0, 2**32, (out_features, k // 8), dtype=torch.int64, device=device,
                          generator=gen).to(torch.int32)
        s = torch.empty((out_features, k // GEMV_GROUP), device=device).uniform_(
            0.005, 0.02, generator=gen).to(torch.bfloat16)
        b = torch.empty((out_features, k // GEMV_GROUP), device=device).uniform_(
            -0.1, 0.1, generator=gen).to(torch.bfloat16)
        weights.append((w, s, b))
    x = torch.randn(k, device=device, generator=gen).to(torch.bfloat16)
    outs = [torch.empty(out_features, dtype=torch.bfloat16, device=device) for _ in weights]
    program = _native.stream_program([([q], x, [y], False) for q, y in zip(weights, outs)])
    flusher = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=device) if flush else None
    stream = torch.cuda.Stream(device=device)
    samples = []
    try:
        with torch.cuda.stream(stream):
            for _ in range(2):
                program.launch(stream)
            for _ in range(repeats):
                if flusher is not None:  # a read: no dirty lines left to write back
                    flusher.sum()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record(stream)
                program.launch(stream)
                end.record(stream)
                end.synchronize()
                samples.append(start.elapsed_time(end) / 1e3)
        if program.failed():
            raise RuntimeError("the streaming engine reported a stalled wait during the probe")
    finally:
        program.close()
    if any(not math.isfinite(v) or v <= 0 for v in samples):
        raise ValueError(f"non-positive probe timings {samples}")
    if raw_samples is not None:
        raw_samples.extend(samples)
    return chain * _weight_bytes(out_features) / statistics.median(samples) / 1e9


def _dispatch_seconds(repeats: int, device: str) -> list[float]:
    """Wall time of DISPATCH_CHAIN dependent one-element additions, host submission and
    the final synchronisation included, per repeat."""
    value = torch.zeros(1, device=device)
    samples = []
    for trial in range(repeats + 1):
        torch.cuda.synchronize(device)
        started = time.perf_counter()
        v = value
        for _ in range(DISPATCH_CHAIN):
            v = v + 1.0
        torch.cuda.synchronize(device)
        if trial:  # the first pass warms the allocator and the kernel cache
            samples.append(time.perf_counter() - started)
    return samples


def _summary(values: list[float]) -> dict[str, float]:
    return {"median": statistics.median(values), "min": min(values), "max": max(values),
            "n": len(values)}


def measure(repeats: int = 5, *, device: str = "cuda:0", flush: bool = True) -> dict[str, Any]:
    """The probe set: dispatch cost, GEMV bandwidth at a layer size and at a head size,
    with the device's published peak beside them."""
    _check_repeats(repeats)
    samples = {"scalar_chain_s": _dispatch_seconds(repeats, device),
               "gemv_small_s": [], "gemv_large_s": []}
    gemv_gbps(*GEMV_SMALL, repeats, raw_samples=samples["gemv_small_s"], flush=flush,
              device=device)
    gemv_gbps(*GEMV_LARGE, repeats, raw_samples=samples["gemv_large_s"], flush=flush,
              device=device)
    summary = {name: _summary(values) for name, values in samples.items()}
    small = gemv_bytes(*GEMV_SMALL) / summary["gemv_small_s"]["median"] / 1e9
    large = gemv_bytes(*GEMV_LARGE) / summary["gemv_large_s"]["median"] / 1e9
    name = device_name(torch.device(device).index or 0)
    peak = bandwidth_gb_s(name)
    return {
        "probe_version": PROBE_VERSION,
        "device_name": name,
        "peak_bandwidth_gbps": peak,
        "dispatch_us": summary["scalar_chain_s"]["median"] / DISPATCH_CHAIN * 1e6,
        "gemv_gbps_small": small, "gemv_gbps_large": large,
        "gemv_size_sensitivity": large / small,
        "gemv_frac_of_peak": {"small": small / peak, "large": large / peak} if peak else None,
        "gemv_chain": {"small": _chain(*GEMV_SMALL), "large": _chain(*GEMV_LARGE)},
        "cache_flushed": flush,
        "raw_timing_samples": samples, "timing_summary": summary, "repeats": repeats,
    }


# ------------------------------------------------------------------ phase roofline

class _Findings:
    """What a diagnostic found missing or invalid, in the order it found it."""

    def __init__(self) -> None:
        self.missing: list[str] = []
        self.invalid: list[str] = []

    def number(self, name: str, value: Any) -> float | None:
        """A finite non-negative number, or None after recording why not."""
        if value is None:
            self.missing.append(name)
            return None
        if isinstance(value, bool) or not isinstance(value, (int, float)):
            self.invalid.append(f"{name}: expected a finite number")
            return None
        try:
            as_float = float(value)
        except (OverflowError, ValueError):
            self.invalid.append(f"{name}: expected a finite number")
            return None
        if not math.isfinite(as_float):
            self.invalid.append(f"{name}: expected a finite number")
            return None
        if as_float < 0:
            self.invalid.append(f"{name}: must be non-negative")
            return None
        return as_float

    def duration(self, name: str, value: Any) -> tuple[float | None, str]:
        """(value, "measured") for a positive duration; otherwise "unavailable" when it
        is absent and "invalid" when it is wrong."""
        seen = len(self.invalid)
        as_float = self.number(name, value)
        if as_float is None:
            return None, "invalid" if len(self.invalid) > seen else "unavailable"
        if as_float == 0:
            self.invalid.append(f"{name}: must be positive when measured")
            return as_float, "invalid"
        return as_float, "measured"

    def ratio(self, name: str, top: float, bottom: float) -> float | None:
        """top / bottom when it is finite and positive, else None after recording it."""
        if not (math.isfinite(top) and math.isfinite(bottom)) or bottom == 0:
            self.invalid.append(f"{name}: non-finite or zero denominator")
            return None
        try:
            value = top / bottom
        except (OverflowError, ZeroDivisionError):
            self.invalid.append(f"{name}: non-finite or zero denominator")
            return None
        if not math.isfinite(value):
            self.invalid.append(f"{name}: result is not finite")
            return None
        if value <= 0:
            self.invalid.append(f"{name}: result is not positive")
            return None
        return value

    def unique_missing(self) -> list[str]:
        return list(dict.fromkeys(self.missing))


def _steps(found: _Findings, decode_steps: Any) -> int | None:
    if decode_steps is None:
        found.missing.append("decode_steps")
        return None
    problem = None
    if isinstance(decode_steps, bool) or not isinstance(decode_steps, int):
        problem = "expected an integer"
    elif decode_steps < 0:
        problem = "must be non-negative"
    elif decode_steps > 2**63 - 1:
        problem = "exceeds 2**63-1"
    if problem:
        found.invalid.append(f"decode_steps: {problem}")
        return None
    return decode_steps


def _decode_phase(found: _Findings, steps: int | None, decode_ns: Any):
    """(duration, status) of the decode phase given its step count."""
    if steps == 0:  # prefill produced the only token: no decode phase to time
        if decode_ns is None:
            return None, "not_applicable"
        if not isinstance(decode_ns, bool) and isinstance(decode_ns, (int, float)) and decode_ns == 0:
            return 0.0, "not_applicable"
        if isinstance(decode_ns, bool):
            found.invalid.append("decode_ns: expected zero, not a boolean")
            return None, "invalid"
        value, _ = found.duration("decode_ns", decode_ns)
        found.invalid.append("decode_ns: must be zero for a zero-step decode")
        return value, "invalid"
    if steps is None:  # a duration without a step count yields no rate
        seen = len(found.invalid)
        value = found.number("decode_ns", decode_ns)
        return value, "invalid" if len(found.invalid) > seen else "unavailable"
    return found.duration("decode_ns", decode_ns)


def _bandwidth_source(found: _Findings, label: Any, kind: Any) -> None:
    if label is None:
        found.missing.append("bandwidth_source")
    elif not isinstance(label, str) or not label.strip():
        found.invalid.append("bandwidth_source: expected a non-empty string")
    if kind is None:
        found.missing.append("bandwidth_source_kind")
    elif not isinstance(kind, str):
        found.invalid.append("bandwidth_source_kind: expected a string")
    elif kind not in BANDWIDTH_KINDS:
        found.invalid.append("bandwidth_source_kind: unknown value")


def _roofline(found: _Findings, decode_status: str, tokens_per_second: float | None, *,
              bandwidth: Any, traffic: dict[str, Any], label: Any, kind: Any) -> dict[str, Any]:
    if decode_status == "not_applicable":
        return {"status": "not_applicable"}
    gbps = found.number("effective_bandwidth_gbps", bandwidth)
    terms = {key: found.number(name, value) for key, (name, value) in traffic.items()}
    _bandwidth_source(found, label, kind)
    total = None
    if gbps is not None and all(v is not None for v in terms.values()):
        try:
            total = math.fsum(terms.values())
        except (OverflowError, ValueError):
            found.invalid.append("bytes_per_token: sum is not finite")
        if total is not None and not math.isfinite(total):
            found.invalid.append("bytes_per_token: sum is not finite")
        if total is not None and total <= 0:
            found.invalid.append("bytes_per_token: denominator must be positive")
        if gbps <= 0:
            found.invalid.append("effective_bandwidth_gbps: denominator must be positive")
    if found.invalid:
        return {"status": "invalid", "invalid": list(found.invalid)}
    if decode_status != "measured" or found.missing:
        return {"status": "inconclusive", "missing": found.unique_missing()}
    source = {"kind": kind, "label": label.strip()}
    bytes_per_token = dict(terms, total=total)
    if kind == "nominal_peak":  # a datasheet figure is provenance, not a yardstick
        return {"status": "inconclusive", "reason": "nominal_peak_not_valid_for_efficiency",
                "bandwidth_gbps": gbps, "bandwidth_source": source,
                "bytes_per_token": bytes_per_token}
    top = gbps * 1e9
    if not math.isfinite(top):
        found.invalid.append("ideal_tokens_per_second: numerator is not finite")
        return {"status": "invalid", "invalid": list(found.invalid)}
    ideal = found.ratio("ideal_tokens_per_second", top, total)
    efficiency = (found.ratio("efficiency", tokens_per_second, ideal)
                  if ideal is not None and tokens_per_second is not None else None)
    if found.invalid or efficiency is None:
        return {"status": "invalid", "invalid": list(found.invalid)}
    result = {"status": "ok", "bandwidth_gbps": gbps, "bandwidth_source": source,
              "bytes_per_token": bytes_per_token, "ideal_tokens_per_second": ideal,
              "efficiency": efficiency}
    if efficiency > 1:
        result["warnings"] = ["efficiency_above_one_input_consistency"]
    return result


def phase_roofline_diagnostic(
    *,
    prefill_ns: int | float | None,
    decode_ns: int | float | None,
    decode_steps: int | None,
    effective_bandwidth_gbps: int | float | None,
    active_weight_bytes_per_token: int | float | None,
    kv_read_bytes_per_token: int | float | None,
    kv_write_bytes_per_token: int | float | None,
    extra_bytes_per_token: int | float | None,
    bandwidth_source: str | None,
    bandwidth_source_kind: str | None,
) -> dict[str, Any]:
    """Prefill and decode phase timings of one run, and the decode phase's position
    against a bandwidth roofline: ideal tokens/s = bandwidth / bytes per token (weights,
    KV reads, KV writes and other traffic), efficiency = measured / ideal.

    `decode_steps` counts decode steps after the first token (which prefill produces).
    Status "ok" needs both phases measured and a `measured_effective` bandwidth; a
    `nominal_peak` bandwidth or any absent input gives "inconclusive", any malformed
    input "invalid"."""
    found = _Findings()
    prefill_value, prefill_status = found.duration("prefill_ns", prefill_ns)
    steps = _steps(found, decode_steps)
    decode_value, decode_status = _decode_phase(found, steps, decode_ns)
    prefill_ms = found.ratio("prefill_ms", prefill_value, 1e6) if prefill_value is not None else None
    rate = (found.ratio("decode_tokens_per_second", float(steps), decode_value / 1e9)
            if steps and decode_value is not None else None)
    phases = {
        "prefill": {"duration_ns": prefill_value, "duration_ms": prefill_ms,
                    "status": prefill_status},
        "decode": {"duration_ns": decode_value, "decode_steps": steps,
                   "tokens_per_second": rate, "status": decode_status},
    }
    roofline = _roofline(
        found, decode_status, rate, bandwidth=effective_bandwidth_gbps,
        traffic={"weights": ("active_weight_bytes_per_token", active_weight_bytes_per_token),
                 "kv_read": ("kv_read_bytes_per_token", kv_read_bytes_per_token),
                 "kv_write": ("kv_write_bytes_per_token", kv_write_bytes_per_token),
                 "extra": ("extra_bytes_per_token", extra_bytes_per_token)},
        label=bandwidth_source, kind=bandwidth_source_kind)
    if found.invalid:
        status = "invalid"
    elif (prefill_status, decode_status, roofline["status"]) == ("measured", "measured", "ok"):
        status = "ok"
    else:
        status = "inconclusive"
    return {"schema": ROOFLINE_SCHEMA, "diagnostic_only": True, "status": status,
            "missing": found.unique_missing(), "phases": phases, "roofline": roofline}
