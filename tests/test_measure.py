"""The measurement surface on the CPU: the bandwidth table, the GEMV probe's byte count,
and the phase roofline diagnostic's arithmetic and fail-closed statuses (the cases of
ironmule's tests/engine/test_benchmark.py:184-411, restated).  The probes themselves
need a GPU and run in bench.py."""

from __future__ import annotations

import json
import math

import pytest

from ironmule_amd import measure


# ------------------------------------------------------------------ bandwidth table

@pytest.mark.parametrize("name,gbs", [
    ("AMD Instinct MI355X (gfx950)", 8000.0),
    ("AMD Instinct MI355X", 8000.0),
    ("AMD Instinct MI350X", 8000.0),
    ("gfx950", 8000.0),
    ("AMD Instinct MI300X (gfx942)", 5300.0),
    ("AMD Instinct MI325X", 6000.0),
    ("AMD Instinct MI250X", 3276.8),
    ("Tesla T4", None),
    ("", None),
    (None, None),
])
def test_published_bandwidth_by_name(name, gbs):
    assert measure.bandwidth_gb_s(name) == gbs


# ------------------------------------------------------------------ probe bytes

def test_gemv_bytes_counts_codes_scales_and_biases_of_the_chained_weights():
    # N=1024, K=2560: 1,310,720 code bytes + 1024 * 40 groups * (2 + 2) bytes
    per_small = 1024 * 2560 // 2 + 1024 * 40 * 4
    assert per_small == 1_474_560
    assert measure.gemv_bytes(*measure.GEMV_SMALL) == 48 * per_small  # 364 fit, 48 kept
    per_large = 262144 * 1280 + 262144 * 160
    assert measure.gemv_bytes(*measure.GEMV_LARGE) == 2 * per_large  # 2 fit in 1 GiB
    assert measure.gemv_bytes(1024, 1) == 2 * per_small  # at least two weights
    assert measure.gemv_bytes(1024, 5 * per_small + 7) == 5 * per_small


@pytest.mark.parametrize("repeats", [0, 33, 2.0, True])
def test_probe_repeats_are_bounded_integers(repeats):
    with pytest.raises(ValueError):
        measure.gemv_gbps(1024, 1, repeats)


# ------------------------------------------------------------------ phase roofline

def _inputs(**changes):
    base = dict(prefill_ns=2_000_000, decode_ns=5_000_000, decode_steps=10,
                effective_bandwidth_gbps=300.0, active_weight_bytes_per_token=100_000_000,
                kv_read_bytes_per_token=1_000, kv_write_bytes_per_token=2_000,
                extra_bytes_per_token=3_000, bandwidth_source="probe",
                bandwidth_source_kind="measured_effective")
    base.update(changes)
    return base


def _diagnose(**changes):
    result = measure.phase_roofline_diagnostic(**_inputs(**changes))
    json.dumps(result, allow_nan=False)  # every outcome serialises without NaN or inf
    return result


def test_a_complete_run_gets_rates_bytes_and_efficiency():
    r = _diagnose()
    assert (r["schema"], r["diagnostic_only"], r["status"], r["missing"]) == (
        "ironmule.phase_roofline.v1", True, "ok", [])
    assert r["phases"]["prefill"] == {"duration_ns": 2e6, "duration_ms": 2.0,
                                      "status": "measured"}
    # 10 decode steps (the prefill's token excluded) in 5 ms
    assert r["phases"]["decode"]["tokens_per_second"] == pytest.approx(2000.0)
    roof = r["roofline"]
    assert roof["bytes_per_token"] == {"weights": 1e8, "kv_read": 1e3, "kv_write": 2e3,
                                       "extra": 3e3, "total": 100_006_000}
    ideal = 300e9 / 100_006_000
    assert roof["ideal_tokens_per_second"] == pytest.approx(ideal)
    assert roof["efficiency"] == pytest.approx(2000.0 / ideal)
    assert roof["bandwidth_source"] == {"kind": "measured_effective", "label": "probe"}
    assert "warnings" not in roof


@pytest.mark.parametrize("field", ["kv_read_bytes_per_token", "prefill_ns", "decode_steps",
                                   "bandwidth_source", "bandwidth_source_kind",
                                   "effective_bandwidth_gbps"])
def test_an_absent_input_is_inconclusive_not_zero(field):
    r = _diagnose(**{field: None})
    assert r["status"] == "inconclusive" and field in r["missing"]
    assert r["roofline"]["status"] == "inconclusive"
    assert "efficiency" not in r["roofline"] and "ideal_tokens_per_second" not in r["roofline"]
    if field == "kv_read_bytes_per_token":  # the phases keep their values
        assert r["phases"]["decode"]["tokens_per_second"] == pytest.approx(2000.0)


def test_a_datasheet_bandwidth_never_yields_an_efficiency():
    r = _diagnose(bandwidth_source_kind="nominal_peak")
    assert r["status"] == "inconclusive"
    assert r["roofline"]["reason"] == "nominal_peak_not_valid_for_efficiency"
    assert r["roofline"]["bytes_per_token"]["total"] == 100_006_000
    assert "efficiency" not in r["roofline"]


def test_zero_decode_steps_make_the_roofline_not_applicable():
    r = _diagnose(decode_steps=0, decode_ns=0)
    assert r["phases"]["decode"] == {"duration_ns": 0.0, "decode_steps": 0,
                                     "tokens_per_second": None, "status": "not_applicable"}
    assert r["roofline"] == {"status": "not_applicable"} and r["status"] == "inconclusive"
    assert _diagnose(decode_steps=0, decode_ns=None)["roofline"]["status"] == "not_applicable"
    assert _diagnose(decode_steps=0, decode_ns=5)["status"] == "invalid"
    boolean = _diagnose(decode_steps=0, decode_ns=False)
    assert boolean["status"] == "invalid"
    assert boolean["phases"]["decode"]["duration_ns"] is None


@pytest.mark.parametrize("field,value", [
    ("prefill_ns", True), ("prefill_ns", 0), ("prefill_ns", 10**400), ("prefill_ns", "2"),
    ("decode_ns", math.nan), ("decode_ns", 0), ("decode_steps", True), ("decode_steps", -1),
    ("decode_steps", 2**63), ("decode_steps", 1.0), ("effective_bandwidth_gbps", -1.0),
    ("effective_bandwidth_gbps", 0.0), ("active_weight_bytes_per_token", math.inf),
    ("kv_read_bytes_per_token", -1), ("bandwidth_source", " "),
    ("bandwidth_source_kind", "estimated"), ("bandwidth_source_kind", 42),
])
def test_malformed_inputs_fail_closed(field, value):
    r = _diagnose(**{field: value})
    assert r["status"] == "invalid" and r["roofline"]["status"] == "invalid"
    assert r["roofline"]["invalid"]
    assert "efficiency" not in r["roofline"]


def test_all_zero_traffic_is_an_invalid_denominator():
    r = _diagnose(active_weight_bytes_per_token=0, kv_read_bytes_per_token=0,
                  kv_write_bytes_per_token=0, extra_bytes_per_token=0)
    assert r["status"] == "invalid"
    assert any("denominator" in m for m in r["roofline"]["invalid"])


@pytest.mark.parametrize("changes,needle", [
    (dict(prefill_ns=5e-324), "prefill_ms"),
    (dict(decode_ns=5e-324, decode_steps=1), "decode_tokens_per_second"),
    (dict(active_weight_bytes_per_token=1e308, kv_read_bytes_per_token=1e308,
          kv_write_bytes_per_token=1e308, extra_bytes_per_token=1e308), "bytes_per_token"),
    (dict(effective_bandwidth_gbps=1e308, active_weight_bytes_per_token=1),
     "ideal_tokens_per_second"),
    (dict(effective_bandwidth_gbps=5e-324, active_weight_bytes_per_token=1e308,
          kv_read_bytes_per_token=0, kv_write_bytes_per_token=0, extra_bytes_per_token=0),
     "ideal_tokens_per_second"),
])
def test_overflow_and_underflow_in_derived_values_fail_closed(changes, needle):
    r = _diagnose(**changes)
    assert r["status"] == "invalid"
    messages = r["roofline"].get("invalid", [])
    assert any(needle in m for m in messages), messages


def test_an_efficiency_above_one_is_reported_with_a_warning_not_clamped():
    r = _diagnose(prefill_ns=1, decode_ns=1e9, decode_steps=1, effective_bandwidth_gbps=1e-10,
                  active_weight_bytes_per_token=1, kv_read_bytes_per_token=0,
                  kv_write_bytes_per_token=0, extra_bytes_per_token=0)
    assert r["status"] == "ok" and r["roofline"]["efficiency"] > 1
    assert r["roofline"]["warnings"] == ["efficiency_above_one_input_consistency"]


def test_a_planted_arithmetic_slip_would_be_caught():
    """The ok case's figures by hand, so that an efficiency computed against the weights
    alone (a dropped KV term) or from steps + 1 (the prefill token counted) fails."""
    r = _diagnose(decode_ns=1e9, decode_steps=4, effective_bandwidth_gbps=1.0,
                  active_weight_bytes_per_token=3e8, kv_read_bytes_per_token=2e8,
                  kv_write_bytes_per_token=0, extra_bytes_per_token=0)
    assert r["roofline"]["ideal_tokens_per_second"] == pytest.approx(2.0)  # 1e9 / 5e8
    assert r["roofline"]["efficiency"] == pytest.approx(2.0)  # 4 tok/s over 2 ideal
