"""The C ABI library without a GPU: it loads, exports every function its header
declares, and refuses malformed calls with the documented codes before touching a
device.  (No compute call is made here.)"""

from __future__ import annotations

import ctypes
import os

import pytest

from ironmule_amd import _native


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.LIB_PATH):
        from ironmule_amd import build
        build.build()
    return _native.lib()


def test_every_declared_function_is_exported(lib):
    declared = _native.declared_functions()
    assert set(declared) == set(_native._SIGNATURES), declared
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.imq_abi_version() == 1


def _qmv(lib, **over):
    args = dict(w=1 << 20, s=1 << 20, b=1 << 20, x=1 << 20, ldx=2560, y=1 << 20, ldy=2560,
                M=1, N=2560, K=2560, gs=64, bits=4, dtype=0)
    args.update(over)
    P = ctypes.c_void_p
    return lib.imq_qmv(P(args["w"]), P(args["s"]), P(args["b"]), P(args["x"]), args["ldx"],
                       P(args["y"]), args["ldy"], args["M"], args["N"], args["K"], args["gs"],
                       args["bits"], args["dtype"], None)


@pytest.mark.parametrize("over,code", [
    ({"bits": 8}, _native.IMQ_EUNSUPPORTED),
    ({"gs": 128}, _native.IMQ_EUNSUPPORTED),
    ({"K": 100}, _native.IMQ_EINVAL),
    ({"K": 0}, _native.IMQ_EINVAL),
    ({"N": 0}, _native.IMQ_EINVAL),
    ({"w": 0}, _native.IMQ_EINVAL),
    ({"w": (1 << 20) + 4}, _native.IMQ_EINVAL),
    ({"M": 0}, _native.IMQ_EINVAL),
    ({"M": 33}, _native.IMQ_EUNSUPPORTED),
    ({"x": 0}, _native.IMQ_EINVAL),
    ({"x": (1 << 20) + 2}, _native.IMQ_EINVAL),
    ({"dtype": 7}, _native.IMQ_EINVAL),
    ({"M": 2, "ldx": 2564}, _native.IMQ_EINVAL),
    ({"M": 2, "ldy": 100}, _native.IMQ_EINVAL),
])
def test_malformed_calls_are_refused_with_codes(lib, over, code):
    assert _qmv(lib, **over) == code
    got, msg = _native.last_error()
    assert got == code and msg


def test_dequant_refuses_bad_dtype(lib):
    P = ctypes.c_void_p
    assert lib.imq_dequant(P(1 << 20), P(1 << 20), P(1 << 20), P(1 << 20), 9, 64, 64, 64, 4,
                           None) == _native.IMQ_EINVAL


def test_multi_refuses_too_many_vectors(lib):
    P = ctypes.c_void_p
    arr = (P * 33)(*([1 << 20] * 33))
    assert lib.imq_qmv_multi(P(1 << 20), P(1 << 20), P(1 << 20), arr, arr, 33, 64, 64, 64, 4,
                             0, None) == _native.IMQ_EUNSUPPORTED


def _residual_planes(lib, **over):
    args = dict(planes=1 << 20, nplanes=4, M=32, N=2560, h=1 << 22, ldh=2560, weight=1 << 24,
                x=1 << 25, ldx=2560, ssq=1 << 26, ld=40)
    args.update(over)
    P = ctypes.c_void_p
    out = _native.ResidualOut(args["h"], args["ldh"], args["weight"], args["x"], args["ldx"],
                              args["ssq"], args["ld"])
    return lib.imq_residual_planes(P(args["planes"]), args["nplanes"], args["M"], args["N"],
                                   ctypes.byref(out), None)


@pytest.mark.parametrize("over", [
    {"planes": 0}, {"planes": (1 << 20) + 2}, {"nplanes": 0}, {"nplanes": 17}, {"M": 0}, {"M": 33},
    {"N": 0}, {"h": 0}, {"ldh": 100}, {"x": 0}, {"ldx": 100}, {"ld": 38}, {"ld": 42},
    {"nplanes": 16, "M": 32, "N": 1 << 20},
])
def test_residual_planes_refusals(lib, over):
    """imq_residual_planes refuses malformed calls before it looks for a device."""
    code = _residual_planes(lib, **over)
    assert code in (_native.IMQ_EINVAL, _native.IMQ_EUNSUPPORTED), (over, code)


def _residual_bands(lib, **over):
    args = dict(w=1 << 20, s=1 << 21, b=1 << 22, x=1 << 23, ldx=4096, N=2560, K=4096, M=32, gs=64, bits=4,
                h=1 << 24, ldh=2560, weight=1 << 25, xo=1 << 26, ldxo=2560, ssq=1 << 27, ld=80)
    args.update(over)
    prob = _native.Problem(args["w"], args["s"], args["b"], args["x"], args["ldx"], None, 0, args["N"], args["K"])
    out = _native.ResidualOut(args["h"], args["ldh"], args["weight"], args["xo"], args["ldxo"],
                              args["ssq"], args["ld"])
    return lib.imq_qmv_residual_bands(ctypes.byref(prob), args["M"], args["gs"], args["bits"],
                                      ctypes.byref(out), None)


@pytest.mark.parametrize("over", [
    {"M": 0}, {"M": 33}, {"x": 0}, {"x": (1 << 23) + 8}, {"ldx": 4000}, {"ldx": 4100}, {"K": 4160},
    {"K": 9984, "ldx": 9984}, {"gs": 32}, {"bits": 8}, {"h": 0}, {"ldh": 100}, {"xo": 0}, {"ldxo": 100},
    {"ldxo": _native.LD_TILED, "N": 2528}, {"ld": 40}, {"ld": 82}, {"w": 0},
])
def test_residual_bands_refusals(lib, over):
    """imq_qmv_residual_bands refuses malformed calls before it looks for a device: rows out
    of 1..32, x misaligned or ldx short or not a multiple of 8, K past 9728 or not a
    multiple of 256, another format, h or x' missing or short, a tiled x' of N not a
    multiple of 64, ssq ld short of the 80 bands or not a multiple of 4."""
    code = _residual_bands(lib, **over)
    assert code in (_native.IMQ_EINVAL, _native.IMQ_EUNSUPPORTED), (over, code)


def test_python_side_validates_before_the_abi():
    import torch
    w = torch.zeros((8, 8), dtype=torch.int32)
    s = torch.zeros((8, 1), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        _native.check_weights(w, s, s)
    with pytest.raises(ValueError, match="bfloat16"):
        _native.check_weights(w, s.float(), s)
    with pytest.raises(ValueError, match="multiple of 64"):
        _native.check_weights(torch.zeros((8, 3), dtype=torch.int32), s, s)


def _c_layout(structs: dict[str, list[str]]) -> dict[str, int]:
    """sizeof and offsetof of the header's structures, as a C compiler lays them out."""
    import subprocess
    import tempfile

    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "ironmule_step.h"',
             "int main(void) {"]
    for name, fields in structs.items():
        lines.append(f'  printf("{name} %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'  printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    lines += ["  return 0;", "}"]
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-I", os.path.join(_native.ROOT, "include"), src, "-o", exe],
                       check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (ln.split() for ln in out.splitlines())}


def test_ctypes_structures_match_the_header():
    """The ctypes mirrors of imq_problem, imq_qweight, imq_step_layer, imq_step_desc and
    imq_qmv_stage have the C compiler's sizes and field offsets."""
    mirrors = {"imq_problem": _native.Problem, "imq_qweight": _native.QWeight,
               "imq_step_layer": _native.StepLayer, "imq_step_desc": _native.StepDesc,
               "imq_qmv_stage": _native.QmvStage}
    structs = {name: [f for f, _ in cls._fields_] for name, cls in mirrors.items()}
    got = _c_layout(structs)
    for name, cls in mirrors.items():
        assert got[name] == ctypes.sizeof(cls), name
        for f, _ in cls._fields_:
            assert got[f"{name}.{f}"] == getattr(cls, f).offset, (name, f)


def test_workspace_keys_follow_the_current_stream(monkeypatch):
    """A launch with stream=None keys its split workspace by the stream that is current
    at the call, so calls under different current streams never share split counters."""
    from types import SimpleNamespace

    current = {"s": SimpleNamespace(cuda_stream=0x1000)}
    monkeypatch.setattr(_native.torch.cuda, "current_stream", lambda *a, **k: current["s"])
    monkeypatch.setattr(_native.torch.cuda, "current_device", lambda: 0)
    first = _native._workspace_key("cuda:0", None)
    current["s"] = SimpleNamespace(cuda_stream=0x2000)
    second = _native._workspace_key("cuda:0", None)
    assert first != second
    explicit = _native._workspace_key("cuda:0", SimpleNamespace(cuda_stream=0x2000))
    assert explicit == second
    assert _native._workspace_key("cuda:1", None)[0] == 1
