"""The ctypes boundary to libironmule_qmv.so (C ABI: include/ironmule_qmv.h).

Everything above this module passes torch tensors; everything below it is plain device
pointers, sizes and a HIP stream.  There is no fallback: if the library is missing or
the device is not a gfx950, calls raise `NativeUnavailable`.

Tensor conventions (the reference's buffers, ironmule/qmv_k3840.py:379-408):
  w       torch.int32 or torch.uint32 (N, K/8): packed words, low nibble first
  scales  torch.bfloat16 (N, K/64);  biases torch.bfloat16 (N, K/64)
  x       torch.bfloat16 (K,) or (M, K), M <= 32
  y       torch.bfloat16 or torch.float32 (M, N)
"""

from __future__ import annotations

import ctypes
import os
import re
import threading

import torch

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libironmule_qmv.so")
HEADER_PATH = os.path.join(ROOT, "include", "ironmule_qmv.h")
HEADER_PATHS = [HEADER_PATH, os.path.join(ROOT, "include", "ironmule_decode.h"),
                os.path.join(ROOT, "include", "ironmule_step.h")]

GROUP_SIZE = 64
BITS = 4
MAX_ROWS = 32

IMQ_OK, IMQ_EINVAL, IMQ_EUNSUPPORTED, IMQ_EUNAVAILABLE, IMQ_ELAUNCH = 0, 1, 2, 3, 6
IMQ_BF16, IMQ_F32, IMQ_F16 = 0, 1, 2
_DTYPE_CODE = {torch.bfloat16: IMQ_BF16, torch.float32: IMQ_F32, torch.float16: IMQ_F16}


class NativeUnavailable(RuntimeError):
    """The HIP library is not built, not loadable, or the device is not a gfx950."""


class NativeError(RuntimeError):
    """The C ABI refused a call; `code` is its IMQ_* return code."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"[imq code {code}] {message}")
        self.code = code


_lib = None
_lock = threading.Lock()

_P = ctypes.c_void_p
_I32, _I64 = ctypes.c_int32, ctypes.c_int64
MAX_PROBLEMS = 8


class Problem(ctypes.Structure):
    """imq_problem: one weight and its activation/output rows for imq_qmv_grouped."""

    _fields_ = [("w", _P), ("scales", _P), ("biases", _P), ("x", _P), ("ldx", _I64),
                ("y", _P), ("ldy", _I64), ("N", _I32), ("K", _I32)]


class NormIn(ctypes.Structure):
    """imq_norm_in: per-row partial sums of squares from which a projection scales its rows."""

    _fields_ = [("ssq", _P), ("tiles", _I32), ("ld", _I32), ("dim", _I32), ("eps", ctypes.c_float)]


class ResidualOut(ctypes.Structure):
    """imq_residual_out: h += bf16(y), x' = bf16(h * weight) and the tiles' sums of squares."""

    _fields_ = [("h", _P), ("ldh", _I64), ("weight", _P), ("x", _P), ("ldx", _I64), ("ssq", _P),
                ("ld", _I32)]


class QWeight(ctypes.Structure):
    """imq_qweight: packed words, bf16 scales, bf16 biases."""

    _fields_ = [("w", _P), ("scales", _P), ("biases", _P)]


class StepLayer(ctypes.Structure):
    """imq_step_layer: one decoder layer's tensors for the persistent decode program."""

    _fields_ = [("q", QWeight), ("k", QWeight), ("v", QWeight), ("o", QWeight), ("gate", QWeight),
                ("up", QWeight), ("down", QWeight), ("input_norm", _P), ("post_norm", _P),
                ("q_norm", _P), ("k_norm", _P), ("k_pool", _P), ("v_pool", _P)]


class StepDesc(ctypes.Structure):
    """imq_step_desc: shapes and device tensors of a decode step."""

    _fields_ = [("layers", _I32), ("batch", _I32), ("hidden", _I32), ("heads", _I32),
                ("kv_heads", _I32), ("intermediate", _I32), ("vocab", _I32), ("capacity", _I32),
                ("num_slots", _I32), ("max_len", _I32), ("eps", ctypes.c_float),
                ("theta", ctypes.c_float), ("layer", ctypes.POINTER(StepLayer)),
                ("final_norm", _P), ("head", QWeight), ("positions", _P), ("slots", _P), ("h", _P),
                ("logits", _P)]


class QmvStage(ctypes.Structure):
    """imq_qmv_stage: 1-3 one-row qmv problems sharing x, optionally after the previous stage."""

    _fields_ = [("count", _I32), ("wait_previous", _I32), ("problems", Problem * 3)]


_SIGNATURES = {
    "imq_abi_version": ([], _I32),
    "imq_device_check": ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_I32)], _I32),
    "imq_qmv": ([_P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _P], _I32),
    "imq_qmv_multi": ([_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P], _I32),
    "imq_qmv_grouped": ([ctypes.POINTER(Problem), _I32, _I32, _I32, _I32, _I32, _P], _I32),
    "imq_qmv_grouped_workspace": ([ctypes.POINTER(Problem), _I32, _I32], ctypes.c_size_t),
    "imq_qmv_grouped_ws": ([ctypes.POINTER(Problem), _I32, _I32, _I32, _I32, _I32, _P,
                            ctypes.c_size_t, _P], _I32),
    "imq_qmv_grouped_noalloc": ([ctypes.POINTER(Problem), _I32, _I32, _I32, _I32, _I32, _P],
                                _I32),
    "imq_qmv_gate_up_silu": ([_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32, _I32,
                              _I32, _P], _I32),
    "imq_qmv_norm_workspace": ([ctypes.POINTER(Problem), _I32, _I32], ctypes.c_size_t),
    "imq_qmv_norm": ([ctypes.POINTER(Problem), _I32, _I32, _I32, _I32, ctypes.POINTER(NormIn),
                      ctypes.POINTER(ResidualOut), _P, ctypes.c_size_t, _P], _I32),
    "imq_qmv_norm_splits": ([ctypes.POINTER(Problem), _I32, _I32], _I32),
    "imq_qmv_norm_planes": ([ctypes.POINTER(Problem), _I32, _I32, _I32, _I32, ctypes.POINTER(NormIn),
                             _P, _I64, ctypes.POINTER(_I32), _P], _I32),
    "imq_residual_planes": ([_P, _I32, _I32, _I32, ctypes.POINTER(ResidualOut), _P], _I32),
    "imq_qmv_residual_bands": ([ctypes.POINTER(Problem), _I32, _I32, _I32, ctypes.POINTER(ResidualOut), _P], _I32),
    "imq_qmv_gate_up_silu_norm_workspace": ([_I32, _I32, _I32], ctypes.c_size_t),
    "imq_qmv_gate_up_silu_norm": ([_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32,
                                   _I32, _I32, ctypes.POINTER(NormIn), _P, ctypes.c_size_t, _P],
                                  _I32),
    "imq_rmsnorm_prescale": ([_P, _P, _P, _P, _P, _I32, _I32, _I32, _P], _I32),
    "imq_dequant": ([_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P], _I32),
    "imq_gather_qmv": ([_P, _P, _P, _I32, _P, _I64, _I32, _P, _I32, _P, _I64, _I32, _I32, _I32,
                        _I32, _I32, _P], _I32),
    "imq_last_error": ([ctypes.c_char_p, ctypes.c_size_t], _I32),
    # decode-step kernels (include/ironmule_decode.h)
    "imq_embed": ([_P, _P, _P, _P, _P, _I32, _I32, _I32, _P], _I32),
    "imq_add_rmsnorm": ([_P, _P, _P, _P, _I32, _I32, ctypes.c_float, _P], _I32),
    "imq_qk_norm_rope": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32,
                          ctypes.c_float, ctypes.c_float, _P], _I32),
    "imq_attention_workspace": ([_I32, _I32, _I32], ctypes.c_size_t),
    "imq_attention_decode": ([_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32,
                              ctypes.c_float, _P, _P], _I32),
    "imq_attention_fused": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                             _I32, _I32, ctypes.c_float, ctypes.c_float, _P, _P, _P], _I32),
    "imq_attention_fused_planes": ([_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32,
                                    _I32, _I32, _I32, ctypes.c_float, ctypes.c_float, _P, _P, _P],
                                   _I32),
    "imq_silu_mul": ([_P, _P, _P, _I64, _P], _I32),
    # persistent programs (include/ironmule_step.h)
    "imq_decode_program_create": ([ctypes.POINTER(StepDesc), ctypes.POINTER(_P)], _I32),
    "imq_qmv_program_create": ([ctypes.POINTER(QmvStage), _I32, ctypes.POINTER(_P)], _I32),
    "imq_program_launch": ([_P, _P], _I32),
    "imq_program_launch_staged": ([_P, _P], _I32),
    "imq_program_status": ([_P, ctypes.POINTER(_I32)], _I32),
    "imq_program_info": ([_P, ctypes.POINTER(_I32), ctypes.POINTER(_I32), ctypes.POINTER(_I32),
                          ctypes.POINTER(_I32)], _I32),
    "imq_program_destroy": ([_P], None),
    # streaming engine (include/ironmule_step.h)
    "imq_stream_create": ([ctypes.POINTER(QmvStage), _I32, _I32, ctypes.POINTER(_P)], _I32),
    "imq_stream_launch": ([_P, _P], _I32),
    "imq_stream_status": ([_P, ctypes.POINTER(_I32)], _I32),
    "imq_stream_trace": ([_P, _P, _I64], _I32),
    "imq_stream_info": ([_P, ctypes.POINTER(_I32), ctypes.POINTER(_I32), ctypes.POINTER(_I32),
                         ctypes.POINTER(_I32), ctypes.POINTER(_I32)], _I32),
    "imq_stream_destroy": ([_P], None),
}


def declared_functions() -> list[str]:
    """Every function the public headers declare (what the library must export)."""
    names = []
    for path in HEADER_PATHS:
        text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        names += re.findall(r"^\s*IMQ_API\s+\w+\s+(imq_\w+)\s*\(", text, flags=re.M)
    return names


def lib() -> ctypes.CDLL:
    """Load the library once.  Raises NativeUnavailable if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeUnavailable(
                        f"{LIB_PATH} is not built; run `python -m ironmule_amd.build`")
                try:
                    handle = ctypes.CDLL(LIB_PATH)
                except OSError as exc:
                    raise NativeUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
                for name, (args, res) in _SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = handle
    return _lib


def last_error() -> tuple[int, str]:
    buf = ctypes.create_string_buffer(512)
    code = lib().imq_last_error(buf, len(buf))
    return int(code), buf.value.decode(errors="replace")


def _check(code: int) -> None:
    if code != IMQ_OK:
        _, msg = last_error()
        if code == IMQ_EUNAVAILABLE:
            raise NativeUnavailable(msg)
        raise NativeError(code, msg)


def device_check() -> tuple[int, str, int]:
    """(code, arch, cu_count) for the current HIP device."""
    arch = ctypes.create_string_buffer(64)
    cus = _I32(0)
    code = lib().imq_device_check(arch, len(arch), ctypes.byref(cus))
    return int(code), arch.value.decode(), int(cus.value)


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(int(stream.cuda_stream))


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def check_weights(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> tuple[int, int]:
    """(N, K) of a well-formed 4-bit group-64 weight on a GPU, else ValueError."""
    if w.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"w must be int32/uint32 packed words, got {w.dtype}")
    if w.dim() != 2:
        raise ValueError(f"w must be (N, K/8), got {tuple(w.shape)}")
    n, k = int(w.shape[0]), int(w.shape[1]) * 8
    if k % GROUP_SIZE:
        raise ValueError(f"K={k} is not a multiple of {GROUP_SIZE}")
    for name, t in (("scales", scales), ("biases", biases)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
        if tuple(t.shape) != (n, k // GROUP_SIZE):
            raise ValueError(f"{name} must be {(n, k // GROUP_SIZE)}, got {tuple(t.shape)}")
    for name, t in (("w", w), ("scales", scales), ("biases", biases)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    return n, k


def qmv(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, x: torch.Tensor,
        out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
        stream=None) -> torch.Tensor:
    """y = x @ dequantize(w, scales, biases).T for M = x.shape[0] <= 32 rows, one weight
    sweep.  x is bf16 (K,) or (M, K); y is bf16 (default) or fp32, shape (M, N)."""
    n, k = check_weights(w, scales, biases)
    x2 = x.reshape(1, -1) if x.dim() == 1 else x
    if x2.dim() != 2 or int(x2.shape[1]) != k:
        raise ValueError(f"x must be (M, {k}), got {tuple(x.shape)}")
    if x2.dtype != torch.bfloat16:
        raise ValueError(f"x must be bfloat16, got {x2.dtype}")
    m = int(x2.shape[0])
    if not 1 <= m <= MAX_ROWS:
        raise ValueError(f"the qmv kernels take 1 to {MAX_ROWS} rows, got {m}")
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    dtype = out_dtype or (out.dtype if out is not None else torch.bfloat16)
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"output must be bfloat16 or float32, got {dtype}")
    if out is None:
        out = torch.empty((m, n), dtype=dtype, device=w.device)
    elif tuple(out.shape) != (m, n) or out.dtype != dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous (M, N) tensor of the output dtype")
    if m >= 3:  # the shared-weight MFMA path, with a workspace for split groups
        probs = (Problem * 1)()
        probs[0] = Problem(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), x2.data_ptr(), k,
                           out.data_ptr(), n, n, k)
        _grouped_launch(probs, 1, m, dtype, w.device, stream)
        return out
    _check(lib().imq_qmv(_ptr(w), _ptr(scales), _ptr(biases), _ptr(x2), k, _ptr(out), n,
                         m, n, k, GROUP_SIZE, BITS, _DTYPE_CODE[dtype], _stream(stream)))
    return out


_workspaces: dict = {}
# Every workspace a (device, stream) outgrew.  A HIP graph captured on that stream before
# the growth still holds the old pointer, so the old buffer is never released: a replay
# keeps reading and writing memory that is still its own, and its split counters are
# still zero (every call returns them to zero).
_retired: list = []


def _workspace_key(device, stream) -> tuple[int, int]:
    """(device index, stream handle) of a launch; stream None is the current stream of
    that device, resolved here so that launches under different current streams never
    share a workspace."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    if stream is None:
        stream = torch.cuda.current_stream(index)
    return index, int(stream.cuda_stream)


def _zeroed(words: int, index: int, stream) -> torch.Tensor:
    """A zero-filled fp32 tensor of `words` on device `index`, allocated and filled on
    `stream` (so the fill is ordered before the launch that uses it)."""
    s = stream if stream is not None else torch.cuda.current_stream(index)
    with torch.cuda.stream(s):
        return torch.zeros(words, dtype=torch.float32, device=torch.device("cuda", index))


def _workspace(nbytes: int, device, stream) -> torch.Tensor:
    """A zero-filled fp32 workspace of at least nbytes for (device, stream), kept for later
    calls: the library's split counters must be zero before a workspace's first use and
    every call leaves them at zero, so one workspace serves every call on that stream
    (calls on one stream never overlap).  A call that needs more gets a new, larger one;
    the smaller one is kept alive in `_retired` for the graphs that may hold it."""
    index, handle = _workspace_key(device, stream)
    key = (index, handle)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        if ws is not None:
            _retired.append(ws)
        ws = _zeroed(-(-nbytes // 4), index, stream)
        _workspaces[key] = ws
    return ws


def _grouped_launch(probs, count: int, m: int, dtype: torch.dtype, device, stream) -> None:
    """imq_qmv_grouped, through imq_qmv_grouped_ws with this stream's workspace when the
    library wants one (M >= 3 and few rows: the groups are split over more workgroups)."""
    nbytes = int(lib().imq_qmv_grouped_workspace(probs, count, m)) if m >= 3 else 0
    if nbytes == 0:
        _check(lib().imq_qmv_grouped(probs, count, m, GROUP_SIZE, BITS, _DTYPE_CODE[dtype],
                                     _stream(stream)))
        return
    ws = _workspace(nbytes, device, stream)
    _check(lib().imq_qmv_grouped_ws(probs, count, m, GROUP_SIZE, BITS, _DTYPE_CODE[dtype],
                                    _ptr(ws), ws.numel() * 4, _stream(stream)))


def qmv_multi(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
              vectors: list[torch.Tensor], out_dtype: torch.dtype = torch.bfloat16,
              outs: list[torch.Tensor] | None = None, stream=None) -> list[torch.Tensor]:
    """One weight sweep, len(vectors) separate results (each (1, N))."""
    n, k = check_weights(w, scales, biases)
    count = len(vectors)
    if not 1 <= count <= MAX_ROWS:
        raise ValueError(f"1 to {MAX_ROWS} vectors, got {count}")
    xs = []
    for v in vectors:
        if v.dtype != torch.bfloat16 or v.numel() != k:
            raise ValueError(f"every vector must be bf16 with {k} elements")
        xs.append(v if v.is_contiguous() else v.contiguous())
    if outs is None:
        outs = [torch.empty((1, n), dtype=out_dtype, device=w.device) for _ in range(count)]
    xa = (ctypes.c_void_p * count)(*[t.data_ptr() for t in xs])
    ya = (ctypes.c_void_p * count)(*[t.data_ptr() for t in outs])
    _check(lib().imq_qmv_multi(_ptr(w), _ptr(scales), _ptr(biases), xa, ya, count, n, k,
                               GROUP_SIZE, BITS, _DTYPE_CODE[out_dtype], _stream(stream)))
    return outs


def qmv_grouped(weights: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
                xs: list[torch.Tensor], outs: list[torch.Tensor] | None = None,
                out_dtype: torch.dtype = torch.bfloat16, stream=None) -> list[torch.Tensor]:
    """One launch for up to 8 weights, each with its own (M, K_i) activation rows (the
    same tensor may serve several weights, e.g. q/k/v); returns the (M, N_i) outputs."""
    count = len(weights)
    if not 1 <= count <= MAX_PROBLEMS or len(xs) != count:
        raise ValueError(f"1 to {MAX_PROBLEMS} weights with one activation each")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"output must be bfloat16 or float32, got {out_dtype}")
    probs = (Problem * count)()
    m = None
    result = []
    for i, ((w, s, b), x) in enumerate(zip(weights, xs)):
        n, k = check_weights(w, s, b)
        x2 = x.reshape(1, -1) if x.dim() == 1 else x
        if x2.dtype != torch.bfloat16 or x2.dim() != 2 or int(x2.shape[1]) != k:
            raise ValueError(f"activation {i} must be bf16 (M, {k})")
        if not x2.is_contiguous():
            raise ValueError(f"activation {i} must be contiguous")
        if m is None:
            m = int(x2.shape[0])
        elif int(x2.shape[0]) != m:
            raise ValueError("every weight of one call takes the same number of rows")
        if outs is None:
            y = torch.empty((m, n), dtype=out_dtype, device=w.device)
        else:
            y = outs[i]
            if tuple(y.shape) != (m, n) or y.dtype != out_dtype or not y.is_contiguous():
                raise ValueError(f"output {i} must be a contiguous ({m}, {n}) {out_dtype} tensor")
        probs[i] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x2.data_ptr(), k,
                           y.data_ptr(), n, n, k)
        result.append(y)
    if not 1 <= m <= MAX_ROWS:
        raise ValueError(f"the qmv kernels take 1 to {MAX_ROWS} rows, got {m}")
    _grouped_launch(probs, count, m, out_dtype, weights[0][0].device, stream)
    return result


def gather_qmv(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, x: torch.Tensor,
               idx: torch.Tensor, rows_per_x: int = 1, out_dtype: torch.dtype = torch.bfloat16,
               out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """MoE gather (imq_gather_qmv): y[p] = x[p // rows_per_x] @ dequant(w[idx[p]]).T for the
    P = idx.numel() pairs; w (E, N, K/8) int32, scales/biases (E, N, K/64) bf16, x (R, K)
    bf16 contiguous rows, idx int32 on the device.  Returns (P, N)."""
    if w.dim() != 3 or w.dtype != torch.int32:
        raise ValueError("w must be an (experts, N, K/8) int32 tensor")
    e, n, k = int(w.shape[0]), int(w.shape[1]), int(w.shape[2]) * 8
    for name, t in (("scales", scales), ("biases", biases)):
        if tuple(t.shape) != (e, n, k // GROUP_SIZE) or t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be a bf16 tensor of shape {(e, n, k // GROUP_SIZE)}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if not w.is_contiguous():
        raise ValueError("w must be contiguous")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != k or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous bf16 (rows, {k}) tensor")
    if idx.dtype != torch.int32 or idx.device != w.device:
        raise ValueError("idx must be an int32 tensor on the weights' device")
    idx = idx.reshape(-1).contiguous()
    pairs = int(idx.numel())
    if pairs < 1 or rows_per_x < 1 or -(-pairs // rows_per_x) > x.shape[0]:
        raise ValueError("need at least one pair and ceil(pairs / rows_per_x) activation rows")
    if out is None:
        out = torch.empty((pairs, n), dtype=out_dtype, device=w.device)
    elif tuple(out.shape) != (pairs, n) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous (pairs, N) tensor of the output dtype")
    _check(lib().imq_gather_qmv(_ptr(w), _ptr(scales), _ptr(biases), e, _ptr(x), k, int(rows_per_x),
                                _ptr(idx), pairs, _ptr(out), n, n, k, GROUP_SIZE, BITS,
                                _DTYPE_CODE[out_dtype], _stream(stream)))
    return out


def dequant(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
            out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """The dense (N, K) weight, scale*q + bias, as fp32 (bit-exact) or rounded to
    bf16/fp16."""
    n, k = check_weights(w, scales, biases)
    if out_dtype not in _DTYPE_CODE:
        raise ValueError(f"out_dtype must be fp32, bf16 or fp16, got {out_dtype}")
    if out is None:
        out = torch.empty((n, k), dtype=out_dtype, device=w.device)
    _check(lib().imq_dequant(_ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                             _DTYPE_CODE[out_dtype], n, k, GROUP_SIZE, BITS, _stream(stream)))
    return out


# --------------------------------------------------------------- decode-step kernels

def _require(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def embed(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, tokens: torch.Tensor,
          out: torch.Tensor, stream=None) -> torch.Tensor:
    """out (B, dim) fp32 = dequantised rows tokens[b] of a 4-bit embedding."""
    vocab, dim = check_weights(w, scales, biases)
    _require(tokens, torch.int32, "tokens")
    _require(out, torch.float32, "out")
    b = int(tokens.numel())
    if tuple(out.shape) != (b, dim):
        raise ValueError(f"out must be ({b}, {dim})")
    _check(lib().imq_embed(_ptr(w), _ptr(scales), _ptr(biases), _ptr(tokens), _ptr(out), b, vocab,
                           dim, _stream(stream)))
    return out


def add_rmsnorm(h: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float,
                delta: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """h += delta (if given); out = bf16 rms_norm(h) * weight, per row."""
    _require(h, torch.float32, "h")
    _require(weight, torch.bfloat16, "weight")
    _require(out, torch.bfloat16, "out")
    b, dim = h.shape
    if delta is not None:
        _require(delta, torch.bfloat16, "delta")
        if delta.numel() != h.numel():
            raise ValueError("delta must match h")
    if out.numel() != h.numel() or weight.numel() != dim:
        raise ValueError("out must match h and weight its row length")
    _check(lib().imq_add_rmsnorm(_ptr(h), _ptr(delta) if delta is not None else None, _ptr(weight),
                                 _ptr(out), b, dim, float(eps), _stream(stream)))
    return out


def qk_norm_rope(q, k, v, q_norm, k_norm, positions, slots, q_out, k_pool, v_pool, theta: float,
                 eps: float, stream=None) -> None:
    """Per-head RMSNorm + rotary embedding of q and k; q to q_out, k and v into the pools
    (slots, kv_heads, capacity, 128)."""
    for name, t in (("q", q), ("k", k), ("v", v), ("q_norm", q_norm), ("k_norm", k_norm),
                    ("q_out", q_out), ("k_pool", k_pool), ("v_pool", v_pool)):
        _require(t, torch.bfloat16, name)
    _require(positions, torch.int32, "positions")
    _require(slots, torch.int32, "slots")
    num_slots, hkv, capacity, d = k_pool.shape
    b = int(positions.numel())
    hq = q.numel() // (b * d)
    if d != 128 or v_pool.shape != k_pool.shape or k.numel() != b * hkv * d or q_out.numel() != q.numel():
        raise ValueError("inconsistent q/k/v/pool shapes (head dim 128)")
    _check(lib().imq_qk_norm_rope(_ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm),
                                  _ptr(positions), _ptr(slots), _ptr(q_out), _ptr(k_pool),
                                  _ptr(v_pool), b, hq, hkv, capacity, num_slots, float(theta),
                                  float(eps), _stream(stream)))


def attention_workspace(b: int, hq: int, max_len: int) -> int:
    """fp32 elements of workspace imq_attention_decode needs."""
    return int(lib().imq_attention_workspace(b, hq, max_len)) // 4


def attention_fused(q, k, v, q_norm, k_norm, positions, slots, k_pool, v_pool, out,
                    max_len: int, theta: float, eps: float, workspace: torch.Tensor,
                    counters: torch.Tensor, stream=None) -> torch.Tensor:
    """One launch: q/k RMSNorm + rotary, this step's k and v into the pools at `positions`,
    and out (B, Hq, 128) bf16 = grouped-query attention over rows 0 .. positions[b] of each
    request's slot; the same bits as qk_norm_rope followed by attention_decode.  `counters`
    is (B * kv_heads,) int32, zero before the first call and left at zero."""
    for name, t in (("q", q), ("k", k), ("v", v), ("q_norm", q_norm), ("k_norm", k_norm),
                    ("k_pool", k_pool), ("v_pool", v_pool), ("out", out)):
        _require(t, torch.bfloat16, name)
    _require(positions, torch.int32, "positions")
    _require(slots, torch.int32, "slots")
    _require(workspace, torch.float32, "workspace")
    _require(counters, torch.int32, "counters")
    num_slots, hkv, capacity, d = k_pool.shape
    b = int(positions.numel())
    hq = q.numel() // (b * d)
    if (d != 128 or v_pool.shape != k_pool.shape or k.numel() != b * hkv * d
            or v.numel() != b * hkv * d or out.numel() != q.numel() or slots.numel() != b):
        raise ValueError("inconsistent q/k/v/pool/out shapes (head dim 128)")
    if workspace.numel() < attention_workspace(b, hq, max_len):
        raise ValueError("workspace too small")
    if counters.numel() < b * hkv:
        raise ValueError("counters too small")
    _check(lib().imq_attention_fused(_ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm),
                                     _ptr(positions), _ptr(slots), _ptr(k_pool), _ptr(v_pool),
                                     _ptr(out), b, hq, hkv, capacity, num_slots, int(max_len),
                                     float(theta), float(eps), _ptr(workspace), _ptr(counters),
                                     _stream(stream)))
    return out


class QkvPlanes:
    """fp32 output planes of the q/k/v projections for `rows` requests (imq_qmv_norm_planes),
    read and reduced by attention_fused_planes: problem i (q, k, v) at offset i * pstride."""

    def __init__(self, rows: int, hq: int, hkv: int, device, max_planes: int = 4) -> None:
        self.rows, self.hq, self.hkv = rows, hq, hkv
        self.pstride = max_planes * rows * hq * 128
        self.max_planes = max_planes
        self.data = torch.empty(3 * self.pstride, dtype=torch.float32, device=device)
        self.planes = 0

    def view(self, i: int) -> torch.Tensor:
        """(planes, rows, N_i) of problem i, for tests."""
        width = (self.hq if i == 0 else self.hkv) * 128
        base = i * self.pstride
        return self.data[base:base + self.planes * self.rows * width].view(self.planes, self.rows, width)


def qmv_norm_planes(weights, x: torch.Tensor, out: QkvPlanes, norm_in: NormStats | None = None,
                    eps: float = 1e-6, stream=None, tiled: bool = False) -> int:
    """The q, k and v projections of x' rows (with the RMSNorm folded in when `norm_in` is
    given) as fp32 output planes, one per K-range of the plan, left for the reader to add
    (imq_qmv_norm_planes); returns the plane count."""
    if len(weights) != 3:
        raise ValueError("q, k and v: three weights")
    _require(x, torch.bfloat16, "x")
    m = out.rows
    if tiled:
        if not x.is_contiguous() or x.dim() != 1:
            raise ValueError("a tiled x is a contiguous tile-layout buffer (tile_rows)")
    elif x.dim() != 2 or not x.is_contiguous() or m != int(x.shape[0]):
        raise ValueError("x must be a contiguous (rows, K) tensor of the planes' rows")
    probs = (Problem * 3)()
    for i, (w, s, b) in enumerate(weights):
        n, k = check_weights(w, s, b)
        if (x.numel() != MAX_ROWS * k if tiled else int(x.shape[1]) != k) or n != (out.hq if i == 0 else out.hkv) * 128:
            raise ValueError(f"weight {i} does not match x or the planes' head counts")
        probs[i] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), LD_TILED if tiled else k,
                           None, n, n, k)
    nin = norm_in.norm_in(eps) if norm_in is not None else None
    splits = _I32(0)
    if int(lib().imq_qmv_norm_splits(probs, 3, m)) > out.max_planes:
        raise ValueError("the plan splits into more planes than the buffer holds")
    _check(lib().imq_qmv_norm_planes(probs, 3, m, GROUP_SIZE, BITS,
                                     ctypes.byref(nin) if nin is not None else None,
                                     _ptr(out.data), out.pstride, ctypes.byref(splits), _stream(stream)))
    out.planes = int(splits.value)
    return out.planes


def attention_fused_planes(qkv: QkvPlanes, q_norm, k_norm, positions, slots, k_pool, v_pool, out,
                           max_len: int, theta: float, eps: float, workspace: torch.Tensor,
                           counters: torch.Tensor, stream=None, tiled: bool = False) -> torch.Tensor:
    """attention_fused reading q, k and v as the planes of qmv_norm_planes (each value the
    sum of its planes in order, rounded to bf16).  With `tiled` out is a 32-row tile layout
    buffer of 32 * Hq * 128 elements (tile_rows) instead of (B, Hq * 128) rows."""
    for name, t in (("q_norm", q_norm), ("k_norm", k_norm), ("k_pool", k_pool), ("v_pool", v_pool),
                    ("out", out)):
        _require(t, torch.bfloat16, name)
    _require(positions, torch.int32, "positions")
    _require(slots, torch.int32, "slots")
    _require(workspace, torch.float32, "workspace")
    _require(counters, torch.int32, "counters")
    num_slots, hkv, capacity, d = k_pool.shape
    b = int(positions.numel())
    want = (MAX_ROWS if tiled else b) * qkv.hq * d
    if (d != 128 or v_pool.shape != k_pool.shape or hkv != qkv.hkv or b != qkv.rows
            or out.numel() != want or slots.numel() != b or qkv.planes < 1):
        raise ValueError("inconsistent planes/pool/out shapes (head dim 128)")
    if workspace.numel() < attention_workspace(b, qkv.hq, max_len):
        raise ValueError("workspace too small")
    if counters.numel() < b * hkv:
        raise ValueError("counters too small")
    _check(lib().imq_attention_fused_planes(_ptr(qkv.data), qkv.pstride, qkv.planes, _ptr(q_norm),
                                            _ptr(k_norm), _ptr(positions), _ptr(slots), _ptr(k_pool),
                                            _ptr(v_pool), _ptr(out), LD_TILED if tiled else qkv.hq * d, b,
                                            qkv.hq, hkv, capacity, num_slots,
                                            int(max_len), float(theta), float(eps), _ptr(workspace),
                                            _ptr(counters), _stream(stream)))
    return out


def attention_decode(q, k_pool, v_pool, lengths, slots, out, max_len: int, scale: float,
                     workspace: torch.Tensor, stream=None) -> torch.Tensor:
    """out (B, Hq, 128) bf16 = grouped-query attention of each request over its slot."""
    for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool), ("out", out)):
        _require(t, torch.bfloat16, name)
    _require(lengths, torch.int32, "lengths")
    _require(slots, torch.int32, "slots")
    _require(workspace, torch.float32, "workspace")
    num_slots, hkv, capacity, d = k_pool.shape
    b = int(lengths.numel())
    hq = q.numel() // (b * d)
    if workspace.numel() < attention_workspace(b, hq, max_len):
        raise ValueError("workspace too small")
    _check(lib().imq_attention_decode(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(lengths),
                                      _ptr(slots), _ptr(out), b, hq, hkv, capacity, num_slots,
                                      int(max_len), float(scale), _ptr(workspace),
                                      _stream(stream)))
    return out


def gate_up_silu(gate: tuple[torch.Tensor, torch.Tensor, torch.Tensor],
                 up: tuple[torch.Tensor, torch.Tensor, torch.Tensor], x: torch.Tensor,
                 out: torch.Tensor, stream=None) -> torch.Tensor:
    """out (M, N) bf16 = silu(bf16(x @ gate.T)) * bf16(x @ up.T), one launch; the bits of
    qmv_grouped over (gate, up) and silu_mul.  5 <= M <= 32, K a multiple of 256
    (NativeError with the unsupported code otherwise)."""
    n, k = check_weights(*gate)
    if check_weights(*up) != (n, k):
        raise ValueError("gate and up must have the same shape")
    _require(x, torch.bfloat16, "x")
    _require(out, torch.bfloat16, "out")
    if x.dim() != 2 or int(x.shape[1]) != k or tuple(out.shape) != (int(x.shape[0]), n):
        raise ValueError(f"x must be (M, {k}) and out (M, {n})")
    m = int(x.shape[0])
    _check(lib().imq_qmv_gate_up_silu(_ptr(gate[0]), _ptr(gate[1]), _ptr(gate[2]), _ptr(up[0]),
                                      _ptr(up[1]), _ptr(up[2]), _ptr(x), k, _ptr(out), n, m, n, k,
                                      GROUP_SIZE, BITS, _stream(stream)))
    return out


# ------------------------------------------------------- RMSNorm folded into projections

LD_TILED = 0  # IMQ_LD_TILED: an activation row stride that selects the 32-row tile layout


def tile_rows(x: torch.Tensor) -> torch.Tensor:
    """x (M <= 32, K) bf16 rows -> the 32-row tile layout (a (32 * K,) tensor, rows past M
    zero): element (m, k) at ((((k/64) * 4 + (k%32)/8) * 2 + (k%64)/32) * 32 + m) * 8 + k%8."""
    m, k = int(x.shape[0]), int(x.shape[1])
    if m > MAX_ROWS or k % 64:
        raise ValueError("at most 32 rows and K a multiple of 64")
    full = torch.zeros((MAX_ROWS, k), dtype=x.dtype, device=x.device)
    full[:m] = x
    # [m][g][kb][t][e] -> [g][t][kb][m][e]
    return full.view(MAX_ROWS, k // 64, 2, 4, 8).permute(1, 3, 2, 0, 4).contiguous().view(-1)


def untile_rows(t: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """The first m rows of a 32-row tile layout buffer of K columns, as (m, K) rows."""
    return t[:MAX_ROWS * k].view(k // 64, 4, 2, MAX_ROWS, 8).permute(3, 0, 2, 1, 4).reshape(MAX_ROWS, k)[:m]


class NormStats:
    """Per-row partial sums of squares of a residual stream h: `ssq` (rows, ld) fp32 with
    `tiles` partials per row, the input of a projection that folds in the RMSNorm
    (imq_norm_in).  The producer fills `tiles` of them: one for rmsnorm_prescale, one per
    64 columns of h for qmv_norm's residual epilogue."""

    def __init__(self, rows: int, dim: int, device) -> None:
        self.dim = dim
        tiles = -(-dim // 32)  # room for the row-band projections' 32-column partials
        self.ld = -(-tiles // 4) * 4
        self.ssq = torch.zeros((rows, self.ld), dtype=torch.float32, device=device)
        self.tiles = 1

    def norm_in(self, eps: float) -> NormIn:
        return NormIn(self.ssq.data_ptr(), self.tiles, self.ld, self.dim, float(eps))


def rmsnorm_prescale(h: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, stats: NormStats,
                     delta: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """h += delta (if given); out = bf16(h * weight) unnormalised, and one sum of squares per
    row into `stats` (the RMSNorm finished by the projection that reads `out`)."""
    _require(h, torch.float32, "h")
    _require(weight, torch.bfloat16, "weight")
    _require(out, torch.bfloat16, "out")
    b, dim = h.shape
    if delta is not None:
        _require(delta, torch.bfloat16, "delta")
        if delta.numel() != h.numel():
            raise ValueError("delta must match h")
    if out.numel() != h.numel() or weight.numel() != dim or stats.dim != dim or stats.ssq.shape[0] < b:
        raise ValueError("out must match h, weight and stats its row length")
    _check(lib().imq_rmsnorm_prescale(_ptr(h), _ptr(delta) if delta is not None else None,
                                      _ptr(weight), _ptr(out), _ptr(stats.ssq), stats.ld, b, dim,
                                      _stream(stream)))
    stats.tiles = 1
    return out


RESIDUAL_MAX_PLANES = 16  # planes imq_residual_planes adds


class ResidualPlanes:
    """fp32 K-range planes of one projection of `cols` columns for `rows` requests
    (imq_qmv_norm_planes over one weight), added into the residual stream by
    residual_planes: plane s, row m, column n at element (s * rows + m) * cols + n."""

    def __init__(self, rows: int, cols: int, device, max_planes: int = RESIDUAL_MAX_PLANES) -> None:
        if not 1 <= max_planes <= RESIDUAL_MAX_PLANES:
            raise ValueError(f"1 to {RESIDUAL_MAX_PLANES} planes")
        self.rows, self.cols, self.max_planes = rows, cols, max_planes
        self.data = torch.empty(max_planes * rows * cols, dtype=torch.float32, device=device)
        self.planes = 0

    def view(self) -> torch.Tensor:
        """(planes, rows, cols) of the last projection, for tests."""
        return self.data[:self.planes * self.rows * self.cols].view(self.planes, self.rows, self.cols)


def _one_problem(weight, x: torch.Tensor) -> tuple[ctypes.Array, int, int]:
    w, s, b = weight
    _require(x, torch.bfloat16, "x")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous (M, K) tensor")
    n, k = check_weights(w, s, b)
    if int(x.shape[1]) != k:
        raise ValueError(f"the weight takes K = {k}, x has {int(x.shape[1])}")
    probs = (Problem * 1)()
    probs[0] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), k, None, n, n, k)
    return probs, n, k


def residual_split_planes(weight, x: torch.Tensor) -> int:
    """The K-ranges (planes) imq_qmv_norm_planes cuts this one-weight projection into at
    x's row count; 0 if it would refuse it."""
    probs, _, _ = _one_problem(weight, x)
    return int(lib().imq_qmv_norm_splits(probs, 1, int(x.shape[0])))


def qmv_residual_planes(weight, x: torch.Tensor, out: ResidualPlanes, stream=None, tiled: bool = False) -> int:
    """One projection of x (M, K) as fp32 K-range planes (imq_qmv_norm_planes, no input
    norm), left for residual_planes to add; returns the plane count.  With `tiled` x is a
    32-row tile layout buffer (tile_rows) of out.rows rows."""
    if tiled:
        w, s, b = weight
        n, k = check_weights(w, s, b)
        _require(x, torch.bfloat16, "x")
        if x.numel() != MAX_ROWS * k or not x.is_contiguous():
            raise ValueError(f"a tiled x holds 32 * {k} elements")
        probs = (Problem * 1)()
        probs[0] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), LD_TILED, None, n, n, k)
        m = out.rows
    else:
        probs, n, _ = _one_problem(weight, x)
        m = int(x.shape[0])
    if m != out.rows or n != out.cols:
        raise ValueError(f"the planes hold ({out.rows}, {out.cols}), the projection is ({m}, {n})")
    if int(lib().imq_qmv_norm_splits(probs, 1, m)) > out.max_planes:
        raise ValueError("the plan splits into more planes than the buffer holds")
    splits = _I32(0)
    _check(lib().imq_qmv_norm_planes(probs, 1, m, GROUP_SIZE, BITS, None, _ptr(out.data),
                                     out.max_planes * m * n, ctypes.byref(splits), _stream(stream)))
    out.planes = int(splits.value)
    return out.planes


def _check_x_out(next_norm, x_out, m: int, n: int, tiled: bool) -> None:
    if next_norm is None:
        return
    _require(next_norm, torch.bfloat16, "next_norm")
    want = (MAX_ROWS * n,) if tiled else (m, n)
    if x_out is None or tuple(x_out.shape) != want or x_out.dtype != torch.bfloat16:
        raise ValueError(f"x_out must be a {want} bf16 tensor")


def residual_planes(planes: ResidualPlanes, residual: torch.Tensor, next_norm: torch.Tensor | None = None,
                    x_out: torch.Tensor | None = None, stats_out: NormStats | None = None,
                    stream=None, tiled_out: bool = False) -> None:
    """qmv_norm's residual epilogue as a launch of its own (imq_residual_planes): y = the
    planes added in order, residual += bf16(y), x_out = bf16(residual * next_norm) and the
    per-tile sums of squares into stats_out; the bits of qmv_norm(..., residual=...)."""
    m, n = planes.rows, planes.cols
    if not 1 <= planes.planes <= planes.max_planes:
        raise ValueError("no planes to add")
    _require(residual, torch.float32, "residual")
    if tuple(residual.shape) != (m, n) or not residual.is_contiguous():
        raise ValueError(f"residual must be a contiguous ({m}, {n}) fp32 tensor")
    _check_x_out(next_norm, x_out, m, n, tiled_out)
    rout = ResidualOut(residual.data_ptr(), n, next_norm.data_ptr() if next_norm is not None else None,
                       x_out.data_ptr() if next_norm is not None else None, LD_TILED if tiled_out else n,
                       stats_out.ssq.data_ptr() if stats_out is not None else None,
                       stats_out.ld if stats_out is not None else 0)
    _check(lib().imq_residual_planes(_ptr(planes.data), planes.planes, m, n, ctypes.byref(rout),
                                     _stream(stream)))
    if stats_out is not None:
        stats_out.tiles = -(-n // 64)


def qmv_residual_bands(weight, x: torch.Tensor, rows: int, residual: torch.Tensor,
                       next_norm: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
                       stats_out: NormStats | None = None, tiled: bool = False, stream=None,
                       tiled_out: bool = False) -> None:
    """One projection of `rows` activation rows over bands of 32 weight rows and the whole K
    (imq_qmv_residual_bands): residual += bf16(x W^T), x_out = bf16(residual * next_norm) and
    per 32-column band the rows' sums of squares into stats_out.  x: (rows, K) rows, or with
    `tiled` a tile-layout buffer of 32 * K elements (tile_rows)."""
    w, s, b = weight
    n, k = check_weights(w, s, b)
    _require(x, torch.bfloat16, "x")
    if not 1 <= rows <= MAX_ROWS:
        raise ValueError("rows must be 1..32")
    if tiled:
        if x.numel() < MAX_ROWS * k or not x.is_contiguous():
            raise ValueError(f"a tiled x holds 32 * {k} elements")
    elif x.dim() != 2 or not x.is_contiguous() or tuple(x.shape) != (rows, k):
        raise ValueError(f"x must be a contiguous ({rows}, {k}) tensor")
    _require(residual, torch.float32, "residual")
    if tuple(residual.shape) != (rows, n) or not residual.is_contiguous():
        raise ValueError(f"residual must be a contiguous ({rows}, {n}) fp32 tensor")
    _check_x_out(next_norm, x_out, rows, n, tiled_out)
    probs = (Problem * 1)()
    probs[0] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), LD_TILED if tiled else k,
                       None, n, n, k)
    rout = ResidualOut(residual.data_ptr(), n, next_norm.data_ptr() if next_norm is not None else None,
                       x_out.data_ptr() if next_norm is not None else None, LD_TILED if tiled_out else n,
                       stats_out.ssq.data_ptr() if stats_out is not None else None,
                       stats_out.ld if stats_out is not None else 0)
    _check(lib().imq_qmv_residual_bands(probs, rows, GROUP_SIZE, BITS, ctypes.byref(rout), _stream(stream)))
    if stats_out is not None:
        stats_out.tiles = -(-n // 32)


def qmv_norm(weights: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]], x: torch.Tensor,
             outs: list[torch.Tensor] | None = None, norm_in: NormStats | None = None,
             eps: float = 1e-6, residual: torch.Tensor | None = None,
             next_norm: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
             stats_out: NormStats | None = None, stream=None):
    """Projections of one bf16 activation x (M, K) with the RMSNorm folded in (imq_qmv_norm).

    norm_in: x is x' = bf16(h * w) and every output row is scaled by 1/rms(h) from these
    statistics.  residual (one weight): no output is written; instead residual (M, N fp32)
    += bf16(y), x_out = bf16(residual * next_norm) and stats_out gets the per-tile sums of
    squares of the new residual.  Returns the bf16 outputs (none with a residual)."""
    count = len(weights)
    if not 1 <= count <= MAX_PROBLEMS:
        raise ValueError(f"1 to {MAX_PROBLEMS} weights")
    _require(x, torch.bfloat16, "x")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous (M, K) tensor")
    m = int(x.shape[0])
    if not 1 <= m <= MAX_ROWS:
        raise ValueError(f"the qmv kernels take 1 to {MAX_ROWS} rows, got {m}")
    if residual is not None and (count != 1 or outs is not None):
        raise ValueError("a residual epilogue takes one weight and writes no output")
    probs = (Problem * count)()
    result = []
    for i, (w, s, b) in enumerate(weights):
        n, k = check_weights(w, s, b)
        if int(x.shape[1]) != k:
            raise ValueError(f"weight {i} takes K = {k}, x has {int(x.shape[1])}")
        y = None
        if residual is None:
            y = outs[i] if outs is not None else torch.empty((m, n), dtype=torch.bfloat16, device=w.device)
            if tuple(y.shape) != (m, n) or y.dtype != torch.bfloat16 or not y.is_contiguous():
                raise ValueError(f"output {i} must be a contiguous ({m}, {n}) bf16 tensor")
            result.append(y)
        probs[i] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), k,
                           y.data_ptr() if y is not None else None, n, n, k)
    nin = norm_in.norm_in(eps) if norm_in is not None else None
    rout = None
    if residual is not None:
        n = int(weights[0][0].shape[0])
        _require(residual, torch.float32, "residual")
        if tuple(residual.shape) != (m, n) or not residual.is_contiguous():
            raise ValueError(f"residual must be a contiguous ({m}, {n}) fp32 tensor")
        if next_norm is not None:
            _require(next_norm, torch.bfloat16, "next_norm")
            if x_out is None or tuple(x_out.shape) != (m, n) or x_out.dtype != torch.bfloat16:
                raise ValueError(f"x_out must be a ({m}, {n}) bf16 tensor")
        rout = ResidualOut(residual.data_ptr(), n, next_norm.data_ptr() if next_norm is not None else None,
                           x_out.data_ptr() if next_norm is not None else None, n,
                           stats_out.ssq.data_ptr() if stats_out is not None else None,
                           stats_out.ld if stats_out is not None else 0)
    nbytes = int(lib().imq_qmv_norm_workspace(probs, count, m))
    ws = _workspace(nbytes, weights[0][0].device, stream) if nbytes else None
    _check(lib().imq_qmv_norm(probs, count, m, GROUP_SIZE, BITS,
                              ctypes.byref(nin) if nin is not None else None,
                              ctypes.byref(rout) if rout is not None else None,
                              _ptr(ws) if ws is not None else None, ws.numel() * 4 if ws is not None else 0,
                              _stream(stream)))
    if stats_out is not None:
        stats_out.tiles = -(-int(weights[0][0].shape[0]) // 64)
    return result


def gate_up_silu_norm(gate, up, x: torch.Tensor, out: torch.Tensor, norm_in: NormStats,
                      eps: float, stream=None, split_tail: bool = True, rows: int | None = None,
                      tiled_x: bool = False, tiled_out: bool = False) -> torch.Tensor:
    """gate_up_silu on x' = bf16(h * w) with the RMSNorm folded in: the gate and up rows are
    scaled by 1/rms(h) from `norm_in` before the SwiGLU.  With `split_tail` the tiles of the
    launch's last, partial round over the CUs run as K-parts (this stream's workspace).
    `tiled_x` / `tiled_out`: x / out are 32-row tile layout buffers (tile_rows) of `rows`
    rows instead of (M, K) / (M, N) rows."""
    n, k = check_weights(*gate)
    if check_weights(*up) != (n, k):
        raise ValueError("gate and up must have the same shape")
    _require(x, torch.bfloat16, "x")
    _require(out, torch.bfloat16, "out")
    m = int(rows if rows is not None else x.shape[0])
    if (x.numel() != MAX_ROWS * k if tiled_x else (x.dim() != 2 or tuple(x.shape) != (m, k))) or \
            (out.numel() != MAX_ROWS * n if tiled_out else tuple(out.shape) != (m, n)):
        raise ValueError(f"x must be (M, {k}) and out (M, {n}) rows, or tile-layout buffers")
    nin = norm_in.norm_in(eps)
    nbytes = int(lib().imq_qmv_gate_up_silu_norm_workspace(m, n, k)) if split_tail else 0
    ws = _workspace(nbytes, gate[0].device, stream) if nbytes else None
    _check(lib().imq_qmv_gate_up_silu_norm(_ptr(gate[0]), _ptr(gate[1]), _ptr(gate[2]), _ptr(up[0]),
                                           _ptr(up[1]), _ptr(up[2]), _ptr(x), LD_TILED if tiled_x else k,
                                           _ptr(out), LD_TILED if tiled_out else n, m, n,
                                           k, GROUP_SIZE, BITS, ctypes.byref(nin),
                                           _ptr(ws) if ws is not None else None,
                                           ws.numel() * 4 if ws is not None else 0, _stream(stream)))
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor, stream=None) -> torch.Tensor:
    """out = bf16(silu(gate) * up)."""
    for name, t in (("gate", gate), ("up", up), ("out", out)):
        _require(t, torch.bfloat16, name)
    if not gate.numel() == up.numel() == out.numel():
        raise ValueError("gate, up and out must have the same size")
    _check(lib().imq_silu_mul(_ptr(gate), _ptr(up), _ptr(out), int(gate.numel()), _stream(stream)))
    return out


# ------------------------------------------------------------ persistent programs


class Program:
    """A program of the persistent engine (include/ironmule_step.h): one launch runs all of
    its stages.  Holds references to every tensor the program points at, so they outlive
    it; `close()` (or garbage collection) frees the device tables."""

    def __init__(self, handle: ctypes.c_void_p, keep: list) -> None:
        self._handle = handle
        self._keep = keep

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise ValueError("the program is closed")
        return self._handle

    def launch(self, stream=None, staged: bool = False) -> None:
        """Enqueue one run on `stream` (capturable in a HIP graph): one persistent launch,
        or with `staged` one launch per stage."""
        fn = lib().imq_program_launch_staged if staged else lib().imq_program_launch
        _check(fn(self.handle, _stream(stream)))

    def failed(self) -> bool:
        """Synchronises the device; True if a run since the last call stopped on a bounded
        wait (the flag is then cleared)."""
        flag = _I32(0)
        _check(lib().imq_program_status(self.handle, ctypes.byref(flag)))
        return bool(flag.value)

    def info(self) -> dict:
        vals = [_I32(0) for _ in range(4)]
        _check(lib().imq_program_info(self.handle, *[ctypes.byref(v) for v in vals]))
        return dict(zip(("tasks", "stages", "workgroups", "lds_bytes"), (v.value for v in vals)))

    def close(self) -> None:
        if self._handle is not None and _lib is not None:
            _lib.imq_program_destroy(self._handle)
        self._handle = None
        self._keep = []

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def _qweight(w, s, b) -> QWeight:
    check_weights(w, s, b)
    return QWeight(w.data_ptr(), s.data_ptr(), b.data_ptr())


def _qmv_stages(stages: list[tuple[list, torch.Tensor, list, bool]]):
    """The imq_qmv_stage array of a chain of one-row qmv stages, and the tensors it
    points at."""
    if not stages:
        raise ValueError("a program needs at least one stage")
    arr = (QmvStage * len(stages))()
    keep = []
    for i, (weights, x, outs, wait_previous) in enumerate(stages):
        if not 1 <= len(weights) <= 3 or len(outs) != len(weights):
            raise ValueError("a stage has 1 to 3 weights and one output per weight")
        if x.dtype != torch.bfloat16 or not x.is_contiguous():
            raise ValueError("x must be a contiguous bf16 row")
        arr[i].count = len(weights)
        arr[i].wait_previous = int(bool(wait_previous))
        for k, ((w, s, b), y) in enumerate(zip(weights, outs)):
            n, kk = check_weights(w, s, b)
            if x.numel() != kk:
                raise ValueError(f"stage {i}: x has {x.numel()} values, the weight takes {kk}")
            if y.dtype != torch.bfloat16 or y.numel() != n or not y.is_contiguous():
                raise ValueError(f"stage {i}: output {k} must be a contiguous bf16 tensor of {n}")
            arr[i].problems[k] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(),
                                         kk, y.data_ptr(), n, n, kk)
            keep += [w, s, b, y]
        keep.append(x)
    return arr, keep


def qmv_program(stages: list[tuple[list, torch.Tensor, list, bool]]) -> Program:
    """A chain of one-row qmv stages, each (weights, x, outs, wait_previous): `weights`
    1-3 (w, scales, biases) triples sharing the bf16 row `x` (K,), `outs` their bf16 (N,)
    outputs; a stage with wait_previous starts after the previous one has finished."""
    arr, keep = _qmv_stages(stages)
    handle = _P()
    _check(lib().imq_qmv_program_create(arr, len(stages), ctypes.byref(handle)))
    return Program(handle, keep)


class StreamProgram:
    """A chain of one-row qmv stages run by the streaming engine (imq_stream_*): one
    persistent launch streams every stage's weights.  Holds references to the tensors it
    points at; `close()` (or garbage collection) frees its device tables."""

    def __init__(self, handle: ctypes.c_void_p, keep: list) -> None:
        self._handle = handle
        self._keep = keep
        self._trace = None

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise ValueError("the program is closed")
        return self._handle

    def launch(self, stream=None) -> None:
        """Enqueue one run on `stream` (capturable in a HIP graph)."""
        _check(lib().imq_stream_launch(self.handle, _stream(stream)))

    def failed(self) -> bool:
        """Synchronises the device; True if a run since the last call stopped on a bounded
        wait (the flag is then cleared)."""
        flag = _I32(0)
        _check(lib().imq_stream_status(self.handle, ctypes.byref(flag)))
        return bool(flag.value)

    def info(self) -> dict:
        vals = [_I32(0) for _ in range(5)]
        _check(lib().imq_stream_info(self.handle, *[ctypes.byref(v) for v in vals]))
        out = dict(zip(("tiles", "stages", "workgroups", "lds_bytes", "chained"),
                       (v.value for v in vals)))
        out["chained"] = bool(out["chained"])
        return out

    def trace(self, buffer: torch.Tensor | None) -> None:
        """Chained programs: later launches record four stamps per (stage, wavefront) into
        `buffer` (int64, stages * workgroups * 12 * 4 elements; imq_stream_trace), or stop
        recording (None).  The program keeps a reference to the buffer."""
        if buffer is None:
            _check(lib().imq_stream_trace(self.handle, None, 0))
            self._trace = None
            return
        _require(buffer, torch.int64, "trace buffer")
        if not buffer.is_contiguous():
            raise ValueError("the trace buffer must be contiguous")
        _check(lib().imq_stream_trace(self.handle, _ptr(buffer), buffer.numel()))
        self._trace = buffer

    def close(self) -> None:
        if self._handle is not None and _lib is not None:
            _lib.imq_stream_destroy(self._handle)
        self._handle = None
        self._keep = []

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def stream_program(stages: list[tuple[list, torch.Tensor, list, bool]],
                   workgroups: int = 0) -> StreamProgram:
    """The chain of `qmv_program` run by the streaming engine: stages without any
    wait_previous are independent and stream with no synchronisation; with waits, a stage
    starts after the previous one has finished.  `workgroups` <= 0: the resident maximum."""
    arr, keep = _qmv_stages(stages)
    handle = _P()
    _check(lib().imq_stream_create(arr, len(stages), int(workgroups), ctypes.byref(handle)))
    return StreamProgram(handle, keep)


def decode_program(config, layers: list[dict], final_norm: torch.Tensor, head: tuple,
                   k_pools: list, v_pools: list, positions: torch.Tensor, slots: torch.Tensor,
                   h: torch.Tensor, logits: torch.Tensor, max_len: int) -> Program:
    """The persistent decode step of a Qwen3-style decoder at batch 1 (imq_step_desc):
    `layers` are dicts of (w, scales, biases) for q k v o gate up down plus bf16
    input_norm, post_norm, q_norm, k_norm; the pools are (slots, kv_heads, capacity, 128)
    bf16; positions/slots int32 (1,); h fp32 (1, hidden) holds the embedded token and is
    updated; logits fp32 (1, vocab) are written."""
    c = config
    for name, t, dt in (("positions", positions, torch.int32), ("slots", slots, torch.int32),
                        ("h", h, torch.float32), ("logits", logits, torch.float32),
                        ("final_norm", final_norm, torch.bfloat16)):
        _require(t, dt, name)
    arr = (StepLayer * len(layers))()
    keep = [positions, slots, h, logits, final_norm, *head]
    for i, L in enumerate(layers):
        for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
            _require(L[name], torch.bfloat16, name)
        _require(k_pools[i], torch.bfloat16, "k_pool")
        _require(v_pools[i], torch.bfloat16, "v_pool")
        arr[i] = StepLayer(*[_qweight(*L[nm]) for nm in ("q", "k", "v", "o", "gate", "up", "down")],
                           L["input_norm"].data_ptr(), L["post_norm"].data_ptr(),
                           L["q_norm"].data_ptr(), L["k_norm"].data_ptr(),
                           k_pools[i].data_ptr(), v_pools[i].data_ptr())
        keep += [t for nm in ("q", "k", "v", "o", "gate", "up", "down") for t in L[nm]]
        keep += [L[nm] for nm in ("input_norm", "post_norm", "q_norm", "k_norm")]
        keep += [k_pools[i], v_pools[i]]
    num_slots, _, capacity, _ = k_pools[0].shape
    desc = StepDesc(len(layers), int(h.shape[0]), c.hidden, c.heads, c.kv_heads, c.intermediate,
                    c.vocab, int(capacity), int(num_slots), int(max_len), float(c.eps),
                    float(c.theta), arr, final_norm.data_ptr(), _qweight(*head),
                    positions.data_ptr(), slots.data_ptr(), h.data_ptr(), logits.data_ptr())
    handle = _P()
    _check(lib().imq_decode_program_create(ctypes.byref(desc), ctypes.byref(handle)))
    return Program(handle, keep + [arr])
