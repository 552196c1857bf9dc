"""ctypes front end of the CPU oracle (``oracle/cpq_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- never by the product package.

All 16-bit float arrays cross this boundary as raw ``uint16`` bit patterns
(numpy has no bfloat16); ``dtype`` is ``"bf16"`` or ``"f16"``.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libcpq_oracle.so")

_DT = {"f32": 0, "f16": 1, "bf16": 2}

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t
_i = ctypes.c_int

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_unpack_row.argtypes = [_u32p, _i, _sz, _u8p]
        L.or_pack_row.argtypes = [_u8p, _i, _sz, _u32p]
        L.or_dequantize.argtypes = [_u32p, _u16p, _u16p, _sz, _sz, _i, _i, _i, _u16p]
        L.or_qmm_ref.argtypes = [_u16p, _sz, _u32p, _u16p, _u16p, _sz, _sz, _i, _i, _i, _f64p, _i]
        L.or_gather_qmm_ref.argtypes = [
            _u16p, ctypes.c_void_p, _u32p, _sz, _u32p, _u16p, _u16p, _sz, _sz, _i, _i, _i, _f64p, _i]
        L.or_qmv_mlx.argtypes = [_u16p, _sz, _u32p, _u16p, _u16p, _sz, _sz, _i, _i, _i, _i, _f32p]
        L.or_qmv_mlx.restype = _i
        _lib = L
    return _lib


def _threads(threads):
    return int(threads) if threads else min(8, os.cpu_count() or 1)


# ----------------------------------------------------------------------------
# Conversions
# ----------------------------------------------------------------------------

def f32_to_bits(a, dtype: str) -> np.ndarray:
    """Round float32 values to T (RNE) and return the uint16 bit patterns."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == "f16":
        return a.astype(np.float16).view(np.uint16)
    out = np.empty(a.shape, np.uint16)
    flat, of = a.reshape(-1), out.reshape(-1)
    u = flat.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    of[:] = r
    return out


def bits_to_f32(b, dtype: str) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    if dtype == "bf16":
        return (b.astype(np.uint32) << 16).view(np.float32)
    return b.view(np.float16).astype(np.float32)


def c_f32_to_bits(v: float, dtype: str) -> int:
    """The C oracle's scalar conversion (pinned against numpy/torch in tests)."""
    return int(lib().or_f32_to_bf16(v) if dtype == "bf16" else lib().or_f32_to_f16(v))


def c_bits_to_f32(b: int, dtype: str) -> float:
    return float(lib().or_bf16_to_f32(b) if dtype == "bf16" else lib().or_f16_to_f32(b))


# ----------------------------------------------------------------------------
# Path functions
# ----------------------------------------------------------------------------

def unpack(w_q: np.ndarray, k: int, bits: int) -> np.ndarray:
    w_q = np.ascontiguousarray(w_q, dtype=np.uint32)
    rows = w_q.shape[0]
    out = np.empty((rows, k), np.uint8)
    for r in range(rows):
        lib().or_unpack_row(np.ascontiguousarray(w_q[r]), bits, k, out[r])
    return out


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows, k = q.shape
    out = np.empty((rows, k * bits // 32), np.uint32)
    for r in range(rows):
        lib().or_pack_row(np.ascontiguousarray(q[r]), bits, k, out[r])
    return out


def dequantize(w_q, scales, biases, rows: int, k: int, gs: int, bits: int, dtype: str) -> np.ndarray:
    out = np.empty((rows, k), np.uint16)
    lib().or_dequantize(np.ascontiguousarray(w_q, np.uint32), np.ascontiguousarray(scales, np.uint16),
                        np.ascontiguousarray(biases, np.uint16), rows, k, gs, bits, _DT[dtype], out)
    return out


def qmm_ref(x, w_q, scales, biases, m: int, n: int, k: int, gs: int, bits: int, dtype: str,
            threads=None) -> np.ndarray:
    """Unrounded float64 Y = X @ dequant(W)^T (dequantized weights rounded to T)."""
    y = np.empty((m, n), np.float64)
    lib().or_qmm_ref(np.ascontiguousarray(x, np.uint16), m, np.ascontiguousarray(w_q, np.uint32),
                     np.ascontiguousarray(scales, np.uint16), np.ascontiguousarray(biases, np.uint16),
                     n, k, gs, bits, _DT[dtype], y, _threads(threads))
    return y


def gather_qmm_ref(x, lhs, rhs, w_q, scales, biases, rows: int, n: int, k: int, gs: int, bits: int,
                   dtype: str, threads=None) -> np.ndarray:
    y = np.empty((rows, n), np.float64)
    lhs_arr = None if lhs is None else np.ascontiguousarray(lhs, np.uint32)
    lhs_ptr = None if lhs_arr is None else lhs_arr.ctypes.data_as(ctypes.c_void_p)
    lib().or_gather_qmm_ref(np.ascontiguousarray(x, np.uint16), lhs_ptr, np.ascontiguousarray(rhs, np.uint32),
                            rows, np.ascontiguousarray(w_q, np.uint32), np.ascontiguousarray(scales, np.uint16),
                            np.ascontiguousarray(biases, np.uint16), n, k, gs, bits, _DT[dtype], y,
                            _threads(threads))
    return y


def qmv_mlx(x, w_q, scales, biases, m: int, n: int, k: int, gs: int, bits: int, dtype: str,
            fast=None) -> np.ndarray:
    """MLX qmv arithmetic; returns the unrounded f32 output [m, n]."""
    if fast is None:
        fast = (n % 8 == 0) and (k % 512 == 0)
    y = np.empty((m, n), np.float32)
    rc = lib().or_qmv_mlx(np.ascontiguousarray(x, np.uint16), m, np.ascontiguousarray(w_q, np.uint32),
                          np.ascontiguousarray(scales, np.uint16), np.ascontiguousarray(biases, np.uint16),
                          n, k, gs, bits, _DT[dtype], int(bool(fast)), y)
    if rc != 0:
        raise ValueError(f"qmv_mlx: unsupported bits={bits}")
    return y


BASELINE_PATH = os.path.join(HERE, "_build", "libcpq_cpu_baseline.so")
BASELINE_FORMS = {"scalar": 0, "avx2": 1, "avx512": 2}
_base_lib = None


def _baseline_lib():
    """The CPU baseline (oracle/cpu_baseline.c: scalar, AVX2 and AVX-512
    forms of the dequantize-and-dot, dispatched at run time)."""
    global _base_lib
    if _base_lib is None:
        if not os.path.exists(BASELINE_PATH):
            build()
        L = ctypes.CDLL(BASELINE_PATH)
        L.cb_form_supported.argtypes = [_i]
        L.cb_form_supported.restype = _i
        L.cb_qmm.argtypes = [_u16p, _sz, _u32p, _u16p, _u16p, _sz, _sz, _i, _i, _i, _u16p, _i, _i]
        L.cb_qmm.restype = _i
        _base_lib = L
    return _base_lib


def baseline_forms() -> list:
    """The baseline forms this host runs, slowest first."""
    L = _baseline_lib()
    return [f for f, code in BASELINE_FORMS.items() if L.cb_form_supported(code)]


def cpu_baseline(x, w_q, scales, biases, m: int, n: int, k: int, gs: int, bits: int, dtype: str,
                 threads=None, form: str = "scalar") -> np.ndarray:
    """T-rounded dequantized weights, fp32 accumulation, output T (raw bits)."""
    y = np.empty((m, n), np.uint16)
    rc = _baseline_lib().cb_qmm(np.ascontiguousarray(x, np.uint16), m, np.ascontiguousarray(w_q, np.uint32),
                                np.ascontiguousarray(scales, np.uint16), np.ascontiguousarray(biases, np.uint16),
                                n, k, gs, bits, _DT[dtype], y, _threads(threads), BASELINE_FORMS[form])
    if rc != 0:
        raise ValueError(f"cpu_baseline: form {form!r} unavailable on this host or bad arguments")
    return y


# ----------------------------------------------------------------------------
# Fixture reader (safetensors header + raw little-endian payload; no pickle)
# ----------------------------------------------------------------------------

_ST_DT = {"BF16": np.uint16, "F16": np.uint16, "U32": np.uint32, "F32": np.float32, "U8": np.uint8}


def read_safetensors(path: str) -> dict:
    with open(path, "rb") as f:
        blob = f.read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        arr = np.frombuffer(blob[base + a:base + b], dtype=_ST_DT[meta["dtype"]]).reshape(meta["shape"])
        out[name] = arr.copy()
    return out


# ----------------------------------------------------------------------------
# Tolerance (BASELINE tolerance vs the unrounded oracle output)
# ----------------------------------------------------------------------------

def half_ulp(v: np.ndarray, dtype: str) -> np.ndarray:
    """Half the spacing of T around |v| (the rounding error of storing v as T)."""
    a = np.abs(np.asarray(v, np.float64))
    mant, min_exp = (7, -126) if dtype == "bf16" else (10, -14)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** min_exp)))
    return 0.5 * np.exp2(e - mant)


def tolerance_report(y_bits, y_ref: np.ndarray, x_bits, k: int, dtype: str) -> dict:
    """BASELINE tolerance against the unrounded reference:
    max abs error <= 1e-2*||x||_inf*sqrt(K)/64 and rel-L2 <= 2e-3.

    The output is stored in T, and storing the exact result already costs up
    to half a T-ULP (at |y| >= 16 in bf16 that is 0.0625, above the max-abs
    bound at K=4096).  So the max-abs bound is applied to the error beyond
    that unavoidable rounding ("excess"); rel-L2 is applied to the raw error
    (it is what separates T-rounded from unrounded weights), except for fewer
    than 4096 outputs, where the rounding of a handful of values dominates
    it and the excess is used instead."""
    y = bits_to_f32(y_bits, dtype).astype(np.float64).reshape(y_ref.shape)
    xmax = float(np.abs(bits_to_f32(x_bits, dtype)).max()) if np.size(x_bits) else 0.0
    err = y - y_ref
    excess = np.maximum(np.abs(err) - half_ulp(y_ref, dtype), 0.0)
    max_abs = float(np.abs(err).max()) if err.size else 0.0
    max_excess = float(excess.max()) if err.size else 0.0
    denom = float(np.linalg.norm(y_ref))
    rel = float(np.linalg.norm(err) / denom) if denom > 0 else float(np.linalg.norm(err))
    rel_excess = float(np.linalg.norm(excess) / denom) if denom > 0 else float(np.linalg.norm(excess))
    bound = 1e-2 * xmax * np.sqrt(k) / 64.0
    rel_ok = rel <= 2e-3 if err.size >= 4096 else rel_excess <= 2e-3
    return {"max_abs": max_abs, "max_abs_beyond_rounding": max_excess, "max_abs_bound": bound,
            "rel_l2": rel, "rel_l2_beyond_rounding": rel_excess, "rel_l2_bound": 2e-3,
            "ok": bool(max_excess <= bound and rel_ok and np.all(np.isfinite(y)))}
