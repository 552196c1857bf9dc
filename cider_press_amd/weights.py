"""On-disk format of the quantized weights: MLX-style safetensors archives.

Host mirror of the models crate's loader plumbing, backed by the native
loader in libcpq.so (csrc/safetensors.cpp):

- ``SafeTensors``: a parsed archive (safetensors::SafeTensors); ``open`` maps
  the file, ``deserialize`` takes bytes.
- ``read_quantized_weight``: the ``{base}.weight`` / ``.scales`` / ``.biases``
  triple as a ``QuantizedWeight`` (safetensors_io.rs:43-134).
- ``read_quantized_weight_k_padded``: the same, zero-padded along K
  (qwen2/weights.rs:297-307, build_padded_twin).
- ``read_dense_tensor``: one dense BF16/F16 tensor (safetensors_io.rs:25-32).
- ``pad_quantized_k``: the host padding routine (qwen2/weights.rs:316-376).
- ``quantization_from_config`` / ``derive_quantization``: the
  ``"quantization": {"group_size", "bits"}`` block of config.json
  (qwen2/config.rs:65-73, qwen2/weights.rs:412-420).

Errors are the models crate's kinds: ``MissingKey``, ``UnsupportedDtype``,
``ShapeMismatch``, ``SafetensorsError``, ``JsonError`` and
``InvalidArgument`` (cider_press_amd._lib).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Union

import numpy as np

from . import _lib
from .kernels import Device
from .runtime import Quantization, QuantizedWeight, Tensor

_NP_DTYPES = {
    "BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "F8_E5M2": np.uint8, "F8_E4M3": np.uint8,
    "I16": np.int16, "U16": np.uint16, "F16": np.uint16, "BF16": np.uint16, "I32": np.int32,
    "U32": np.uint32, "F32": np.float32, "F64": np.float64, "I64": np.int64, "U64": np.uint64,
}
_T = {0: "f32", 1: "f16", 2: "bf16"}


class TensorView:
    """One archive entry: dtype name, shape and a host copy of its bytes
    (16-bit floats as raw uint16 bit patterns)."""

    def __init__(self, dtype: str, shape, data: np.ndarray):
        self.dtype = dtype
        self.shape = tuple(shape)
        self.data = data

    def numpy(self) -> np.ndarray:
        return self.data.view(_NP_DTYPES[self.dtype]).reshape(self.shape)


class SafeTensors:
    """Parsed safetensors archive (header validated natively)."""

    def __init__(self, handle):
        self._h = handle
        self._lib = _lib.lib()

    @staticmethod
    def open(path: Union[str, os.PathLike]) -> "SafeTensors":
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_safetensors_open(os.fsencode(path), ctypes.byref(h)))
        return SafeTensors(h)

    @staticmethod
    def deserialize(data: bytes) -> "SafeTensors":
        buf = np.frombuffer(bytes(data), np.uint8)
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_safetensors_deserialize(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes,
                                                          ctypes.byref(h)))
        return SafeTensors(h)

    @property
    def handle(self):
        return self._h

    def names(self) -> list:
        n = ctypes.c_size_t()
        _lib.check(self._lib.cpq_safetensors_len(self._h, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            p = ctypes.c_char_p()
            _lib.check(self._lib.cpq_safetensors_name(self._h, i, ctypes.byref(p)))
            out.append(p.value.decode())
        return out

    def info(self, key: str):
        """(dtype name, shape) of one entry, without copying its bytes."""
        dt, shape, _, _ = self._entry(key)
        return dt, shape

    def tensor(self, key: str) -> TensorView:
        dt, shape, ptr, nbytes = self._entry(key)
        raw = np.empty(nbytes, np.uint8)
        if nbytes:
            ctypes.memmove(raw.ctypes.data, ptr, nbytes)
        return TensorView(dt, shape, raw)

    def _entry(self, key: str):
        dt = ctypes.c_char_p()
        dims = (ctypes.c_size_t * 16)()
        nd = ctypes.c_size_t()
        data = ctypes.c_void_p()
        nbytes = ctypes.c_size_t()
        _lib.check(self._lib.cpq_safetensors_tensor(self._h, key.encode(), ctypes.byref(dt), dims, 16,
                                                    ctypes.byref(nd), ctypes.byref(data), ctypes.byref(nbytes)))
        return dt.value.decode(), tuple(dims[i] for i in range(nd.value)), data.value, nbytes.value

    def metadata(self, key: str) -> str:
        v = ctypes.c_char_p()
        _lib.check(self._lib.cpq_safetensors_metadata(self._h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cpq_safetensors_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        if getattr(self, "_lib", None) is not None:
            self.close()


def _wrap_qweight(h: ctypes.c_void_p, device: Device) -> QuantizedWeight:
    n, kp, kl = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    bits, gs, dt = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_int()
    _lib.check(_lib.lib().cpq_qweight_info(h, ctypes.byref(n), ctypes.byref(kp), ctypes.byref(kl),
                                           ctypes.byref(bits), ctypes.byref(gs), ctypes.byref(dt)))
    return QuantizedWeight(h, device, (n.value, kp.value), kl.value, Quantization(bits.value, gs.value),
                           _T[dt.value])


def read_quantized_weight(archive: SafeTensors, base_name: str, quantization: Quantization,
                          device: Optional[Device]) -> QuantizedWeight:
    """``{base_name}.weight`` (U32 [N, K*bits/32]) with ``.scales`` / ``.biases``
    ([N, K/gs]) as a QuantizedWeight of logical shape [N, K]."""
    h = ctypes.c_void_p()
    _lib.check(_lib.lib().cpq_read_quantized_weight(device.handle if device else None, archive.handle,
                                                    base_name.encode(), quantization.bits,
                                                    quantization.group_size, ctypes.byref(h)))
    return _wrap_qweight(h, device)


def read_quantized_weight_k_padded(archive: SafeTensors, base_name: str, quantization: Quantization,
                                   device: Optional[Device], k_pad: int) -> QuantizedWeight:
    """The triple zero-padded along K to ``k_pad``; logical K unchanged."""
    h = ctypes.c_void_p()
    _lib.check(_lib.lib().cpq_read_quantized_weight_k_padded(
        device.handle if device else None, archive.handle, base_name.encode(), quantization.bits,
        quantization.group_size, k_pad, ctypes.byref(h)))
    return _wrap_qweight(h, device)


def read_dense_tensor(archive: SafeTensors, key: str, device: Optional[Device]) -> Tensor:
    """One dense BF16/F16 entry as a leaf Tensor, shape taken verbatim."""
    h = ctypes.c_void_p()
    _lib.check(_lib.lib().cpq_read_dense_tensor(device.handle if device else None, archive.handle,
                                                key.encode(), ctypes.byref(h)))
    dt, _ = archive.info(key)
    return Tensor(h, device, "bf16" if dt == "BF16" else "f16")


def pad_quantized_k(weights, scales, biases, n: int, k: int, k_pad: int, quantization: Quantization):
    """Zero-pad packed rows from k to k_pad columns (pad groups: zero words,
    zero scales, zero biases).  Returns (weights, scales, biases) as bytes."""
    w = np.ascontiguousarray(np.frombuffer(bytes(weights), np.uint8))
    s = np.ascontiguousarray(np.frombuffer(bytes(scales), np.uint8))
    b = np.ascontiguousarray(np.frombuffer(bytes(biases), np.uint8))
    bits, gs = quantization.bits, quantization.group_size
    # The reference's preconditions, in its order (weights.rs:327-351).
    if k % gs:
        raise _lib.InvalidArgument(f"pad_quantized_k: k={k} must be a multiple of group_size={gs}")
    if k_pad < k:
        raise _lib.InvalidArgument(f"pad_quantized_k: k_pad={k_pad} must be >= k={k}")
    if k_pad % gs:
        raise _lib.InvalidArgument(f"pad_quantized_k: k_pad={k_pad} must be a multiple of group_size={gs}")
    if w.nbytes != n * k * bits // 8:
        raise _lib.InvalidArgument("pad_quantized_k: weights buffer length mismatch")
    if s.nbytes != n * (k // gs) * 2:
        raise _lib.InvalidArgument("pad_quantized_k: scales buffer length mismatch")
    if b.nbytes != n * (k // gs) * 2:
        raise _lib.InvalidArgument("pad_quantized_k: biases buffer length mismatch")
    wo = np.empty(n * k_pad * bits // 8, np.uint8)
    so = np.empty(n * (k_pad // gs) * 2, np.uint8)
    bo = np.empty(n * (k_pad // gs) * 2, np.uint8)
    _lib.check(_lib.lib().cpq_pad_quantized_k(w.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p),
                                              b.ctypes.data_as(ctypes.c_void_p), n, k, k_pad, bits, gs, 2,
                                              wo.ctypes.data_as(ctypes.c_void_p), so.ctypes.data_as(ctypes.c_void_p),
                                              bo.ctypes.data_as(ctypes.c_void_p)))
    return wo.tobytes(), so.tobytes(), bo.tobytes()


def quantization_from_config(config: Union[bytes, str, os.PathLike]) -> Optional[Quantization]:
    """The config.json quantization block, or None when absent / null.
    ``config`` is the JSON text (str or bytes) or a path (os.PathLike) to
    config.json."""
    if isinstance(config, os.PathLike):
        with open(config, "rb") as f:
            data = f.read()
    else:
        data = config.encode() if isinstance(config, str) else bytes(config)
    present, bits, gs = ctypes.c_int(), ctypes.c_uint32(), ctypes.c_uint32()
    _lib.check(_lib.lib().cpq_quantization_from_config(data, len(data), ctypes.byref(present), ctypes.byref(bits),
                                                       ctypes.byref(gs)))
    return Quantization(bits.value, gs.value) if present.value else None


def derive_quantization(config) -> Quantization:
    """derive_quantization (qwen2/weights.rs:412-420): the checkpoint must be
    pre-quantized, and (bits, group_size) must be a supported pair."""
    q = quantization_from_config(config)
    if q is None:
        raise _lib.InvalidArgument(
            "config.quantization is None -- this loader requires a pre-quantized checkpoint")
    q.validate()
    return q
