"""Runtime node of the quantized-matmul path (mirror of cider-press-runtime at the
scope of this path), backed by libcpq.so's graph API.

    Quantization         -> crates/cider-press-runtime/src/quantization.rs:43-153
    QuantizedWeight      -> crates/cider-press-runtime/src/quantized.rs:35-201
    Tensor.quantized_matmul / dequantize_affine / eval
                         -> tensor.rs:2064-2171, 1558-1637, 2681; eval.rs:1293-1394
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .kernels import Device

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)


class Quantization:
    """{bits, group_size}; validated on construction (quantization.rs:60-106)."""

    def __init__(self, bits: int, group_size: int):
        _lib.check(_lib.lib().cpq_quantization_validate(bits, group_size))
        self._bits = bits
        self._gs = group_size

    @property
    def bits(self) -> int:
        return self._bits

    @property
    def group_size(self) -> int:
        return self._gs

    def validate(self) -> None:
        _lib.check(_lib.lib().cpq_quantization_validate(self._bits, self._gs))

    def packed_word_count(self, scalar_count: int) -> int:
        out = ctypes.c_size_t()
        _lib.check(_lib.lib().cpq_packed_word_count(self._bits, self._gs, scalar_count, ctypes.byref(out)))
        return out.value

    def group_count(self, scalar_count: int) -> int:
        out = ctypes.c_size_t()
        _lib.check(_lib.lib().cpq_group_count(self._bits, self._gs, scalar_count, ctypes.byref(out)))
        return out.value

    def __eq__(self, other):
        return isinstance(other, Quantization) and (self.bits, self.group_size) == (other.bits, other.group_size)

    def __repr__(self):
        return f"Quantization(bits={self._bits}, group_size={self._gs})"


Q4_GS64 = None  # set lazily (constructing validates through the library)


def q4_gs64() -> Quantization:
    global Q4_GS64
    if Q4_GS64 is None:
        Q4_GS64 = Quantization(4, 64)
    return Q4_GS64


def _bytes(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(a, np.uint8) if isinstance(a, (bytes, bytearray))
                                else np.asarray(a).view(np.uint8).reshape(-1))


class QuantizedWeight:
    """Three-buffer quantized leaf with logical vs physical K (quantized.rs:35-125)."""

    def __init__(self, handle, device: Device, shape, k_logical: int, quantization: Quantization, dtype: str):
        self._h = handle
        self.device = device
        self._shape = tuple(shape)
        self._k_logical = k_logical
        self._q = quantization
        self.dtype = dtype
        self._lib = _lib.lib()

    @staticmethod
    def from_bytes(device: Device, shape, quantization: Quantization, weights, scales, biases,
                   dtype: str = "bf16") -> "QuantizedWeight":
        n, k = QuantizedWeight._rank2(shape)
        return QuantizedWeight._make(device, n, k, k, quantization, weights, scales, biases, dtype)

    @staticmethod
    def from_bytes_k_padded(device: Device, shape, k_logical: int, quantization: Quantization, weights, scales,
                            biases, dtype: str = "bf16") -> "QuantizedWeight":
        n, k = QuantizedWeight._rank2(shape)
        return QuantizedWeight._make(device, n, k, k_logical, quantization, weights, scales, biases, dtype)

    @staticmethod
    def _rank2(shape):
        """[N, K] or InvalidArgument (quantized.rs:137-143)."""
        dims = tuple(int(d) for d in shape)
        if len(dims) != 2:
            raise _lib.InvalidArgument(f"QuantizedWeight: shape must be rank 2 ([N, K]); got rank {len(dims)} "
                                       f"({list(dims)})")
        return dims

    @staticmethod
    def _make(device, n, k_phys, k_log, q, weights, scales, biases, dtype):
        w, s, b = _bytes(weights), _bytes(scales), _bytes(biases)
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_qweight_from_bytes(
            device.handle, _lib.DTYPES[dtype], n, k_phys, k_log, q.bits, q.group_size,
            w.ctypes.data_as(ctypes.c_void_p), w.nbytes, s.ctypes.data_as(ctypes.c_void_p), s.nbytes,
            b.ctypes.data_as(ctypes.c_void_p), b.nbytes, ctypes.byref(h)))
        return QuantizedWeight(h, device, (n, k_phys), k_log, q, dtype)

    @property
    def handle(self):
        return self._h

    def shape(self):
        return self._shape

    def k_logical(self) -> int:
        return self._k_logical

    def quantization(self) -> Quantization:
        return self._q

    def __del__(self):
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_qweight_release(self._h)
            self._h = None


class Tensor:
    """Dense tensor handle; op results are lazy until eval() (tensor.rs)."""

    def __init__(self, handle, device: Device, dtype: str, keep=()):
        self._h = handle
        self.device = device
        self.dtype = dtype
        self._keep = keep  # inputs kept alive for the lazy graph
        self._lib = _lib.lib()

    @staticmethod
    def from_host(device: Device, data: np.ndarray, dtype: str = "bf16") -> "Tensor":
        """BF16 / F16 data as raw uint16 bit patterns, or "u32" token ids."""
        a = np.ascontiguousarray(data, dtype=np.uint32 if dtype == "u32" else np.uint16)
        dims = (ctypes.c_size_t * max(1, a.ndim))(*a.shape)
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_tensor_from_host(device.handle, _lib.DTYPES[dtype], dims, a.ndim,
                                                   a.ctypes.data_as(ctypes.c_void_p), ctypes.byref(h)))
        return Tensor(h, device, dtype)

    def quantized_matmul(self, weight: QuantizedWeight, transpose: bool = True) -> "Tensor":
        h = ctypes.c_void_p()
        _lib.check(self._lib.cpq_tensor_quantized_matmul(self._h, weight.handle, int(bool(transpose)),
                                                         ctypes.byref(h)))
        return Tensor(h, self.device, weight.dtype, keep=(self, weight))

    @staticmethod
    def dequantize_affine(weight: QuantizedWeight) -> "Tensor":
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_tensor_dequantize(weight.handle, ctypes.byref(h)))
        return Tensor(h, weight.device, weight.dtype, keep=(weight,))

    @staticmethod
    def embed_tokens(input_ids: "Tensor", weight: QuantizedWeight) -> "Tensor":
        """embed_tokens (nn.rs:123-136) as a lazy node: rank-1 u32 ids."""
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().cpq_tensor_embed_tokens(input_ids._h, weight.handle, ctypes.byref(h)))
        return Tensor(h, weight.device, weight.dtype, keep=(input_ids, weight))

    def eval(self) -> "Tensor":
        _lib.check(self._lib.cpq_tensor_eval(self._h))
        return self

    def shape(self):
        dims = (ctypes.c_size_t * 16)()
        nd = ctypes.c_size_t()
        _lib.check(self._lib.cpq_tensor_shape(self._h, dims, 16, ctypes.byref(nd)))
        return tuple(dims[i] for i in range(nd.value))

    def cpu_slice(self) -> np.ndarray:
        """Host copy of the evaluated tensor as raw uint16 bit patterns, shaped."""
        shape = self.shape()
        out = np.empty(shape, np.uint32 if self.dtype == "u32" else np.uint16)
        _lib.check(self._lib.cpq_tensor_read(self._h, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def __del__(self):
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_tensor_release(self._h)
            self._h = None
