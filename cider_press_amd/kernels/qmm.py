"""Quantized matrix-matrix dispatch (crates/cider-press-kernels/src/kernels/qmm.rs:66-220)."""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, KernelLibrary, _ptr


def affine_qmm_t(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                 x: Buffer, y: Buffer, m: int, n: int, k: int, group_size: int, bits: int) -> None:
    """Y[M,N] = X[M,K] . dequant(W[N,K])^T; T is scales.dtype. Encodes only."""
    del library
    _lib.check(_lib.lib().cpq_affine_qmm_t(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), len(x), _ptr(y), len(y), m, n, k, group_size, bits))


def affine_qmm_t_bf16(commands, library, w_q, scales, biases, x, y, m, n, k, group_size, bits):
    """The reference's bf16-typed entry point (qmm.rs:66-79)."""
    for b in (scales, biases, x, y):
        if b.dtype != "bf16":
            raise TypeError("affine_qmm_t_bf16: scales, biases, x and y must be bf16 buffers")
    affine_qmm_t(commands, library, w_q, scales, biases, x, y, m, n, k, group_size, bits)


def quantized_matmul(commands: Commands, w_q: Buffer, scales: Buffer, biases: Buffer, x: Buffer, y: Buffer,
                     m: int, n: int, k_physical: int, group_size: int, bits: int, x_len=None) -> None:
    """The runtime's routed dispatch (eval.rs:1293-1394): M==1 decode, small-M, or prefill."""
    _lib.check(_lib.lib().cpq_quantized_matmul(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), len(x) if x_len is None else x_len, x.alloc_len, _ptr(y),
        m, n, k_physical, group_size, bits))


def affine_qmm_n(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                 x: Buffer, y: Buffer, m: int, n: int, k: int, group_size: int, bits: int) -> None:
    """MLX transpose=false (quantized.h:1215-1349): Y[M,N] = X[M,K] . dequant(W) with
    W logically [K, N] (w_q [K, N*bits/32], scales/biases [K, N/gs]). Encodes only."""
    del library
    _lib.check(_lib.lib().cpq_affine_qmm_n(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), len(x), _ptr(y), len(y), m, n, k, group_size, bits))


def affine_qvm(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
               x: Buffer, y: Buffer, in_vec_size: int, out_vec_size: int, group_size: int, bits: int) -> None:
    """MLX affine_qvm (quantized.h:977-1086): y = x . dequant(W), W [in_vec_size, out_vec_size]."""
    affine_qmm_n(commands, library, w_q, scales, biases, x, y, 1, out_vec_size, in_vec_size, group_size, bits)


def _batch_args(batch_shape, *strides):
    import ctypes

    nd = len(batch_shape)
    shape = (ctypes.c_int * max(1, nd))(*batch_shape)
    arrs = [(ctypes.c_int64 * max(1, nd))(*st) for st in strides]
    return nd, shape, arrs


def affine_qmm_t_batched(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                         x: Buffer, y: Buffer, m: int, n: int, k: int, group_size: int, bits: int, batch_shape,
                         w_strides, s_strides, b_strides, x_strides) -> None:
    """MLX's batched qmm_t (adjust_matrix_offsets, quantized.h:1351-1388): for each
    element of batch_shape, its W / scales / biases / X at the given element
    strides (0 broadcasts); y holds one contiguous [M, N] block per element."""
    del library
    nd, shape, (ws, ss, bs, xs) = _batch_args(batch_shape, w_strides, s_strides, b_strides, x_strides)
    _lib.check(_lib.lib().cpq_affine_qmm_t_batched(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), len(x), _ptr(y), len(y), m, n, k, group_size, bits, nd, shape, ws, ss,
        bs, xs))
