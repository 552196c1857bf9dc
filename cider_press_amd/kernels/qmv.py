"""Quantized matrix-vector dispatch (crates/cider-press-kernels/src/kernels/qmv.rs:77-205)."""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, KernelLibrary, _ptr


def affine_qmv(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
               x: Buffer, y: Buffer, in_vec_size: int, group_size: int, bits: int) -> None:
    """y = x . dequant(w_q)^T for one activation row; T is scales.dtype.

    `in_vec_size` is the PHYSICAL K of the weight (qmv.rs:48-55): for a
    K-padded weight x is shorter and its allocation's zeroed slack is read.
    Encodes only; the caller commits and waits.
    """
    del library
    _lib.check(_lib.lib().cpq_affine_qmv(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), x.alloc_len, _ptr(y), len(y), in_vec_size, group_size, bits))


def affine_qmv_bf16(commands, library, w_q, scales, biases, x, y, in_vec_size, group_size, bits):
    """The reference's bf16-typed entry point (qmv.rs:77-88)."""
    for b in (scales, biases, x, y):
        if b.dtype != "bf16":
            raise TypeError("affine_qmv_bf16: scales, biases, x and y must be bf16 buffers")
    affine_qmv(commands, library, w_q, scales, biases, x, y, in_vec_size, group_size, bits)


def affine_qmv_batched(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                       x: Buffer, y: Buffer, in_vec_size: int, out_vec_size: int, group_size: int, bits: int,
                       batch_shape, w_strides, s_strides, b_strides, x_strides) -> None:
    """MLX's batched qmv (quantized.h:1496-1546 with batched=true): one activation
    row per batch element, W / scales / biases / x at element strides (0
    broadcasts); y holds out_vec_size values per element."""
    from .qmm import _batch_args

    del library
    nd, shape, (ws, ss, bs, xs) = _batch_args(batch_shape, w_strides, s_strides, b_strides, x_strides)
    _lib.check(_lib.lib().cpq_affine_qmv_batched(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(x), len(x), _ptr(y), len(y), out_vec_size, in_vec_size, group_size, bits,
        nd, shape, ws, ss, bs, xs))
