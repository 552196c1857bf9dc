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
