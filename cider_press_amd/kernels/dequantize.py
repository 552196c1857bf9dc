"""Affine dequantize (crates/cider-press-kernels/src/kernels/dequantize.rs:58-137)."""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, KernelLibrary, _ptr

BITS = 4
GROUP_SIZE = 64


def affine_dequantize(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                      out: Buffer, group_size: int, bits: int) -> None:
    """out[i] = RNE_T(fmaf(scale, q_i, bias)); out.len() elements. Encodes only."""
    del library
    _lib.check(_lib.lib().cpq_affine_dequantize(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(out), len(out), group_size, bits))


def affine_dequantize_bf16_gs64_b4(commands, library, w_q, scales, biases, out):
    """The reference's entry point (dequantize.rs:58-65): bf16, group_size 64, 4-bit."""
    for b in (scales, biases, out):
        if b.dtype != "bf16":
            raise TypeError("affine_dequantize_bf16_gs64_b4: scales, biases and out must be bf16 buffers")
    affine_dequantize(commands, library, w_q, scales, biases, out, GROUP_SIZE, BITS)
