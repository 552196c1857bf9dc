"""Routed-expert quantized matmul.

The reference has no wired dispatcher for this op; its semantics come from the
vendored MSL affine_gather_qmm_t / affine_gather_qmm_rhs
(kernels-mlx/mlx/backend/metal/kernels/quantized.h:2092-2172, 2242-2436), with
the bind order x, w, scales, biases, indices, y, M, N, K of the rhs variant.
"""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, KernelLibrary, _ptr


def affine_gather_qmm(commands: Commands, library: KernelLibrary, x: Buffer, w_q: Buffer, scales: Buffer,
                      biases: Buffer, lhs_indices, rhs_indices: Buffer, y: Buffer, n_rows: int, n: int, k: int,
                      n_experts: int, group_size: int, bits: int, sorted_indices: bool = False,
                      x_rows=None) -> None:
    """Y[r] = X[lhs[r]] . dequant(W[rhs[r]])^T for r < n_rows. Encodes only.

    W holds `n_experts` [N, K] matrices back to back.  `lhs_indices` may be
    None (row r reads X row r).  Out-of-range indices zero their row and are
    reported by the next wait as InvalidArgument.
    """
    del library
    if x_rows is None:
        x_rows = len(x) // k
    _lib.check(_lib.lib().cpq_affine_gather_qmm(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(x), x_rows, _ptr(w_q), len(w_q), _ptr(scales),
        len(scales), _ptr(biases), len(biases), _ptr(lhs_indices), _ptr(rhs_indices), n_rows, _ptr(y), len(y),
        n_experts, n, k, group_size, bits, int(bool(sorted_indices))))


def affine_gather_qmm_bf16(commands, library, x, w_q, scales, biases, lhs_indices, rhs_indices, y, n_rows, n, k,
                           n_experts, group_size, bits, sorted_indices=False):
    for b in (x, scales, biases, y):
        if b.dtype != "bf16":
            raise TypeError("affine_gather_qmm_bf16: x, scales, biases and y must be bf16 buffers")
    affine_gather_qmm(commands, library, x, w_q, scales, biases, lhs_indices, rhs_indices, y, n_rows, n, k,
                      n_experts, group_size, bits, sorted_indices)
