"""Quantized embedding lookup (crates/cider-press-models/src/nn.rs:123-136).

The reference gathers the table's packed words, scales and biases by token
id (Tensor::gather, runtime/src/tensor.rs:1444-1530) and dequantizes the
gathered triple (dequantize.rs:58-137); `embed_tokens` here is one fused
kernel with the same result bits.
"""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, KernelLibrary, _ptr


def embed_tokens(commands: Commands, library: KernelLibrary, w_q: Buffer, scales: Buffer, biases: Buffer,
                 ids: Buffer, out: Buffer, vocab: int, hidden: int, group_size: int, bits: int) -> None:
    """out[t, :] = RNE_T(fmaf(s, q, b)) over row ids[t] of the [vocab, hidden]
    table; out.len() == len(ids) * hidden.  Ids at or past vocab give zero
    rows and make the next wait raise InvalidArgument.  Encodes only."""
    del library
    if ids.dtype != "u32":
        raise TypeError("embed_tokens: ids must be a u32 buffer")
    _lib.check(_lib.lib().cpq_embed_tokens(
        commands.handle, _lib.DTYPES[scales.dtype], _ptr(w_q), len(w_q), _ptr(scales), len(scales),
        _ptr(biases), len(biases), _ptr(ids), len(ids), vocab, hidden, _ptr(out), len(out), group_size, bits))
