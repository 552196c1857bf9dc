"""Model-level helpers over the runtime graph (crates/cider-press-models/src/nn.rs)."""
from __future__ import annotations

from .runtime import QuantizedWeight, Tensor


def embed_tokens(input_ids: Tensor, weight: QuantizedWeight) -> Tensor:
    """nn.rs:123-136: dequantized rows of a quantized [vocab, hidden] table for
    a rank-1 U32 ids tensor; a lazy [n_ids, hidden] tensor of the table's T."""
    return Tensor.embed_tokens(input_ids, weight)
