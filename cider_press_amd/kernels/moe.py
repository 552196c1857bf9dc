"""Routed experts around gather_qmm: router top-k, the sort of (token, slot)
rows by expert that gather_qmm's sorted form takes, and the weighted combine.

No reference counterpart: the reference names this as its unbuilt MoE
feature (docs/inference/feed-forward.md:98-107, 131-137).  Semantics are
stated in include/cpq.h (cpq_moe_route, cpq_moe_combine).
"""
from __future__ import annotations

from .. import _lib
from . import Buffer, Commands, _ptr


def moe_route(commands: Commands, logits: Buffer, tokens: int, n_experts: int, top_k: int, normalize: bool,
              experts: Buffer, scores: Buffer, lhs: Buffer, rhs: Buffer, inv: Buffer, offsets: Buffer) -> None:
    """Softmax top-k per token, then the stable sort of the tokens*top_k rows
    by expert.  experts/lhs/rhs/inv: u32 [tokens*top_k]; scores: f32
    [tokens*top_k]; offsets: u32 [n_experts + 1].  Encodes only."""
    for b, dt in ((experts, "u32"), (scores, "f32"), (lhs, "u32"), (rhs, "u32"), (inv, "u32"), (offsets, "u32")):
        if b.dtype != dt:
            raise TypeError(f"moe_route: expected a {dt} buffer, got {b.dtype}")
    rows = tokens * top_k
    for b in (experts, scores, lhs, rhs, inv):
        if len(b) < rows:
            raise _lib.InvalidArgument("moe_route: an output buffer is shorter than tokens*top_k")
    if len(offsets) < n_experts + 1 or len(logits) < tokens * n_experts:
        raise _lib.InvalidArgument("moe_route: offsets or logits buffer too short")
    _lib.check(_lib.lib().cpq_moe_route(
        commands.handle, _lib.DTYPES[logits.dtype], _ptr(logits), tokens, n_experts, top_k, int(bool(normalize)),
        _ptr(experts), _ptr(scores), _ptr(lhs), _ptr(rhs), _ptr(inv), _ptr(offsets)))


def moe_combine(commands: Commands, y: Buffer, scores: Buffer, inv: Buffer, tokens: int, top_k: int, n: int,
                out: Buffer) -> None:
    """out[t, :] = sum_j scores[t*k + j] * y[inv[t*k + j], :] (fp32, rounded to
    T); y holds the expert outputs in sorted row order.  Encodes only."""
    if scores.dtype != "f32" or inv.dtype != "u32":
        raise TypeError("moe_combine: scores must be f32 and inv u32 buffers")
    if len(scores) < tokens * top_k or len(inv) < tokens * top_k:
        raise _lib.InvalidArgument("moe_combine: scores or inv shorter than tokens*top_k")
    _lib.check(_lib.lib().cpq_moe_combine(
        commands.handle, _lib.DTYPES[y.dtype], _ptr(y), len(y), _ptr(scores), _ptr(inv), tokens, top_k, n,
        _ptr(out), len(out)))
