"""embed_tokens (crates/cider-press-models/src/nn.rs:123-136): the fused
gather + dequantize against the oracle's dequantize of the whole table
indexed by the ids (gather then dequantize, as the reference composes it).
Results must be bit-identical: the dequantize contract is bit-exact.

Argument validation runs on the CPU; the kernel tests are marked gpu.
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.synthetic import make_weight


def _check(dtype="bf16", w_q_len=896 * 100 // 8, s_len=14 * 100, b_len=14 * 100, n_ids=3, vocab=100, hidden=896,
           out_len=3 * 896, gs=64, bits=4):
    return _lib.lib().cpq_check_embed_args(_lib.DTYPES[dtype], w_q_len, s_len, b_len, n_ids, vocab, hidden,
                                           out_len, gs, bits)


def test_embed_args_validation():
    assert _check() == _lib.OK
    assert _check(n_ids=0, out_len=0) == _lib.OK
    for bad in (dict(w_q_len=1), dict(s_len=13 * 100), dict(b_len=0), dict(out_len=2 * 896),
                dict(hidden=900, w_q_len=450 * 100 // 4), dict(vocab=0), dict(bits=7), dict(gs=48),
                dict(dtype="u32")):
        assert _check(**bad) == _lib.INVALID_ARGUMENT, bad


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

def _run(device, library, w_q, s, b, ids, vocab, hidden, gs, bits, dtype):
    from cider_press_amd.kernels import embed as kembed

    W = device.upload(w_q.reshape(-1), "u32")
    S = device.upload(s.reshape(-1), dtype)
    B = device.upload(b.reshape(-1), dtype)
    I = device.upload(np.asarray(ids, np.uint32), "u32")
    O = device.alloc_buffer(len(ids) * hidden, dtype)
    cmds = device.commands()
    kembed.embed_tokens(cmds, library, W, S, B, I, O, vocab, hidden, gs, bits)
    return cmds, O


@pytest.mark.gpu
@pytest.mark.parametrize("vocab,hidden,gs,bits,dtype,n_ids", [
    (1000, 896, 64, 4, "bf16", 257),     # Qwen2 hidden, prefill-sized
    (300, 4096, 32, 4, "f16", 64),
    (128, 1024, 64, 8, "bf16", 33),
    (64, 512, 128, 3, "bf16", 17),       # odd width (3-bit packs)
    (50, 768, 32, 6, "f16", 5),
    (4000, 2048, 64, 4, "bf16", 1),      # decode
])
def test_embed_tokens_bit_exact(device, library, oracle, vocab, hidden, gs, bits, dtype, n_ids):
    rng = np.random.default_rng(vocab + hidden + bits)
    w_q, s, b = make_weight(rng, vocab, hidden, gs, bits, dtype, bias_noise=1e-3)
    ids = rng.integers(0, vocab, size=n_ids).astype(np.uint32)
    ids[: min(3, n_ids)] = [vocab - 1, 0, vocab - 1][: min(3, n_ids)]  # table ends, repeats
    cmds, O = _run(device, library, w_q, s, b, ids, vocab, hidden, gs, bits, dtype)
    cmds.commit_and_wait()
    got = O.to_numpy()[: n_ids * hidden].reshape(n_ids, hidden)
    table = oracle.dequantize(w_q, s, b, vocab, hidden, gs, bits, dtype)
    assert np.array_equal(got, table[ids])


@pytest.mark.gpu
def test_embed_tokens_out_of_range_ids(device, library, oracle):
    rng = np.random.default_rng(7)
    vocab, hidden = 200, 512
    w_q, s, b = make_weight(rng, vocab, hidden, 64, 4, "bf16")
    ids = np.array([5, vocab, 7, 0xFFFFFFFF, vocab - 1], np.uint32)
    cmds, O = _run(device, library, w_q, s, b, ids, vocab, hidden, 64, 4, "bf16")
    with pytest.raises(_lib.InvalidArgument, match="embed_tokens: 2 id"):
        cmds.commit_and_wait()
    got = O.to_numpy()[: len(ids) * hidden].reshape(len(ids), hidden)
    table = oracle.dequantize(w_q, s, b, vocab, hidden, 64, 4, "bf16")
    ok = np.array([0, 2, 4])
    assert np.array_equal(got[ok], table[ids[ok]])
    assert not got[[1, 3]].any()
    cmds.commit_and_wait()  # the status words were cleared by the failed wait


@pytest.mark.gpu
def test_embed_tokens_graph_node(device, oracle):
    from cider_press_amd import nn
    from cider_press_amd.runtime import QuantizedWeight, Tensor, q4_gs64

    rng = np.random.default_rng(11)
    vocab, hidden = 512, 896
    w_q, s, b = make_weight(rng, vocab, hidden, 64, 4, "bf16")
    w = QuantizedWeight.from_bytes(device, (vocab, hidden), q4_gs64(), w_q, s, b)
    ids = rng.integers(0, vocab, size=40).astype(np.uint32)
    x = Tensor.from_host(device, ids, "u32")
    e = nn.embed_tokens(x, w)
    assert e.shape() == (40, hidden)
    got = e.eval().cpu_slice()
    assert np.array_equal(got, oracle.dequantize(w_q, s, b, vocab, hidden, 64, 4, "bf16")[ids])
    # The embedding feeds the next op like any activation.
    y = e.quantized_matmul(w).eval().cpu_slice()
    assert y.shape == (40, vocab)
    with pytest.raises(_lib.InvalidArgument, match="rank-1"):
        nn.embed_tokens(Tensor.from_host(device, ids.reshape(4, 10), "u32"), w)
    with pytest.raises(_lib.InvalidArgument, match="U32"):
        nn.embed_tokens(Tensor.from_host(device, ids.astype(np.uint16), "bf16"), w)
