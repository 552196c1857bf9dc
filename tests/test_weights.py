"""On-disk format (MLX-style safetensors): the native archive parser, the
quantized-triple loader's checks, K padding and config.json quantization.

CPU only.  The parser is pinned against the `safetensors` package (an
independent implementation of the format) on the reference's committed
fixtures and on archives it writes; the loader's error behaviour follows
crates/cider-press-models/src/safetensors_io.rs:43-134 and its tests
(:284-318), the padding follows qwen2/weights.rs:316-376 and its tests
(:462-560), the config block follows qwen2/config.rs:65-73 and its pinned
config.json (:120-165).  Loader calls pass device=None: the archive is fully
checked before the device is touched, so a valid archive ends in
InvalidArgument("NULL device") here and uploads on a GPU box.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch
import safetensors.torch as stt

from cider_press_amd import _lib
from cider_press_amd import weights as W
from cider_press_amd.runtime import Quantization

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _torch_bytes(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().reshape(-1)
    if t.dtype == torch.uint32:
        t = t.view(torch.int32)
    return t.view(torch.uint8).numpy().reshape(-1) if t.numel() else np.zeros(0, np.uint8)


@pytest.mark.parametrize("name", ["qmv.safetensors", "qmm_qwen2.safetensors"])
def test_parser_matches_safetensors_package_on_reference_fixtures(name):
    path = os.path.join(GOLDEN, name)
    ref = stt.load_file(path)
    with W.SafeTensors.open(path) as st:
        assert st.names() == sorted(ref)
        for k, t in ref.items():
            v = st.tensor(k)
            assert v.shape == tuple(t.shape)
            assert v.dtype == {torch.bfloat16: "BF16", torch.uint32: "U32"}[t.dtype]
            np.testing.assert_array_equal(v.data, _torch_bytes(t))


def test_written_archives_round_trip(tmp_path):
    g = torch.Generator().manual_seed(0)
    tensors = {
        "model.layers.0.mlp.up_proj.weight": torch.randint(0, 2**31, (64, 16), generator=g).to(torch.int32)
        .view(torch.uint32),
        "a/ü-name": torch.randn(3, 5, generator=g).to(torch.bfloat16),
        "f16": torch.randn(7, generator=g).to(torch.float16),
        "f32": torch.randn(2, 2, 2, generator=g),
        "i64": torch.arange(5, dtype=torch.int64),
        "u8": torch.arange(11, dtype=torch.uint8),
        "bool": torch.tensor([True, False, True]),
        "empty": torch.zeros(0, 4, dtype=torch.bfloat16),
        "scalar": torch.tensor(3.5, dtype=torch.float64),
    }
    path = tmp_path / "a.safetensors"
    stt.save_file(tensors, str(path), metadata={"format": "mlx", "note": "x"})
    names = {torch.uint32: "U32", torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32",
             torch.int64: "I64", torch.uint8: "U8", torch.bool: "BOOL", torch.float64: "F64"}
    for st in (W.SafeTensors.open(path), W.SafeTensors.deserialize(path.read_bytes())):
        assert st.names() == sorted(tensors)
        assert st.metadata("format") == "mlx"
        with pytest.raises(_lib.MissingKey):
            st.metadata("absent")
        for k, t in tensors.items():
            v = st.tensor(k)
            assert v.dtype == names[t.dtype] and v.shape == tuple(t.shape)
            np.testing.assert_array_equal(v.data, _torch_bytes(t))
        with pytest.raises(_lib.MissingKey):
            st.tensor("absent")
        st.close()


def _archive(header: dict, buffer: bytes, pad: int = 0) -> bytes:
    h = json.dumps(header).encode() + b" " * pad
    return struct.pack("<Q", len(h)) + h + buffer


@pytest.mark.parametrize("blob", [
    b"",                                                                 # no length
    b"\x05\x00\x00",                                                     # short length
    struct.pack("<Q", 100) + b"{}",                                      # header past the end
    struct.pack("<Q", 3) + b"{x}",                                       # not JSON
    struct.pack("<Q", 2) + b"[]",                                        # not an object
    _archive({"a": {"dtype": "Q4", "shape": [1], "data_offsets": [0, 1]}}, b"\0"),      # unknown dtype
    _archive({"a": {"dtype": "U32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4),  # 4 bytes for 8
    _archive({"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}, b"\0" * 3),   # past the buffer
    _archive({"a": {"dtype": "U8", "shape": [2], "data_offsets": [2, 4]}}, b"\0" * 4),   # gap at the start
    _archive({"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]},
              "b": {"dtype": "U8", "shape": [2], "data_offsets": [1, 3]}}, b"\0" * 3),  # overlap
    _archive({"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}}, b"\0" * 3),   # trailing bytes
    _archive({"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 0]}}, b""),       # negative dim
    _archive({"a": {"dtype": "U8", "shape": [1.5], "data_offsets": [0, 1]}}, b"\0"),    # fractional dim
    _archive({"a": {"dtype": "U8", "shape": [1]}}, b"\0"),                               # no offsets
    _archive({"__metadata__": {"k": 1}}, b""),                                           # non-string metadata
])
def test_malformed_archives_are_rejected(blob):
    with pytest.raises(_lib.SafetensorsError):
        W.SafeTensors.deserialize(blob)


def test_header_padding_and_empty_archive():
    st = W.SafeTensors.deserialize(_archive({"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}},
                                            b"\x07\x09", pad=6))
    np.testing.assert_array_equal(st.tensor("a").data, [7, 9])
    assert W.SafeTensors.deserialize(_archive({}, b"")).names() == []


def test_open_missing_file_is_a_safetensors_error(tmp_path):
    with pytest.raises(_lib.SafetensorsError):
        W.SafeTensors.open(tmp_path / "absent.safetensors")


# ---------------------------------------------------------------------------
# The quantized triple (safetensors_io.rs:43-134)
# ---------------------------------------------------------------------------

def _triple(base="ln", n=64, k=128, bits=4, gs=64, sdt=torch.bfloat16, bdt=None, wdt=torch.uint32,
            wshape=None, sshape=None, bshape=None, drop=()):
    """Synthetic triple like the reference's synthetic_q4_gs64_entries (:256-282)."""
    pk, groups = k * bits // 32, k // gs
    w = (torch.arange(n * pk * 4) & 0xFF).to(torch.uint8).view(torch.int32).reshape(n, pk)
    s = ((torch.arange(n * groups * 2) * 3) & 0xFF).to(torch.uint8).view(torch.int16).reshape(n, groups)
    b = ((torch.arange(n * groups * 2) * 7) & 0xFF).to(torch.uint8).view(torch.int16).reshape(n, groups)
    ents = {
        f"{base}.weight": w.view(torch.uint32) if wdt == torch.uint32 else w.view(torch.float32),
        f"{base}.scales": s.view(sdt) if sdt != torch.float32 else s.reshape(-1)[: n * groups // 2].view(torch.float32),
        f"{base}.biases": b.view(bdt or sdt) if (bdt or sdt) != torch.float32 else b.reshape(-1)[: n * groups // 2]
        .view(torch.float32),
    }
    if wshape:
        ents[f"{base}.weight"] = ents[f"{base}.weight"].reshape(wshape)
    if sshape:
        ents[f"{base}.scales"] = ents[f"{base}.scales"].reshape(sshape)
    if bshape:
        ents[f"{base}.biases"] = ents[f"{base}.biases"].reshape(bshape)
    for d in drop:
        del ents[f"{base}.{d}"]
    return W.SafeTensors.deserialize(stt.save(ents))


def q(bits=4, gs=64):
    return Quantization(bits, gs)


def test_valid_triple_reaches_the_device_step():
    st = _triple()
    with pytest.raises(_lib.InvalidArgument, match="NULL device"):
        W.read_quantized_weight(st, "ln", q(), None)
    with pytest.raises(_lib.InvalidArgument, match="NULL device"):
        W.read_quantized_weight_k_padded(st, "ln", q(), None, 192)


@pytest.mark.parametrize("drop,key", [(("weight",), "ln.weight"), (("scales", "biases"), "ln.scales"),
                                      (("biases",), "ln.biases")])
def test_missing_component(drop, key):
    with pytest.raises(_lib.MissingKey, match=key.replace(".", r"\.")):
        W.read_quantized_weight(_triple(drop=drop), "ln", q(), None)


def test_unsupported_dtypes():
    with pytest.raises(_lib.UnsupportedDtype, match="ln.weight"):
        W.read_quantized_weight(_triple(wdt=torch.float32), "ln", q(), None)
    with pytest.raises(_lib.UnsupportedDtype, match="ln.scales"):
        W.read_quantized_weight(_triple(sdt=torch.float32), "ln", q(), None)
    with pytest.raises(_lib.UnsupportedDtype, match="ln.biases"):
        W.read_quantized_weight(_triple(sdt=torch.bfloat16, bdt=torch.float16), "ln", q(), None)
    # F16 scales and biases together are accepted (the kernels run f16 too).
    with pytest.raises(_lib.InvalidArgument, match="NULL device"):
        W.read_quantized_weight(_triple(sdt=torch.float16), "ln", q(), None)


def test_wrong_aux_shape_is_a_shape_mismatch():
    # The reference's read_quantized_weight_wrong_aux_shape_errors (:300-317):
    # [64, 2] scales presented as [128, 1].
    with pytest.raises(_lib.ShapeMismatch, match=r"ln\.scales.*\[64, 2\].*\[128, 1\]"):
        W.read_quantized_weight(_triple(sshape=(128, 1)), "ln", q(), None)
    with pytest.raises(_lib.ShapeMismatch, match=r"ln\.biases"):
        W.read_quantized_weight(_triple(bshape=(32, 4)), "ln", q(), None)


def test_weight_geometry_checks():
    with pytest.raises(_lib.InvalidArgument, match="rank-2"):
        W.read_quantized_weight(_triple(wshape=(64, 4, 4)), "ln", q(), None)
    # 3-bit: one packed word per row is 32 bits, not a multiple of 3.
    st = W.SafeTensors.deserialize(stt.save({
        "t.weight": torch.zeros(4, 1, dtype=torch.int32).view(torch.uint32),
        "t.scales": torch.zeros(4, 1, dtype=torch.bfloat16), "t.biases": torch.zeros(4, 1, dtype=torch.bfloat16)}))
    with pytest.raises(_lib.InvalidArgument, match="not divisible by bits"):
        W.read_quantized_weight(st, "t", q(3, 32), None)
    # 4-bit, 4 words -> K = 32, not a multiple of gs = 64.
    st = W.SafeTensors.deserialize(stt.save({
        "t.weight": torch.zeros(4, 4, dtype=torch.int32).view(torch.uint32),
        "t.scales": torch.zeros(4, 1, dtype=torch.bfloat16), "t.biases": torch.zeros(4, 1, dtype=torch.bfloat16)}))
    with pytest.raises(_lib.InvalidArgument, match="not divisible by group_size"):
        W.read_quantized_weight(st, "t", q(4, 64), None)


def test_k_pad_must_cover_k_and_align():
    st = _triple()
    for bad in (64, 160):
        with pytest.raises(_lib.InvalidArgument, match="k_pad"):
            W.read_quantized_weight_k_padded(st, "ln", q(), None, bad)


def test_dense_tensor_dtypes():
    st = W.SafeTensors.deserialize(stt.save({"g": torch.ones(8, dtype=torch.bfloat16),
                                             "f": torch.ones(2), "h": torch.ones(3, dtype=torch.float16)}))
    with pytest.raises(_lib.UnsupportedDtype, match='"f"'):
        W.read_dense_tensor(st, "f", None)
    with pytest.raises(_lib.MissingKey):
        W.read_dense_tensor(st, "absent", None)
    for key in ("g", "h"):
        with pytest.raises(_lib.InvalidArgument, match="NULL device"):
            W.read_dense_tensor(st, key, None)


# ---------------------------------------------------------------------------
# pad_quantized_k (qwen2/weights.rs:316-376; tests :462-560)
# ---------------------------------------------------------------------------

def test_pad_quantized_k_row_strides():
    w, s, b = W.pad_quantized_k(b"\xff" * (2 * 64), b"\xee" * (2 * 4), b"\xdd" * (2 * 4), 2, 128, 192, q())
    assert (len(w), len(s), len(b)) == (2 * 96, 2 * 6, 2 * 6)


def test_pad_quantized_k_preserves_bytes_and_zeroes_pad():
    n = 3
    w_src = bytes(((i + 1) & 0xFF) for i in range(n * 64))
    s_src = bytes(((i + 0x40) & 0xFF) for i in range(n * 4))
    b_src = bytes(((i + 0x80) & 0xFF) for i in range(n * 4))
    w, s, b = W.pad_quantized_k(w_src, s_src, b_src, n, 128, 192, q())
    for r in range(n):
        assert w[r * 96:r * 96 + 64] == w_src[r * 64:(r + 1) * 64]
        assert s[r * 6:r * 6 + 4] == s_src[r * 4:(r + 1) * 4]
        assert b[r * 6:r * 6 + 4] == b_src[r * 4:(r + 1) * 4]
        assert w[r * 96 + 64:r * 96 + 96] == bytes(32)
        assert s[r * 6 + 4:r * 6 + 6] == bytes(2) and b[r * 6 + 4:r * 6 + 6] == bytes(2)


def test_pad_quantized_k_no_op_and_8_bit():
    w_src, s_src, b_src = b"\xaa" * 128, b"\xbb" * 8, b"\xcc" * 8
    assert W.pad_quantized_k(w_src, s_src, b_src, 2, 128, 128, q()) == (w_src, s_src, b_src)
    # 8-bit gs32: K=64 -> 96, rows 64 -> 96 bytes, 2 -> 3 groups.
    w, s, b = W.pad_quantized_k(bytes(range(128)), b"\x01" * 8, b"\x02" * 8, 2, 64, 96, q(8, 32))
    assert w == bytes(range(64)) + bytes(32) + bytes(range(64, 128)) + bytes(32)
    assert s == b"\x01" * 4 + bytes(2) + b"\x01" * 4 + bytes(2)


@pytest.mark.parametrize("k,k_pad,msg", [(96, 128, "k=96"), (128, 64, "k_pad=64"), (128, 160, "k_pad=160")])
def test_pad_quantized_k_preconditions(k, k_pad, msg):
    with pytest.raises(_lib.InvalidArgument, match=msg):
        W.pad_quantized_k(b"\0" * (k // 2), b"\0" * 4, b"\0" * 4, 1, k, k_pad, q())


# ---------------------------------------------------------------------------
# config.json quantization (qwen2/config.rs:65-73, :120-165)
# ---------------------------------------------------------------------------

PINNED_CONFIG = """{
    "architectures": ["Qwen2ForCausalLM"], "attention_dropout": 0.0, "bos_token_id": 151643,
    "eos_token_id": 151645, "hidden_act": "silu", "hidden_size": 896, "initializer_range": 0.02,
    "intermediate_size": 4864, "max_position_embeddings": 32768, "max_window_layers": 21,
    "model_type": "qwen2", "num_attention_heads": 14, "num_hidden_layers": 24, "num_key_value_heads": 2,
    "quantization": { "group_size": 64, "bits": 4 }, "rms_norm_eps": 1e-06, "rope_theta": 1000000.0,
    "sliding_window": 32768, "tie_word_embeddings": true, "torch_dtype": "bfloat16",
    "transformers_version": "4.43.1", "use_cache": true, "use_sliding_window": false, "vocab_size": 151936
}"""


def test_pinned_config_quantization(tmp_path):
    assert W.quantization_from_config(PINNED_CONFIG) == Quantization(4, 64)
    p = tmp_path / "config.json"
    p.write_text(PINNED_CONFIG)
    assert W.derive_quantization(p) == Quantization(4, 64)
    assert W.quantization_from_config(PINNED_CONFIG.encode()) == Quantization(4, 64)


def test_config_without_quantization():
    for cfg in ('{"hidden_size": 896}', '{"quantization": null, "x": [1, {"y": "\\u00fc"}]}'):
        assert W.quantization_from_config(cfg) is None
        with pytest.raises(_lib.InvalidArgument, match="pre-quantized"):
            W.derive_quantization(cfg)


@pytest.mark.parametrize("cfg", [
    '{"quantization": {"bits": 4}}',                      # missing group_size
    '{"quantization": {"group_size": 64}}',               # missing bits
    '{"quantization": {"group_size": 64, "bits": 4.5}}',  # not an integer
    '{"quantization": {"group_size": 64, "bits": 300}}',  # not a u8
    '{"quantization": {"group_size": -64, "bits": 4}}',   # not a u32
    '{"quantization": [64, 4]}',
    '{"quantization": {"group_size": 64, "bits": 4}',     # truncated
    '{"a": 1,}',                                          # trailing comma
    '["not an object"]',
])
def test_malformed_config_is_a_json_error(cfg):
    with pytest.raises(_lib.JsonError):
        W.quantization_from_config(cfg)


def test_unsupported_quantization_is_rejected():
    with pytest.raises(_lib.InvalidArgument):
        W.derive_quantization('{"quantization": {"group_size": 64, "bits": 7}}')
