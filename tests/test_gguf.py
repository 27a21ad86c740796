"""GGUF reader (fl_gguf_*, flarellm_amd/csrc/gguf.cpp) on the CPU.

The header tests restate flare-loader/src/gguf.rs's own tests (983-1300):
magic, versions, metadata types, tensor infos, to_model_config with full /
default / missing / unsupported metadata.  The model tests write synthetic
models with flarellm_amd.gguf.write_gguf and read every tensor back: raw
bytes identical, RawWeight fields as read_raw_weight computes them
(gguf.rs:616-653), norms identical, tied output detected.
"""
import struct

import numpy as np
import pytest

from flarellm_amd import FL_F32, FL_Q4K, FL_Q6K, FL_Q8_0, FlareError
from flarellm_amd import synth as S
from flarellm_amd.gguf import GgufFile, write_gguf


def header(n_tensors, n_meta, version=3, magic=0x46554747):
    return struct.pack("<IIQQ", magic, version, n_tensors, n_meta)


def gstr(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def meta_u32(k, v):
    return gstr(k) + struct.pack("<II", 4, v)


def meta_str(k, v):
    return gstr(k) + struct.pack("<I", 8) + gstr(v)


def meta_f32(k, v):
    return gstr(k) + struct.pack("<If", 6, v)


def test_invalid_magic():
    with pytest.raises(FlareError, match="invalid GGUF magic"):
        GgufFile(data=header(0, 0, magic=0x12345678))


@pytest.mark.parametrize("v", [1, 4, 99])
def test_unsupported_version(v):
    with pytest.raises(FlareError, match=f"unsupported GGUF version: {v}"):
        GgufFile(data=header(0, 0, version=v))


@pytest.mark.parametrize("v", [2, 3])
def test_empty_file_and_alignment(v):
    g = GgufFile(data=header(0, 0, version=v))
    assert g.version == v and g.tensors() == []
    assert g.tensor_data_offset == 32  # 24-byte header rounded up to 32


def test_truncated():
    buf = header(1, 1) + gstr("general.architecture")
    with pytest.raises(FlareError, match="unexpected end"):
        GgufFile(data=buf)


def test_limits():
    with pytest.raises(FlareError, match="tensor count"):
        GgufFile(data=header(1_000_001, 0))
    with pytest.raises(FlareError, match="metadata count"):
        GgufFile(data=header(0, 100_001))
    with pytest.raises(FlareError, match="string length"):
        GgufFile(data=header(0, 1) + struct.pack("<Q", (1 << 20) + 1))


def test_metadata_types():
    body = b""
    vals = [(0, "<B", 7), (1, "<b", -7), (2, "<H", 700), (3, "<h", -700), (4, "<I", 70000), (5, "<i", -70000),
            (10, "<Q", 1 << 40), (11, "<q", -(1 << 40)), (7, "<B", 1)]
    for i, (t, f, v) in enumerate(vals):
        body += gstr(f"k{i}") + struct.pack("<I", t) + struct.pack(f, v)
    body += gstr("f32") + struct.pack("<If", 6, 1.5) + gstr("f64") + struct.pack("<Id", 12, 2.25)
    body += meta_str("s", "héllo")
    body += gstr("arr") + struct.pack("<IIQ", 9, 4, 3) + struct.pack("<3I", 1, 2, 3)
    body += gstr("sarr") + struct.pack("<IIQ", 9, 8, 2) + gstr("a") + gstr("bc")
    g = GgufFile(data=header(0, len(vals) + 5) + body)
    assert g.meta_u64("k0") == 7 and g.meta_u64("k2") == 700 and g.meta_u64("k4") == 70000
    assert g.meta_u64("k6") == 1 << 40 and g.meta_u64("k5") == (-70000) & ((1 << 64) - 1)
    with pytest.raises(FlareError):  # meta_usize does not take i8 / i16 / bool (gguf.rs:218-237)
        g.meta_u64("k1")
    with pytest.raises(FlareError):
        g.meta_u64("k8")
    assert g.meta_f32("f32") == 1.5 and g.meta_f32("f64") == 2.25
    assert g.meta_str("s") == "héllo" and g.meta_str("k0") is None and g.meta_str("missing") is None


def test_invalid_value_type():
    with pytest.raises(FlareError, match="invalid metadata value type: 13"):
        GgufFile(data=header(0, 1) + gstr("k") + struct.pack("<I", 13))
    with pytest.raises(FlareError, match="invalid metadata value type: 9"):  # nested arrays
        GgufFile(data=header(0, 1) + gstr("k") + struct.pack("<IIQ", 9, 9, 1))


def test_parse_tensor_info():
    """test_parse_tensor_info (gguf.rs:1159-1180)."""
    buf = header(1, 0) + gstr("blk.0.attn_q.weight") + struct.pack("<I2QIQ", 2, 4096, 4096, 0, 0)
    g = GgufFile(data=buf)
    (name, dims, typ, off, nb), = g.tensors()
    assert name == "blk.0.attn_q.weight" and dims == [4096, 4096] and typ == 0 and off == 0
    assert nb == 4096 * 4096 * 4
    assert g.find_tensor("blk.0.attn_q.weight") == 0 and g.find_tensor("nope") == -1


def _cfg_file(*metas, tensors=b"", n_tensors=0):
    return GgufFile(data=header(n_tensors, len(metas)) + b"".join(metas) + tensors)


def test_to_model_config_full():
    g = _cfg_file(meta_str("general.architecture", "LLaMA"), meta_u32("llama.embedding_length", 4096),
                  meta_u32("llama.block_count", 32), meta_u32("llama.attention.head_count", 32),
                  meta_u32("llama.attention.head_count_kv", 8), meta_u32("llama.feed_forward_length", 14336),
                  meta_u32("llama.context_length", 8192), meta_f32("llama.rope.freq_base", 500000.0),
                  meta_f32("llama.attention.layer_norm_rms_epsilon", 1e-6), meta_u32("llama.vocab_size", 1000),
                  tensors=gstr("token_embd.weight") + struct.pack("<I2QIQ", 2, 4096, 128256, 12, 0), n_tensors=1)
    cfg, arch = g.model_config()
    assert arch == 0
    assert (cfg.hidden_dim, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim) == (4096, 32, 32, 8, 128)
    assert (cfg.intermediate_dim, cfg.max_seq_len, cfg.vocab_size) == (14336, 8192, 128256)  # vocab from the embedding
    assert cfg.rope_theta == 500000.0 and cfg.rms_norm_eps == pytest.approx(1e-6)


def test_to_model_config_defaults():
    """test_to_model_config_defaults (gguf.rs:1111-1130)."""
    g = _cfg_file(meta_str("general.architecture", "llama"), meta_u32("llama.embedding_length", 128),
                  meta_u32("llama.block_count", 2), meta_u32("llama.attention.head_count", 4))
    cfg, _ = g.model_config()
    assert cfg.num_kv_heads == 4 and cfg.intermediate_dim == 512 and cfg.max_seq_len == 2048
    assert cfg.rope_theta == 10000.0 and cfg.rms_norm_eps == pytest.approx(1e-5) and cfg.vocab_size == 32000


def test_to_model_config_missing_required():
    """test_to_model_config_missing_required (gguf.rs:1132-1144)."""
    g = _cfg_file(meta_str("general.architecture", "llama"), meta_u32("llama.block_count", 2))
    with pytest.raises(FlareError, match="embedding_length"):
        g.model_config()


def test_to_model_config_unsupported_arch():
    """test_to_model_config_unsupported_arch (gguf.rs:1146-1157)."""
    g = _cfg_file(meta_str("general.architecture", "gpt_neox"))
    with pytest.raises(FlareError, match="gpt_neox"):
        g.model_config()


MODEL_SPECS = [
    S.tiny_spec(FL_Q8_0),
    S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K),
    S.tiny_spec(FL_Q8_0, output_fmt=FL_Q8_0, embed_fmt=FL_F32, norm_one=False),
]


@pytest.mark.parametrize("spec", MODEL_SPECS, ids=["q8_tied", "q4k_q6k", "q8_f32emb"])
def test_synthetic_model_round_trip(tmp_path, spec):
    model = S.make_model(spec, seed=3)
    path = str(tmp_path / "m.gguf")
    write_gguf(path, model)
    g = GgufFile(path)
    assert g.version == 3 and g.tensor_data_offset % 32 == 0
    assert g.meta_str("general.architecture") == "llama"
    cfg, arch = g.model_config()
    assert arch == 0
    assert (cfg.hidden_dim, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_dim,
            cfg.vocab_size, cfg.max_seq_len) == (spec.hidden, spec.layers, spec.heads, spec.kv_heads,
                                                 spec.head_dim, spec.inter, spec.vocab, spec.max_seq)
    names = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
    for i, ws in enumerate(model.layers):
        for n, w in zip(names, ws):
            data, fmt, rows, bpr = g.raw_weight(f"blk.{i}.{n}.weight")
            assert np.array_equal(data, w.data) and fmt == w.fmt and rows == w.rows
            assert bpr == S.blocks_per_row(w.fmt, w.cols)
        assert np.array_equal(g.tensor_f32(f"blk.{i}.attn_norm.weight", spec.hidden), model.attn_norms[i])
        assert np.array_equal(g.tensor_f32(f"blk.{i}.ffn_norm.weight", spec.hidden), model.ffn_norms[i])
    assert np.array_equal(g.tensor_f32("output_norm.weight", spec.hidden), model.output_norm)
    data, fmt, rows, _ = g.raw_weight("token_embd.weight")
    assert np.array_equal(data, model.embedding.data) and fmt == spec.embed_fmt and rows == spec.vocab
    assert (g.find_tensor("output.weight") >= 0) == (spec.output_fmt is not None)
    with pytest.raises(FlareError, match="tensor not found"):
        g.raw_weight("blk.99.attn_q.weight")
    g.close()


def test_f16_tensor_dequant(tmp_path):
    """A 1-D F16 tensor reads back as numpy's binary16 -> binary32 (subnormals,
    infinities and signed zeros included)."""
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    bits = bits[((bits & 0x7C00) != 0x7C00) | ((bits & 0x3FF) == 0)]  # drop NaNs
    n = bits.size
    buf = header(1, 0) + gstr("w") + struct.pack("<I1QIQ", 1, n, 1, 0)
    buf += b"\0" * ((-len(buf)) % 32) + bits.tobytes()
    g = GgufFile(data=buf)
    got = g.tensor_f32("w", n)
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _one_tensor(dims, typ, offset, payload=b""):
    buf = header(1, 0) + gstr("w") + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) + \
        struct.pack("<IQ", typ, offset)
    buf += b"\0" * (-len(buf) % 32)
    return GgufFile(data=buf + payload)


def test_crafted_offset_does_not_wrap():
    """A tensor offset near 2**64 must be rejected, not wrapped to a small
    start inside the file."""
    payload = bytes(34 * 4)
    g = _one_tensor([32, 4], 8, (1 << 64) - 64, payload)
    with pytest.raises(FlareError):
        g.raw_weight("w")
    # the same tensor at offset 0 reads back
    data, fmt, rows, bpr = _one_tensor([32, 4], 8, 0, payload).raw_weight("w")
    assert (fmt, rows, bpr) == (FL_Q8_0, 4, 1) and data.size == 34 * 4


def test_dims_overflow_rejected():
    """Dimensions whose product overflows 64 bits are rejected."""
    g = _one_tensor([1 << 40, 1 << 40], 8, 0, bytes(64))
    with pytest.raises(FlareError):
        g.raw_weight("w")
