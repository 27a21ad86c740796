"""Seeded synthetic Llama-shaped models in GGUF block layout.

The benchmark configurations (Llama-3.2-1B Q8_0, Llama-3-8B Q4_K/Q6_K,
SmolLM2-135M Q8_0) are rebuilt offline from random N(0, 0.02) weights, since
no real checkpoint is available.  Weights are generated and block-quantized
by the library's host code (fl_synth_normal / fl_synth_quantize) and are laid
out exactly as GGUF tensors: rows = out features, row-major blocks
(flare-loader/src/gguf.rs:616-653).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field, replace

import numpy as np

from . import _lib
from ._lib import FL_F32, FL_Q4K, FL_Q6K, FL_Q8_0


@dataclass(frozen=True)
class ModelSpec:
    name: str
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    max_seq: int
    layer_fmt: int
    embed_fmt: int
    output_fmt: int | None  # None = tied to the embedding
    eps: float = 1e-5
    theta: float = 10000.0
    std: float = 0.02
    norm_one: bool = True  # norms exactly 1.0 (configs) or N(1, 0.1)

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    def layer_shapes(self):
        """(rows, cols) of wq, wk, wv, wo, w_gate, w_up, w_down."""
        H, F = self.hidden, self.inter
        return [(self.q_dim, H), (self.kv_dim, H), (self.kv_dim, H), (H, self.q_dim), (F, H), (F, H), (H, F)]

    def weight_bytes_per_token(self) -> int:
        """Algorithmic weight bytes streamed per decoded token."""
        lib = _lib.load()
        total = 0
        for r, c in self.layer_shapes():
            total += r * lib.fl_format_row_bytes(self.layer_fmt, c)
        total *= self.layers
        out_fmt = self.embed_fmt if self.output_fmt is None else self.output_fmt
        total += self.vocab * lib.fl_format_row_bytes(out_fmt, self.hidden)
        return total


# BASELINE.json configs
SMOLLM2_135M = ModelSpec("SmolLM2-135M", 576, 30, 9, 3, 64, 1536, 49152, 256,
                         FL_Q8_0, FL_Q8_0, None, theta=100000.0)
LLAMA32_1B = ModelSpec("Llama-3.2-1B", 2048, 16, 32, 8, 64, 8192, 128256, 2048,
                       FL_Q8_0, FL_Q8_0, None, theta=500000.0)
LLAMA3_8B = ModelSpec("Llama-3-8B", 4096, 32, 32, 8, 128, 14336, 128256, 4352,
                      FL_Q4K, FL_Q6K, FL_Q6K, theta=500000.0)
CONFIGS = {s.name: s for s in (SMOLLM2_135M, LLAMA32_1B, LLAMA3_8B)}


def tiny_spec(layer_fmt=FL_Q8_0, embed_fmt=None, output_fmt=None, **kw) -> ModelSpec:
    """Small model for parity tests (oracle finishes in well under a second)."""
    base = dict(name="tiny", hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512,
                vocab=512, max_seq=96, layer_fmt=layer_fmt,
                embed_fmt=layer_fmt if embed_fmt is None else embed_fmt,
                output_fmt=output_fmt, norm_one=False)
    base.update(kw)
    return ModelSpec(**base)


def blocks_per_row(fmt: int, cols: int) -> int:
    return {FL_F32: cols, FL_Q8_0: cols // 32, FL_Q4K: cols // 256, FL_Q6K: cols // 256}[fmt]


def normal(seed: int, offset: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.load().fl_synth_normal(seed, offset, n, mean, std, out.ctypes.data)
    return out


def quantize(w: np.ndarray, fmt: int) -> np.ndarray:
    """Quantize an f32 [rows, cols] array into GGUF block bytes."""
    lib = _lib.load()
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    rb = lib.fl_format_row_bytes(fmt, cols)
    if rb == 0:
        raise ValueError(f"cols={cols} incompatible with format {fmt}")
    out = np.empty(rows * rb, dtype=np.uint8)
    n = lib.fl_synth_quantize(w.ctypes.data, rows, cols, fmt, out.ctypes.data)
    assert n == out.size
    return out


@dataclass
class QWeight:
    data: np.ndarray  # uint8 GGUF bytes
    fmt: int
    rows: int
    cols: int

    def raw(self) -> _lib.RawWeight:
        return _lib.RawWeight(self.data.ctypes.data, self.data.size, self.fmt, self.rows,
                              blocks_per_row(self.fmt, self.cols))


@dataclass
class SynthModel:
    spec: ModelSpec
    layers: list = field(default_factory=list)  # per layer: list of 7 QWeight
    attn_norms: list = field(default_factory=list)
    ffn_norms: list = field(default_factory=list)
    output_norm: np.ndarray | None = None
    embedding: QWeight | None = None
    output: QWeight | None = None


def _qweight(seed: int, stream: int, rows: int, cols: int, fmt: int, std: float) -> QWeight:
    w = normal(seed, stream << 40, rows * cols, 0.0, std).reshape(rows, cols)
    return QWeight(quantize(w, fmt), fmt, rows, cols)


def make_model(spec: ModelSpec, seed: int = 0) -> SynthModel:
    """Random N(0, std) weights quantized to the spec's formats."""
    m = SynthModel(spec)
    stream = 1
    for _ in range(spec.layers):
        ws = []
        for rows, cols in spec.layer_shapes():
            ws.append(_qweight(seed, stream, rows, cols, spec.layer_fmt, spec.std))
            stream += 1
        m.layers.append(ws)
        if spec.norm_one:
            m.attn_norms.append(np.ones(spec.hidden, np.float32))
            m.ffn_norms.append(np.ones(spec.hidden, np.float32))
        else:
            m.attn_norms.append(normal(seed, stream << 40, spec.hidden, 1.0, 0.1))
            m.ffn_norms.append(normal(seed, (stream + 1) << 40, spec.hidden, 1.0, 0.1))
        stream += 2
    m.output_norm = (np.ones(spec.hidden, np.float32) if spec.norm_one
                     else normal(seed, stream << 40, spec.hidden, 1.0, 0.1))
    stream += 1
    m.embedding = _qweight(seed, stream, spec.vocab, spec.hidden, spec.embed_fmt, spec.std)
    stream += 1
    if spec.output_fmt is not None:
        m.output = _qweight(seed, stream, spec.vocab, spec.hidden, spec.output_fmt, spec.std)
    return m


def random_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    """Uniform-random prompt tokens in [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.uint32)


__all__ = ["ModelSpec", "SynthModel", "QWeight", "CONFIGS", "SMOLLM2_135M", "LLAMA32_1B", "LLAMA3_8B",
           "tiny_spec", "make_model", "quantize", "normal", "random_tokens", "blocks_per_row", "replace"]
