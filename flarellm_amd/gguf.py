"""GGUF files: a writer for synthetic models and the ctypes mirror of the
library's reader (fl_gguf_*, flarellm_amd/csrc/gguf.cpp).

The writer lays a SynthModel out as llama.cpp / flarellm name it
(flare-loader/src/weights.rs:30-66; blk.N.attn_q.weight ...), with GGUF v3
framing (gguf.rs:131-204): little-endian header, metadata, tensor infos with
dimensions in [cols, rows] order, tensor data at a 32-byte boundary and every
tensor offset a multiple of 32.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import _lib
from ._lib import FL_F32, FL_Q4K, FL_Q6K, FL_Q8_0, ModelConfig, RawWeight, check

GGUF_MAGIC = 0x46554747
ALIGN = 32
# ggml type ids (flare-loader/src/quantize.rs:32-60)
GGML_TYPE = {FL_F32: 0, FL_Q8_0: 8, FL_Q4K: 12, FL_Q6K: 14}
T_U32, T_F32, T_STR, T_ARR, T_U64 = 4, 6, 8, 9, 10


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _meta(key: str, typ: int, val) -> bytes:
    out = _str(key) + struct.pack("<I", typ)
    if typ == T_U32:
        return out + struct.pack("<I", val)
    if typ == T_U64:
        return out + struct.pack("<Q", val)
    if typ == T_F32:
        return out + struct.pack("<f", val)
    if typ == T_STR:
        return out + _str(val)
    if typ == T_ARR:  # (element type, values)
        et, vals = val
        body = struct.pack("<IQ", et, len(vals))
        for v in vals:
            body += _str(v) if et == T_STR else struct.pack("<I" if et == T_U32 else "<f", v)
        return out + body
    raise ValueError(typ)


def model_tensors(model):
    """(name, GGUF dims [cols, rows], ggml type, bytes) of a SynthModel."""
    spec = model.spec
    names = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
    out = [("token_embd.weight", [spec.hidden, spec.vocab], GGML_TYPE[model.embedding.fmt], model.embedding.data)]
    for i, ws in enumerate(model.layers):
        out.append((f"blk.{i}.attn_norm.weight", [spec.hidden], 0, model.attn_norms[i].view(np.uint8)))
        for n, w in zip(names, ws):
            out.append((f"blk.{i}.{n}.weight", [w.cols, w.rows], GGML_TYPE[w.fmt], w.data))
        out.append((f"blk.{i}.ffn_norm.weight", [spec.hidden], 0, model.ffn_norms[i].view(np.uint8)))
    out.append(("output_norm.weight", [spec.hidden], 0, model.output_norm.view(np.uint8)))
    if model.output is not None:
        out.append(("output.weight", [spec.hidden, spec.vocab], GGML_TYPE[model.output.fmt], model.output.data))
    return out


def write_gguf(path: str, model, context_length: int | None = None, extra_meta=()) -> None:
    """Write a SynthModel as a llama-architecture GGUF v3 file."""
    spec = model.spec
    meta = [
        ("general.architecture", T_STR, "llama"),
        ("general.name", T_STR, spec.name),
        ("general.alignment", T_U32, ALIGN),
        ("llama.context_length", T_U32, context_length or spec.max_seq),
        ("llama.embedding_length", T_U32, spec.hidden),
        ("llama.block_count", T_U32, spec.layers),
        ("llama.feed_forward_length", T_U32, spec.inter),
        ("llama.attention.head_count", T_U32, spec.heads),
        ("llama.attention.head_count_kv", T_U32, spec.kv_heads),
        ("llama.rope.freq_base", T_F32, spec.theta),
        ("llama.attention.layer_norm_rms_epsilon", T_F32, spec.eps),
        ("tokenizer.ggml.tokens", T_ARR, (T_STR, [f"<t{i}>" for i in range(4)])),
        *extra_meta,
    ]
    tensors = model_tensors(model)
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta))
    head += b"".join(_meta(k, t, v) for k, t, v in meta)
    offsets, off = [], 0
    for name, dims, typ, data in tensors:
        offsets.append(off)
        off += (data.nbytes + ALIGN - 1) // ALIGN * ALIGN
    for (name, dims, typ, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", typ, o)
    pad = (-len(head)) % ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, typ, data), o in zip(tensors, offsets):
            f.write(np.ascontiguousarray(data).tobytes())
            f.write(b"\0" * ((-data.nbytes) % ALIGN))


class GgufFile:
    """flarellm GgufFile (gguf.rs) over the library's memory-mapped reader."""

    def __init__(self, path: str | None = None, data: bytes | None = None):
        self.lib = _lib.load()
        h = C.c_void_p()
        if path is not None:
            check(self.lib.fl_gguf_open(path.encode(), C.byref(h)))
        else:
            buf = C.create_string_buffer(bytes(data), len(data))
            check(self.lib.fl_gguf_open_memory(buf, len(data), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.fl_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self) -> int:
        return self.lib.fl_gguf_version(self.h)

    @property
    def tensor_data_offset(self) -> int:
        return self.lib.fl_gguf_data_offset(self.h)

    def tensors(self):
        out = []
        for i in range(self.lib.fl_gguf_tensor_count(self.h)):
            name = C.c_char_p()
            nd = C.c_int()
            dims = (C.c_uint64 * 8)()
            typ = C.c_uint32()
            off = C.c_uint64()
            nb = C.c_uint64()
            check(self.lib.fl_gguf_tensor_info(self.h, i, C.byref(name), C.byref(nd), dims, C.byref(typ),
                                               C.byref(off), C.byref(nb)))
            out.append((name.value.decode(), list(dims[:nd.value]), typ.value, off.value, nb.value))
        return out

    def find_tensor(self, name: str) -> int:
        return self.lib.fl_gguf_find_tensor(self.h, name.encode())

    def meta_u64(self, key: str) -> int:
        v = C.c_uint64()
        check(self.lib.fl_gguf_meta_u64(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f32(self, key: str) -> float:
        v = C.c_float()
        check(self.lib.fl_gguf_meta_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key: str):
        v = self.lib.fl_gguf_meta_str(self.h, key.encode())
        return None if v is None else v.decode()

    def model_config(self):
        cfg = ModelConfig()
        arch = C.c_int()
        check(self.lib.fl_gguf_model_config(self.h, C.byref(cfg), C.byref(arch)))
        return cfg, arch.value

    def raw_weight(self, name: str):
        """read_raw_weight: (bytes, format, num_rows, blocks_per_row)."""
        rw = RawWeight()
        check(self.lib.fl_gguf_raw_weight(self.h, name.encode(), C.byref(rw)))
        data = np.ctypeslib.as_array(C.cast(rw.data, C.POINTER(C.c_uint8)), shape=(rw.nbytes,)).copy()
        return data, rw.format, rw.num_rows, rw.blocks_per_row

    def tensor_f32(self, name: str, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        check(self.lib.fl_gguf_tensor_f32(self.h, name.encode(), out.ctypes.data, n))
        return out


__all__ = ["write_gguf", "GgufFile", "model_tensors"]
