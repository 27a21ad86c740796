"""ctypes binding of libflare_hip.so (the C-ABI in include/flare_hip.h).

The library is built in-tree by ``flarellm_amd.build``.  There is no Python
or CPU fallback: if the library is missing, loading raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os

# FLARE_LIB: load another build of the library (diagnostic builds, e.g. with
# FLARE_BUILD_DEFS; measurement only)
LIB_PATH = os.environ.get("FLARE_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflare_hip.so")

FL_F32, FL_Q8_0, FL_Q4K, FL_Q6K = 0, 1, 2, 3
FL_KV_F32, FL_KV_F16, FL_KV_Q8, FL_KV_KIVI2 = 0, 1, 2, 3
FL_OPT_VERIFY_FUSE, FL_OPT_VERIFY_GRAPH, FL_OPT_EXACT, FL_OPT_FUSE_ATTN = 1, 2, 3, 4
FORMAT_NAMES = {FL_F32: "F32", FL_Q8_0: "Q8_0", FL_Q4K: "Q4_K", FL_Q6K: "Q6_K"}


class FlareError(RuntimeError):
    pass


class RawWeight(C.Structure):
    """fl_raw_weight == flarellm RawWeight (model.rs:123-130)."""

    _fields_ = [
        ("data", C.c_void_p),
        ("nbytes", C.c_size_t),
        ("format", C.c_int),
        ("num_rows", C.c_int),
        ("blocks_per_row", C.c_int),
    ]


class ModelConfig(C.Structure):
    _fields_ = [
        ("hidden_dim", C.c_int),
        ("num_layers", C.c_int),
        ("num_heads", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("intermediate_dim", C.c_int),
        ("vocab_size", C.c_int),
        ("max_seq_len", C.c_int),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
    ]


vp, i32, f32, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t


class SamplingParams(C.Structure):
    """fl_sampling_params == flarellm SamplingParams (sampling.rs:19-54)
    without the self-speculation fields."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_int),
        ("repeat_penalty", C.c_float),
        ("min_p", C.c_float),
        ("speculative", C.c_int),
    ]


class SpecStats(C.Structure):
    """fl_spec_stats == SpeculativeStats (generate.rs:22-30)."""

    _fields_ = [("attempts", C.c_uint64), ("drafted", C.c_uint64), ("accepted", C.c_uint64)]


RNG_FN = C.CFUNCTYPE(C.c_float, C.c_void_p)
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_uint32, C.c_size_t, C.c_void_p)

# name -> (restype, argtypes); every symbol here must be declared in
# include/flare_hip.h (checked by tests/test_abi.py).
SIGNATURES = {
    "fl_abi_version": (i32, []),
    "fl_backend_name": (C.c_char_p, []),
    "fl_ctx_create": (i32, [i32, C.POINTER(vp)]),
    "fl_ctx_destroy": (None, [vp]),
    "fl_last_error": (C.c_char_p, [vp]),
    "fl_ctx_stream": (vp, [vp]),
    "fl_sync": (i32, [vp]),
    "fl_set_option": (i32, [vp, i32, i32]),
    "fl_weight_upload": (i32, [vp, C.POINTER(RawWeight), C.POINTER(vp)]),
    "fl_weight_free": (None, [vp, vp]),
    "fl_op_quantize_q8": (i32, [vp, vp, i32, vp, vp, vp]),
    "fl_op_rmsnorm_quantize_q8": (i32, [vp, vp, vp, i32, f32, i32, vp, vp, vp]),
    "fl_op_rmsnorm": (i32, [vp, vp, vp, i32, f32, vp]),
    "fl_op_matvec_q8in": (i32, [vp, vp, vp, vp, vp, vp]),
    "fl_op_matvec_f32in": (i32, [vp, vp, vp, vp]),
    "fl_op_batched_matvec_q8in": (i32, [vp, vp, i32, vp, vp, vp, vp]),
    "fl_op_batched_matvec_f32in": (i32, [vp, vp, i32, vp, vp]),
    "fl_op_batched_matvec_q8in_noalloc": (i32, [vp, vp, i32, vp, vp, vp, vp]),
    "fl_op_batched_dequant_matmul": (i32, [vp, vp, vp, i32, vp]),
    "fl_op_prefill_attention": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "fl_decode_step_embed": (i32, [vp, vp, i32, vp, C.POINTER(C.c_int32), C.POINTER(f32)]),
    "fl_op_block_dots": (i32, [vp, vp, vp, vp]),
    "fl_op_dequant": (i32, [vp, vp, vp]),
    "fl_op_matvec_argmax": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
    "fl_op_rope": (i32, [vp, vp, i32, i32, i32, f32]),
    "fl_op_silu_mul": (i32, [vp, vp, vp, i32, vp]),
    "fl_op_attention": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
    "fl_model_init": (i32, [vp, C.POINTER(ModelConfig), i32]),
    "fl_upload_weights": (
        i32,
        [vp, C.POINTER(RawWeight), C.POINTER(vp), C.POINTER(vp), vp, C.POINTER(RawWeight), C.POINTER(RawWeight)],
    ),
    "fl_has_weights": (i32, [vp]),
    "fl_has_kv_cache": (i32, [vp]),
    "fl_kv_write": (i32, [vp, i32, i32, vp, vp]),
    "fl_reset": (i32, [vp]),
    "fl_kv_write_batch": (i32, [vp, i32, i32, i32, vp, vp]),
    "fl_gqa_from_cache": (i32, [vp, i32, vp, i32, vp]),
    "fl_probe_layer": (i32, [vp, i32, vp]),
    "fl_op_batched_block_dots": (i32, [vp, vp, i32, vp, vp, vp, vp]),
    "fl_probe_layout": (i32, [vp, C.POINTER(C.c_size_t), i32]),
    "fl_bench_attention": (i32, [vp, i32, i32, C.POINTER(C.c_double)]),
    "fl_decode_step": (i32, [vp, C.c_uint32, i32, vp, C.POINTER(C.c_int32), C.POINTER(f32)]),
    "fl_generate": (i32, [vp, vp, i32, i32, vp]),
    "fl_decode_continue": (i32, [vp, i32]),
    "fl_verify": (i32, [vp, vp, i32, i32, vp, vp]),
    "fl_prefill": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "fl_decode_run": (i32, [vp, C.c_uint32, i32, i32, vp]),
    "fl_read_tokens": (i32, [vp, i32, i32, vp]),
    "fl_sampling_params_default": (None, [vp]),
    "fl_op_sample": (i32, [vp, vp, i32, vp, vp, i32, f32, C.POINTER(C.c_int32)]),
    "fl_decode_step_sample": (i32, [vp, C.c_uint32, i32, vp, vp, i32, f32, C.POINTER(C.c_int32)]),
    "fl_ngram_create": (vp, []),
    "fl_ngram_destroy": (None, [vp]),
    "fl_ngram_record": (None, [vp, vp, sz]),
    "fl_ngram_record_all": (None, [vp, vp, sz]),
    "fl_ngram_lookup": (i32, [vp, vp, sz, vp]),
    "fl_ngram_entries": (sz, [vp]),
    "fl_generator_create": (i32, [vp, vp, C.POINTER(vp)]),
    "fl_generator_destroy": (None, [vp]),
    "fl_generator_prefill": (i32, [vp, vp, i32, vp]),
    "fl_generator_step": (i32, [vp, f32, C.POINTER(C.c_uint32)]),
    "fl_generator_generate": (i32, [vp, vp, i32, i32, C.c_int64, vp, vp, vp, vp, vp, C.POINTER(i32)]),
    "fl_generator_stats": (i32, [vp, vp]),
    "fl_generator_position": (i32, [vp]),
    "fl_generator_tokens": (i32, [vp, vp, i32]),
    "fl_gguf_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "fl_gguf_open_memory": (i32, [vp, sz, C.POINTER(vp)]),
    "fl_gguf_close": (None, [vp]),
    "fl_gguf_version": (i32, [vp]),
    "fl_gguf_data_offset": (C.c_uint64, [vp]),
    "fl_gguf_tensor_count": (i32, [vp]),
    "fl_gguf_find_tensor": (i32, [vp, C.c_char_p]),
    "fl_gguf_tensor_info": (i32, [vp, i32, C.POINTER(C.c_char_p), C.POINTER(i32), vp, C.POINTER(C.c_uint32),
                                   C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "fl_gguf_meta_u64": (i32, [vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "fl_gguf_meta_f32": (i32, [vp, C.c_char_p, C.POINTER(f32)]),
    "fl_gguf_meta_str": (C.c_char_p, [vp, C.c_char_p]),
    "fl_gguf_model_config": (i32, [vp, C.POINTER(ModelConfig), C.POINTER(i32)]),
    "fl_gguf_raw_weight": (i32, [vp, C.c_char_p, C.POINTER(RawWeight)]),
    "fl_gguf_tensor_f32": (i32, [vp, C.c_char_p, vp, sz]),
    "fl_model_load_gguf": (i32, [vp, vp, i32, i32]),
    "fl_bench_layer_kernel": (i32, [vp, i32, i32, i32, C.POINTER(C.c_double)]),
    "fl_bench_kernel_name": (C.c_char_p, [vp, i32]),
    "fl_synth_normal": (None, [C.c_uint64, C.c_uint64, sz, f32, f32, vp]),
    "fl_synth_quantize": (sz, [vp, sz, sz, i32, vp]),
    "fl_format_row_bytes": (sz, [i32, sz]),
}

_lib = None


def load() -> C.CDLL:
    """Load libflare_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FlareError(
            f"{LIB_PATH} is missing: build it with `python -m flarellm_amd.build` "
            "(there is no CPU fallback)"
        )
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, ctx=None) -> None:
    if rc != 0:
        lib = load()
        msg = lib.fl_last_error(ctx)
        raise FlareError(f"flare_hip error {rc}: {msg.decode() if msg else ''}")
