"""Host-side mirror of flarellm's ComputeBackend decode hooks over the C-ABI.

`HipBackend` is what a flarellm `Model` would hold as `Box<dyn
ComputeBackend>` (flare-core/src/model.rs:176-618): it owns one fl_ctx
(one GPU, one HIP stream), the uploaded weights and the KV cache, and exposes
the decode entry points with the reference's names and argument meaning.
Per-op methods take torch tensors (device memory plumbing) and call the HIP
kernels through ctypes; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import FL_KV_F16, FL_KV_F32, FlareError, ModelConfig, RawWeight, check
from .synth import ModelSpec, SynthModel


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


class Weight:
    """A RawWeight uploaded to the device (fl_weight)."""

    def __init__(self, backend: "HipBackend", raw: RawWeight):
        self._b = backend
        h = C.c_void_p()
        check(backend.lib.fl_weight_upload(backend.ctx, C.byref(raw), C.byref(h)), backend.ctx)
        self.handle = h
        self.format = raw.format
        self.rows = raw.num_rows
        self.blocks_per_row = raw.blocks_per_row

    def free(self):
        if self.handle:
            self._b.lib.fl_weight_free(self._b.ctx, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipBackend:
    """ComputeBackend over libflare_hip.so (name(): model.rs:615)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        ctx = C.c_void_p()
        check(self.lib.fl_ctx_create(device, C.byref(ctx)))
        self.ctx = ctx
        self.spec: ModelSpec | None = None
        self._keep = []  # host buffers referenced by the last upload

    # ---- lifecycle ---------------------------------------------------------
    def name(self) -> str:
        return self.lib.fl_backend_name().decode()

    def close(self):
        if self.ctx:
            self.lib.fl_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return self.lib.fl_ctx_stream(self.ctx)

    def set_option(self, option: int, value: int):
        """fl_set_option: FL_OPT_VERIFY_FUSE / FL_OPT_VERIFY_GRAPH switches."""
        check(self.lib.fl_set_option(self.ctx, option, int(value)), self.ctx)

    def sync(self):
        check(self.lib.fl_sync(self.ctx), self.ctx)

    def _torch_sync(self):
        import torch

        torch.cuda.synchronize()

    # ---- per-op entry points (torch tensors on cuda) ------------------------
    def upload(self, qw) -> Weight:
        return Weight(self, qw.raw() if hasattr(qw, "raw") else qw)

    def quantize_q8(self, x):
        """quantize_input_q8_0_into (model.rs:5534-5571) -> (q, scales, sums)."""
        import torch

        n = x.numel()
        q = torch.empty(n, dtype=torch.int8, device=x.device)
        s = torch.empty(n // 32, dtype=torch.float32, device=x.device)
        su = torch.empty(n // 32, dtype=torch.int32, device=x.device)
        self._torch_sync()
        check(self.lib.fl_op_quantize_q8(self.ctx, _ptr(x), n, _ptr(q), _ptr(s), _ptr(su)), self.ctx)
        self.sync()
        return q, s, su

    def rmsnorm_quantize_q8(self, x, w, eps: float, order: int = 0):
        import torch

        n = x.numel()
        q = torch.empty(n, dtype=torch.int8, device=x.device)
        s = torch.empty(n // 32, dtype=torch.float32, device=x.device)
        su = torch.empty(n // 32, dtype=torch.int32, device=x.device)
        self._torch_sync()
        check(self.lib.fl_op_rmsnorm_quantize_q8(self.ctx, _ptr(x), _ptr(w), n, eps, order, _ptr(q), _ptr(s),
                                                 _ptr(su)), self.ctx)
        self.sync()
        return q, s, su

    def rmsnorm(self, x, w, eps: float):
        import torch

        out = torch.empty_like(x)
        self._torch_sync()
        check(self.lib.fl_op_rmsnorm(self.ctx, _ptr(x), _ptr(w), x.numel(), eps, _ptr(out)), self.ctx)
        self.sync()
        return out

    def matvec_q8in(self, w: Weight, q, s, su):
        import torch

        out = torch.empty(w.rows, dtype=torch.float32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_matvec_q8in(self.ctx, w.handle, _ptr(q), _ptr(s), _ptr(su), _ptr(out)), self.ctx)
        self.sync()
        return out

    def batched_matvec_q8in(self, w: Weight, q, s, su):
        """batched_dequant_matmul (model.rs:740) over n pre-quantized rows:
        q [n, cols] int8, s / su [n, cols/32] -> [n, rows] f32."""
        import torch

        n = q.shape[0]
        out = torch.empty((n, w.rows), dtype=torch.float32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_batched_matvec_q8in(self.ctx, w.handle, n, _ptr(q), _ptr(s), _ptr(su), _ptr(out)),
              self.ctx)
        return out

    def batched_block_dots(self, w: Weight, q, s, su):
        """Per-block integer dots of the batched GEMM (fl_op_batched_block_dots):
        [n_tokens, rows, K/32] int32."""
        import torch

        M = q.shape[0]
        out = torch.empty((M, w.rows, q.shape[1] // 32), dtype=torch.int32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_batched_block_dots(self.ctx, w.handle, M, _ptr(q), _ptr(s), _ptr(su), _ptr(out)),
              self.ctx)
        self.sync()
        return out

    def batched_matvec_f32in(self, w: Weight, x):
        """f32-input matvec for n rows x [n, cols] (Q6_K / Q8_0) -> [n, rows]."""
        import torch

        n = x.shape[0]
        out = torch.empty((n, w.rows), dtype=torch.float32, device=x.device)
        self._torch_sync()
        check(self.lib.fl_op_batched_matvec_f32in(self.ctx, w.handle, n, _ptr(x), _ptr(out)), self.ctx)
        self.sync()
        return out

    def batched_dequant_matmul(self, w: Weight, x):
        """ComputeBackend::batched_dequant_matmul (model.rs:468, 740-1036):
        f32 rows x [batch, cols] quantized on the device, then the quantized
        matvec of each row -> [batch, rows]."""
        import torch

        n = x.shape[0]
        out = torch.empty((n, w.rows), dtype=torch.float32, device=x.device)
        self._torch_sync()
        check(self.lib.fl_op_batched_dequant_matmul(self.ctx, w.handle, _ptr(x), n, _ptr(out)), self.ctx)
        return out

    def prefill_attention_gpu(self, q, k, v, seq_len: int, num_heads: int, num_kv_heads: int, head_dim: int):
        """ComputeBackend::prefill_attention_gpu (model.rs:336-368): causal
        attention of seq_len tokens (token t over 0..t); q [seq_len, nh*hd],
        k / v [seq_len, nkv*hd] -> [seq_len, nh*hd]."""
        import torch

        out = torch.empty((seq_len, num_heads * head_dim), dtype=torch.float32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_prefill_attention(self.ctx, _ptr(q), _ptr(k), _ptr(v), seq_len, num_heads,
                                               num_kv_heads, head_dim, _ptr(out)), self.ctx)
        return out

    def matvec_f32in(self, w: Weight, x):
        import torch

        out = torch.empty(w.rows, dtype=torch.float32, device=x.device)
        self._torch_sync()
        check(self.lib.fl_op_matvec_f32in(self.ctx, w.handle, _ptr(x), _ptr(out)), self.ctx)
        self.sync()
        return out

    def block_dots(self, w: Weight, q):
        import torch

        per_row = w.blocks_per_row * (8 if w.format == _lib.FL_Q4K else 1)
        out = torch.empty(w.rows * per_row, dtype=torch.int32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_block_dots(self.ctx, w.handle, _ptr(q), _ptr(out)), self.ctx)
        self.sync()
        return out.view(w.rows, per_row)

    def dequant(self, w: Weight, cols: int):
        import torch

        out = torch.empty(w.rows * cols, dtype=torch.float32, device="cuda")
        self._torch_sync()
        check(self.lib.fl_op_dequant(self.ctx, w.handle, _ptr(out)), self.ctx)
        self.sync()
        return out.view(w.rows, cols)

    def matvec_argmax(self, w: Weight, q=None, s=None, su=None, x=None):
        import torch

        dev = (q if q is not None else x).device
        idx = torch.zeros(1, dtype=torch.int64, device=dev)
        val = torch.zeros(1, dtype=torch.float32, device=dev)
        self._torch_sync()
        check(self.lib.fl_op_matvec_argmax(self.ctx, w.handle, _ptr(q), _ptr(s), _ptr(su), _ptr(x), _ptr(idx),
                                           _ptr(val)), self.ctx)
        self.sync()
        return int(idx.item()), float(val.item())

    def rope(self, data, num_heads: int, head_dim: int, pos: int, theta: float):
        """apply_rope_with_table in place (model.rs:7256-7297)."""
        self._torch_sync()
        check(self.lib.fl_op_rope(self.ctx, _ptr(data), num_heads, head_dim, pos, theta), self.ctx)
        self.sync()
        return data

    def silu_mul(self, gate, up):
        import torch

        out = torch.empty_like(gate)
        self._torch_sync()
        check(self.lib.fl_op_silu_mul(self.ctx, _ptr(gate), _ptr(up), gate.numel(), _ptr(out)), self.ctx)
        self.sync()
        return out

    def attention(self, q, k_cache, v_cache, num_heads: int, num_kv_heads: int, head_dim: int, seq_len: int,
                  num_splits: int = 0):
        """grouped_query_attention over a [slots, nkv, hd] cache (model.rs:9849)."""
        import torch

        fmt = FL_KV_F16 if k_cache.dtype == torch.float16 else FL_KV_F32
        out = torch.empty(num_heads * head_dim, dtype=torch.float32, device=q.device)
        self._torch_sync()
        check(self.lib.fl_op_attention(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache), fmt, num_heads,
                                       num_kv_heads, head_dim, seq_len, num_splits, _ptr(out)), self.ctx)
        self.sync()
        return out

    # ---- model decode hooks -------------------------------------------------
    def init_gpu_kv_cache(self, spec: ModelSpec, kv_format: int = FL_KV_F16):
        """init_gpu_kv_cache (model.rs:274) with the model config."""
        cfg = ModelConfig(spec.hidden, spec.layers, spec.heads, spec.kv_heads, spec.head_dim, spec.inter,
                          spec.vocab, spec.max_seq, spec.eps, spec.theta)
        check(self.lib.fl_model_init(self.ctx, C.byref(cfg), kv_format), self.ctx)
        self.spec = spec

    def upload_weights_to_gpu(self, model: SynthModel):
        """upload_weights_to_gpu (model.rs:526) from raw GGUF-layout weights."""
        L = model.spec.layers
        raws = (RawWeight * (7 * L))()
        for l, ws in enumerate(model.layers):
            for j, w in enumerate(ws):
                raws[7 * l + j] = w.raw()
        an = (C.c_void_p * L)(*[a.ctypes.data for a in model.attn_norms])
        fn = (C.c_void_p * L)(*[a.ctypes.data for a in model.ffn_norms])
        emb = model.embedding.raw()
        out = model.output.raw() if model.output is not None else None
        check(self.lib.fl_upload_weights(self.ctx, raws, an, fn, model.output_norm.ctypes.data, C.byref(emb),
                                         C.byref(out) if out is not None else None), self.ctx)

    def load_gguf(self, path: str, kv_format: int = FL_KV_F16, max_seq_len: int = 0) -> ModelSpec:
        """init_gpu_kv_cache + upload_weights_to_gpu from a GGUF file
        (fl_model_load_gguf: memory-mapped, weights streamed from the
        mapping).  Returns the model's spec."""
        from .gguf import GgufFile

        g = GgufFile(path)
        try:
            cfg, _arch = g.model_config()
            fmts = {}
            for name in ("blk.0.attn_q.weight", "token_embd.weight", "output.weight"):
                if g.find_tensor(name) >= 0:
                    fmts[name] = g.raw_weight(name)[1]
            check(self.lib.fl_model_load_gguf(self.ctx, g.h, kv_format, max_seq_len), self.ctx)
        finally:
            g.close()
        self.spec = ModelSpec(path, cfg.hidden_dim, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                              cfg.intermediate_dim, cfg.vocab_size, max_seq_len or cfg.max_seq_len,
                              fmts["blk.0.attn_q.weight"], fmts["token_embd.weight"], fmts.get("output.weight"),
                              cfg.rms_norm_eps, cfg.rope_theta)
        return self.spec

    def has_gpu_weights(self) -> bool:
        return bool(self.lib.fl_has_weights(self.ctx))

    def has_gpu_kv_cache(self) -> bool:
        return bool(self.lib.fl_has_kv_cache(self.ctx))

    def gpu_kv_write(self, layer: int, position: int, key: np.ndarray, value: np.ndarray):
        key = np.ascontiguousarray(key, np.float32)
        value = np.ascontiguousarray(value, np.float32)
        check(self.lib.fl_kv_write(self.ctx, layer, position, key.ctypes.data, value.ctypes.data), self.ctx)

    def gpu_kv_write_batch(self, layer: int, pos0: int, keys: np.ndarray, values: np.ndarray):
        """gpu_kv_write (model.rs:287) for consecutive rows [n, nkv*hd] at pos0.."""
        keys = np.ascontiguousarray(keys, np.float32)
        values = np.ascontiguousarray(values, np.float32)
        n = keys.shape[0]
        check(self.lib.fl_kv_write_batch(self.ctx, layer, pos0, n, keys.ctypes.data, values.ctypes.data), self.ctx)

    def grouped_query_attention_from_gpu_cache(self, q: np.ndarray, layer: int, seq_len: int) -> np.ndarray:
        """grouped_query_attention_from_gpu_cache (model.rs:311): one query
        token (RoPE applied) over slots 0..seq_len-1 of layer's cache."""
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty(self.spec.heads * self.spec.head_dim, np.float32)
        check(self.lib.fl_gqa_from_cache(self.ctx, layer, q.ctypes.data, seq_len, out.ctypes.data), self.ctx)
        return out

    def bench_attention(self, seq_len: int, iters: int) -> float:
        """Enqueue iters attention launches over seq_len tokens (synchronises);
        returns the algorithmic K+V bytes of one launch."""
        b = C.c_double()
        check(self.lib.fl_bench_attention(self.ctx, seq_len, iters, C.byref(b)), self.ctx)
        return b.value

    def reset(self):
        check(self.lib.fl_reset(self.ctx), self.ctx)

    def forward_greedy(self, token: int, pos: int) -> tuple[int, float]:
        """Model::forward_greedy (model.rs:1872-1942) on the device."""
        t = C.c_int32()
        v = C.c_float()
        check(self.lib.fl_decode_step(self.ctx, token, pos, None, C.byref(t), C.byref(v)), self.ctx)
        return t.value, v.value

    def forward_single_token_gpu(self, token, pos: int) -> np.ndarray:
        """forward_single_token_gpu (model.rs:555): full logits.  `token` is
        the f32 embedding row (the reference's argument) or a token id whose
        row the device dequantizes."""
        out = np.empty(self.spec.vocab, np.float32)
        t = C.c_int32()
        v = C.c_float()
        if isinstance(token, np.ndarray):
            emb = np.ascontiguousarray(token, np.float32)
            assert emb.size == self.spec.hidden
            check(self.lib.fl_decode_step_embed(self.ctx, emb.ctypes.data, pos, out.ctypes.data, C.byref(t),
                                                C.byref(v)), self.ctx)
        else:
            check(self.lib.fl_decode_step(self.ctx, int(token), pos, out.ctypes.data, C.byref(t), C.byref(v)),
                  self.ctx)
        return out

    PROBE_FIELDS = ("x_in", "q", "k", "v", "attn", "attn_s", "x_mid", "h_s", "x_out", "x_final", "attn_q", "h_q",
                    "x_q", "x_s", "f_q", "f_s")
    PROBE_TOKENS = 16

    def probe_layer(self, layer: int):
        """Layer probe (fl_probe_layer): the following decode steps and
        verify passes record layer `layer`'s intermediates; read them with
        probe_read().  None turns it off."""
        if layer is None or layer < 0:
            check(self.lib.fl_probe_layer(self.ctx, -1, None), self.ctx)
            self._probe = None
            return
        off = (C.c_size_t * 16)()
        total = self.lib.fl_probe_layout(self.ctx, off, 16)
        assert total > 0
        self._probe = (np.zeros(total, np.uint8), list(off))
        check(self.lib.fl_probe_layer(self.ctx, layer, self._probe[0].ctypes.data), self.ctx)

    def probe_read(self, n_tokens: int = 1) -> dict:
        """The last probed step's (or verify pass's) intermediates, [n_tokens, n]
        arrays (copies); n_tokens = 1 for a decode step, squeezed."""
        buf, off = self._probe
        sp = self.spec
        nq, nk, H, F = sp.heads * sp.head_dim, sp.kv_heads * sp.head_dim, sp.hidden, sp.inter
        sizes = {"x_in": H, "q": nq, "k": nk, "v": nk, "attn": nq, "attn_s": nq // 32, "x_mid": H, "h_s": F // 32,
                 "x_out": H, "x_final": H, "attn_q": nq, "h_q": F, "x_q": H, "x_s": H // 32, "f_q": H,
                 "f_s": H // 32}
        out = {}
        for i, name in enumerate(self.PROBE_FIELDS):
            n = sizes[name] * n_tokens
            if name in ("attn_q", "h_q", "x_q", "f_q"):
                a = buf[off[i]:off[i] + n].view(np.int8).copy()
            else:
                a = buf[off[i]:off[i] + 4 * n].view(np.float32).copy()
            a = a.reshape(n_tokens, -1)
            out[name] = a[0] if n_tokens == 1 else a
        return out

    def generate(self, prompt, n_gen: int) -> np.ndarray:
        """Greedy Generator loop (generate.rs:186-206), device-resident."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_gen, np.uint32)
        check(self.lib.fl_generate(self.ctx, prompt.ctypes.data, prompt.size, n_gen, out.ctypes.data), self.ctx)
        return out

    def verify(self, tokens, pos0: int):
        """Speculative verify of draft tokens at pos0.. in one pass: the greedy
        token after each draft (and its logit)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(tokens.size, np.int32)
        vals = np.empty(tokens.size, np.float32)
        check(self.lib.fl_verify(self.ctx, tokens.ctypes.data, tokens.size, pos0, out.ctypes.data,
                                 vals.ctypes.data), self.ctx)
        return out, vals

    def forward_prefill(self, tokens, pos0: int = 0, logits: bool = True):
        """Model::forward_prefill (model.rs:2578-3040): the prompt in batched
        passes; returns (logits of the last token or None, greedy token,
        its value)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.spec.vocab, np.float32) if logits else None
        t = C.c_int32()
        v = C.c_float()
        check(self.lib.fl_prefill(self.ctx, tokens.ctypes.data, tokens.size, pos0,
                                  out.ctypes.data if logits else None, C.byref(t), C.byref(v)), self.ctx)
        return out, t.value, v.value

    def decode_run(self, token: int, pos: int, n_steps: int) -> np.ndarray:
        """n_steps device-resident greedy steps from `token` at `pos`."""
        out = np.empty(n_steps, np.uint32)
        check(self.lib.fl_decode_run(self.ctx, int(token), pos, n_steps, out.ctypes.data), self.ctx)
        return out

    def decode_continue(self, n_steps: int):
        """Enqueue n_steps more device-resident greedy steps (asynchronous)."""
        check(self.lib.fl_decode_continue(self.ctx, n_steps), self.ctx)

    def read_tokens(self, start: int, n: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        check(self.lib.fl_read_tokens(self.ctx, start, n, out.ctypes.data), self.ctx)
        return out

    def bench_layer_kernel(self, which: int, iters: int, first_layer: int = 0) -> float:
        b = C.c_double()
        check(self.lib.fl_bench_layer_kernel(self.ctx, which, first_layer, iters, C.byref(b)), self.ctx)
        return b.value

    def bench_kernel_name(self, which: int) -> str:
        return self.lib.fl_bench_kernel_name(self.ctx, which).decode()


class Generator:
    """flarellm Generator (flare-core/src/generate.rs:106-560) over a backend
    holding a model: fl_generator_* in the library (n-gram drafts verified in
    one fl_verify pass, sampling on the device)."""

    def __init__(self, backend: "HipBackend", temperature=0.7, top_p=0.9, top_k=40, repeat_penalty=1.1,
                 min_p=0.0, speculative=True):
        self.b = backend
        self.lib = backend.lib
        self.params = _lib.SamplingParams(temperature, top_p, int(top_k), repeat_penalty, min_p, int(bool(speculative)))
        h = C.c_void_p()
        check(self.lib.fl_generator_create(backend.ctx, C.byref(self.params), C.byref(h)), backend.ctx)
        self.h = h

    def close(self):
        if self.h:
            self.lib.fl_generator_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, prompt, logits: bool = False):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(self.b.spec.vocab, np.float32) if logits else None
        check(self.lib.fl_generator_prefill(self.h, prompt.ctypes.data, prompt.size,
                                            out.ctypes.data if logits else None), self.b.ctx)
        return out

    def step(self, u: float = 0.5) -> int:
        t = C.c_uint32()
        check(self.lib.fl_generator_step(self.h, u, C.byref(t)), self.b.ctx)
        return t.value

    def generate(self, prompt, max_tokens: int, eos=None, rng=None, on_token=None) -> list:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_tokens, 1), np.uint32)
        n = C.c_int()
        rng_cb = _lib.RNG_FN(lambda _u: float(rng())) if rng is not None else None
        tok_cb = _lib.TOKEN_FN(lambda t, s, _u: 1 if on_token(int(t), int(s)) else 0) if on_token is not None else None
        check(self.lib.fl_generator_generate(self.h, prompt.ctypes.data, prompt.size, max_tokens,
                                             -1 if eos is None else int(eos),
                                             C.cast(rng_cb, C.c_void_p) if rng_cb else None, None,
                                             C.cast(tok_cb, C.c_void_p) if tok_cb else None, None,
                                             out.ctypes.data, C.byref(n)), self.b.ctx)
        return [int(x) for x in out[:n.value]]

    def stats(self):
        st = _lib.SpecStats()
        check(self.lib.fl_generator_stats(self.h, C.byref(st)), self.b.ctx)
        return st.attempts, st.drafted, st.accepted

    @property
    def position(self) -> int:
        return self.lib.fl_generator_position(self.h)

    def tokens(self) -> list:
        n = self.lib.fl_generator_tokens(self.h, None, 0)
        out = np.empty(max(n, 1), np.uint32)
        self.lib.fl_generator_tokens(self.h, out.ctypes.data, n)
        return [int(x) for x in out[:n]]


def sample_logits(backend: "HipBackend", logits_dev, temperature=0.7, top_p=0.9, top_k=40, repeat_penalty=1.1,
                  min_p=0.0, prev=(), u=0.5) -> int:
    """fl_op_sample over a device logits row (a torch tensor)."""
    params = _lib.SamplingParams(temperature, top_p, int(top_k), repeat_penalty, min_p, 0)
    prev = np.ascontiguousarray(prev, np.uint32)
    t = C.c_int32()
    check(backend.lib.fl_op_sample(backend.ctx, logits_dev.data_ptr(), logits_dev.numel(), C.byref(params),
                                   prev.ctypes.data if prev.size else None, prev.size, u, C.byref(t)), backend.ctx)
    return t.value


__all__ = ["HipBackend", "Generator", "Weight", "FlareError", "sample_logits"]
