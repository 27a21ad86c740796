"""GPU checks of the ComputeBackend entry points whose arguments mirror the
reference trait exactly (flare-core/src/model.rs:176-618):

* forward_single_token_gpu(token_embedding, pos, ...) (555-557): the f32
  embedding row as input -- fl_decode_step_embed;
* batched_dequant_matmul(&RawWeight, input: &[f32], batch) (468; CPU
  740-1036): f32 rows quantized on the device, then the quantized matvec --
  fl_op_batched_dequant_matmul;
* prefill_attention_gpu(q, k, v, seq_len, ...) (336-368): causal attention,
  token t over 0..t -- fl_op_prefill_attention.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(got, want, rel=1e-3, floor=1e-6):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    bound = rel * np.maximum(np.abs(want), 1e-3 * scale) + floor * scale
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}, scale {scale:.3e}"


@pytest.mark.parametrize("name,spec", [
    ("q8_tied", S.tiny_spec(FL_Q8_0)),
    ("q4k_q6k_out", S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K)),
])
@pytest.mark.parametrize("kv", [FL_KV_F32, FL_KV_F16])
def test_forward_single_token_gpu_takes_the_embedding(backend, oracle, name, spec, kv):
    """The embedding-row entry point gives the same logits as the token-id
    one (the same x enters the same step), position by position."""
    print(f"[embed] {name} kv={kv}", flush=True)
    model = S.make_model(spec, seed=8)
    emb = oracle.dequant(model.embedding.data, spec.embed_fmt, spec.vocab, spec.hidden)
    toks = S.random_tokens(9, 10, spec.vocab)
    backend.init_gpu_kv_cache(spec, kv)
    backend.upload_weights_to_gpu(model)
    by_id = [backend.forward_single_token_gpu(int(t), p) for p, t in enumerate(toks)]
    backend.reset()
    by_row = [backend.forward_single_token_gpu(emb[int(t)], p) for p, t in enumerate(toks)]
    for a, b in zip(by_id, by_row):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("fmt,rows,cols,batch", [
    (FL_Q8_0, 300, 576, 1), (FL_Q8_0, 2048, 2048, 7), (FL_Q8_0, 1000, 256, 40),
    (FL_Q4K, 1024, 4096, 8), (FL_Q4K, 257, 512, 21),
])
def test_batched_dequant_matmul_f32_input(backend, oracle, fmt, rows, cols, batch):
    print(f"[batched-dequant] fmt={fmt} {rows}x{cols} batch={batch}", flush=True)
    w = S.quantize(S.normal(rows * 3 + cols, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    x = np.stack([S.normal(500 + b, 0, cols, 0.0, 1.0) for b in range(batch)]).astype(np.float32)
    got = backend.batched_dequant_matmul(W, _t(x)).cpu().numpy()
    for b in range(batch):
        q, s = oracle.quantize_q8(x[b])
        _close(got[b], oracle.matvec(w, fmt, rows, cols, q, s))


@pytest.mark.parametrize("nh,nkv,hd,T", [(4, 2, 64, 1), (4, 2, 64, 37), (9, 3, 64, 130), (32, 8, 128, 300),
                                         (8, 8, 128, 65), (32, 8, 64, 520)])
def test_prefill_attention_causal(backend, oracle, nh, nkv, hd, T):
    """Every query t against cpu_grouped_query_attention over rows 0..t
    (or_gqa_attention, the reference's online softmax)."""
    print(f"[prefill-attn] nh={nh} nkv={nkv} hd={hd} T={T}", flush=True)
    rng = np.random.default_rng(T + hd)
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    got = backend.prefill_attention_gpu(_t(q), _t(k), _t(v), T, nh, nkv, hd).cpu().numpy()
    for t in range(T):
        want = oracle.gqa_attention(q[t], k[:t + 1], v[:t + 1], nh, nkv, hd, t + 1)
        _close(got[t], want, floor=1e-5)


@pytest.mark.parametrize("name,spec", [
    ("q8_tied", S.tiny_spec(FL_Q8_0)),
    ("q4k_q6k_out", S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K)),
])
def test_upload_f32_tables_as_the_trait_passes_them(backend, oracle, name, spec):
    """upload_weights_to_gpu (model.rs:526) hands over the output and
    embedding as f32 tables.  Uploaded as FL_F32 weights, the reference-order
    step gives logits bit-identical to the oracle's (which dequantizes the
    same tables)."""
    from flarellm_amd import _lib as L

    print(f"[f32-tables] {name}", flush=True)
    model = S.make_model(spec, seed=13)
    emb = oracle.dequant(model.embedding.data, spec.embed_fmt, spec.vocab, spec.hidden)
    f32 = S.SynthModel(spec, model.layers, model.attn_norms, model.ffn_norms, model.output_norm,
                       S.QWeight(np.ascontiguousarray(emb).view(np.uint8).ravel(), S.FL_F32, spec.vocab, spec.hidden),
                       None)
    if model.output is not None:
        out = oracle.dequant(model.output.data, spec.output_fmt, spec.vocab, spec.hidden)
        f32.output = S.QWeight(np.ascontiguousarray(out).view(np.uint8).ravel(), S.FL_F32, spec.vocab, spec.hidden)
    backend.set_option(L.FL_OPT_EXACT, 1)
    try:
        backend.init_gpu_kv_cache(spec, FL_KV_F32)
        backend.upload_weights_to_gpu(f32)
        om = oracle.OracleModel(model)
        toks = S.random_tokens(14, 12, spec.vocab)
        for pos, t in enumerate(toks):
            g = backend.forward_single_token_gpu(emb[int(t)], pos)
            w = om.forward_logits(int(t), pos)
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), pos
    finally:
        backend.set_option(L.FL_OPT_EXACT, 0)
