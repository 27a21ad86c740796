"""Speculative verify (BASELINE config 5's pass) on the GPU.

* fl_op_batched_matvec_q8in: every token row of the int8-MFMA GEMM equals the
  oracle's single-token quantized matvec within 1e-3 relative (only the fp32
  order of the block terms differs);
* fl_op_batched_block_dots: the per-block integer dots those GEMMs' MFMAs
  form equal the oracle's bit for bit, at the C3 / C5 shapes for M = 8
  (verify) and 64 (prefill).
* fl_verify: the greedy token after each of M drafts equals what sequential
  decode gives -- the GPU's own fl_decode_step loop and the oracle -- wherever
  the oracle's top-2 logit gap is not a near-tie.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_KV_KIVI2, FL_KV_Q8, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

REL = 1e-3


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(got, want, rel=REL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    bound = rel * np.maximum(np.abs(want), 1e-3 * scale) + 1e-6 * scale
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}, scale {scale:.3e}"


GEMM_SHAPES = [(FL_Q8_0, 96, 256, 1), (FL_Q8_0, 1001, 2048, 8), (FL_Q8_0, 64, 576, 3), (FL_Q8_0, 200, 8192, 16),
               (FL_Q4K, 96, 256, 8), (FL_Q4K, 130, 4096, 5), (FL_Q4K, 64, 14336, 8), (FL_Q4K, 6144, 4096, 8),
               (FL_Q4K, 1536, 4096, 16),
               # prefill batches (17..64 tokens): 256-value steps staged through LDS
               (FL_Q8_0, 3072, 2048, 64), (FL_Q8_0, 513, 8192, 37), (FL_Q4K, 6144, 4096, 64),
               (FL_Q4K, 4096, 14336, 50), (FL_Q4K, 130, 4096, 17)]


# the BASELINE C5 / C3 GEMM shapes at M = 8 (verify) and 64 (prefill pass),
# plus one shape per token-tile kernel (M 5, 16, 37)
DOT_SHAPES = [(FL_Q4K, 6144, 4096, 8), (FL_Q4K, 28672, 4096, 8), (FL_Q4K, 4096, 14336, 8),
              (FL_Q4K, 6144, 4096, 64), (FL_Q4K, 28672, 4096, 64), (FL_Q4K, 4096, 14336, 64),
              (FL_Q4K, 1536, 4096, 16), (FL_Q4K, 130, 4096, 37),
              (FL_Q8_0, 3072, 2048, 8), (FL_Q8_0, 16384, 2048, 64), (FL_Q8_0, 2048, 8192, 5),
              (FL_Q8_0, 1001, 2048, 16)]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("fmt,rows,cols,M", DOT_SHAPES)
def test_batched_block_dots_bit_exact(backend, oracle, fmt, rows, cols, M):
    """The per-block integer dots the verify / prefill GEMMs form on the int8
    MFMA, read back from the MFMA results (fl_op_batched_block_dots), equal
    the oracle's block dots of every token bit for bit (model.rs:8082-8099,
    8997-9014)."""
    print(f"[block-dots] fmt={fmt} {rows}x{cols} M={M}", flush=True)
    w = S.quantize(S.normal(rows + 7, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    qs, ss, sums = [], [], []
    for m in range(M):
        q, s = oracle.quantize_q8(S.normal(70 + m, 0, cols, 0.0, 1.0))
        qs.append(q)
        ss.append(s)
        sums.append(q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32))
    got = backend.batched_block_dots(W, _t(np.stack(qs)), _t(np.stack(ss)), _t(np.stack(sums))).cpu().numpy()
    for m in range(M):
        want = oracle.block_dots(w, fmt, rows, cols, qs[m])
        if fmt == FL_Q4K:
            # the oracle interleaves (sub-block j, sub-block j + 4); the readback is in sub-block order
            want = want.reshape(rows, cols // 256, 4, 2).transpose(0, 1, 3, 2).reshape(rows, cols // 32)
        assert np.array_equal(got[m], want), f"token {m}: {(got[m] != want).sum()} block dots differ"


@pytest.mark.parametrize("fmt,rows,cols,M", GEMM_SHAPES)
def test_batched_matvec_q8in(backend, oracle, fmt, rows, cols, M):
    print(f"[batched] fmt={fmt} {rows}x{cols} M={M}", flush=True)
    w = S.quantize(S.normal(rows + 3, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    qs, ss, sums = [], [], []
    for m in range(M):
        q, s = oracle.quantize_q8(S.normal(50 + m, 0, cols, 0.0, 1.0))
        qs.append(q)
        ss.append(s)
        sums.append(q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32))
    got = backend.batched_matvec_q8in(W, _t(np.stack(qs)), _t(np.stack(ss)), _t(np.stack(sums))).cpu().numpy()
    for m in range(M):
        _close(got[m], oracle.matvec(w, fmt, rows, cols, qs[m], ss[m]))


F32IN_SHAPES = [(FL_Q6K, 45, 4096, 8), (FL_Q6K, 1000, 256, 3), (FL_Q6K, 129, 4096, 1), (FL_Q8_0, 77, 576, 8),
                (FL_Q8_0, 1001, 2048, 5), (FL_Q8_0, 16, 64, 1)]


@pytest.mark.parametrize("fmt,rows,cols,M", F32IN_SHAPES)
def test_batched_matvec_f32in(backend, oracle, fmt, rows, cols, M):
    """MFMA logits kernel (f16 split input, exact codes) vs the oracle's f32
    dot over dequantized weights (matvec_f32, model.rs:7549), per token."""
    print(f"[batched-f32in] fmt={fmt} {rows}x{cols} M={M}", flush=True)
    w = S.quantize(S.normal(rows + 7, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    xs = np.stack([S.normal(70 + m, 0, cols, 0.0, 1.0) for m in range(M)]).astype(np.float32)
    got = backend.batched_matvec_f32in(W, _t(xs)).cpu().numpy()
    dq = oracle.dequant(w, fmt, rows, cols)
    for m in range(M):
        _close(got[m], oracle.matvec_f32(dq, xs[m]))


MODELS = {
    "q8_tied": S.tiny_spec(FL_Q8_0, max_seq=128),
    "q4k_q6k_out": S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K, max_seq=128),
    "q8_hd128": S.tiny_spec(FL_Q8_0, heads=8, kv_heads=2, head_dim=128, hidden=512, inter=768, max_seq=128),
}
KV = {"f32": FL_KV_F32, "f16": FL_KV_F16, "q8": FL_KV_Q8, "kivi": FL_KV_KIVI2}
MARGIN = 2e-2  # top-2 gap (relative) below which a position counts as a near-tie


def _omode(oracle, kv):
    return {FL_KV_F32: oracle.OR_KV_F32, FL_KV_F16: oracle.OR_KV_F16, FL_KV_Q8: oracle.OR_KV_Q8,
            FL_KV_KIVI2: oracle.OR_KV_KIVI32}[kv]


def _check_verify(backend, oracle, spec, kv, n_prompt, seed):
    M = 8
    model = S.make_model(spec, seed=seed)
    prompt = S.random_tokens(seed + 100, n_prompt, spec.vocab)
    drafts = S.random_tokens(seed + 200, M, spec.vocab)
    backend.init_gpu_kv_cache(spec, kv)
    backend.upload_weights_to_gpu(model)
    backend.generate(prompt, 1)  # positions 0..n_prompt-1
    got, vals = backend.verify(drafts, n_prompt)
    # the GPU's own sequential decode over the same drafts, full logits
    seq = [backend.forward_single_token_gpu(int(t), n_prompt + i) for i, t in enumerate(drafts)]
    # oracle logits for the near-tie margin
    om = oracle.OracleModel(model, _omode(oracle, kv))
    for pos, t in enumerate(prompt):
        om.forward_greedy(int(t), pos)
    checked = 0
    for i, t in enumerate(drafts):
        logits = om.forward_logits(int(t), n_prompt + i)
        top2 = np.sort(logits)[-2:]
        # verify's winning logit equals sequential decode's logit of that token
        assert abs(vals[i] - seq[i][got[i]]) <= 1e-2 * abs(top2[1]), (i, vals[i], seq[i][got[i]])
        if top2[1] - top2[0] > MARGIN * abs(top2[1]):
            assert got[i] == int(np.argmax(seq[i])) == int(np.argmax(logits)), (i, got[i], int(np.argmax(seq[i])))
            checked += 1
    assert checked >= M // 2


@pytest.mark.parametrize("name", list(MODELS))
@pytest.mark.parametrize("kv", list(KV))
def test_verify_matches_sequential_decode(backend, oracle, name, kv):
    print(f"[verify] {name} kv={kv}", flush=True)
    _check_verify(backend, oracle, MODELS[name], KV[kv], 40, 6)


@pytest.mark.parametrize("kv", ["f16", "q8", "kivi"])
def test_verify_long_context_split_attention(backend, oracle, kv):
    """Context above one attention split (1100 tokens): every draft query
    merges several split partials of its own."""
    print(f"[verify-long] kv={kv}", flush=True)
    spec = S.tiny_spec(FL_Q8_0, heads=8, kv_heads=2, head_dim=128, hidden=512, inter=768, max_seq=1200)
    _check_verify(backend, oracle, spec, KV[kv], 1100, 16)


def test_verify_accepts_sequential_greedy_stream(backend, oracle):
    """Drafts taken from the model's own greedy stream are all accepted:
    verify returns the stream shifted by one."""
    spec = MODELS["q8_tied"]
    model = S.make_model(spec, seed=8)
    prompt = S.random_tokens(108, 20, spec.vocab)
    backend.init_gpu_kv_cache(spec, FL_KV_F16)
    backend.upload_weights_to_gpu(model)
    stream = backend.generate(prompt, 17)  # greedy tokens after the prompt
    backend.reset()
    for pos, t in enumerate(prompt):
        backend.forward_greedy(int(t), pos)
    drafts = stream[:8].astype(np.uint32)
    got, _ = backend.verify(drafts, len(prompt))
    assert got.tolist() == stream[1:9].tolist()


@pytest.mark.parametrize("kv", ["f16", "q8"])
def test_verify_graph_replays_match_eager(backend, oracle, kv, monkeypatch):
    """The captured verify graph (F16 / Q8 caches) against the same pass
    enqueued kernel by kernel: identical tokens and logits on every replay,
    with the program's own decode steps and synchronizations in between, at
    two batch sizes and two positions (the position is read on the device)."""
    print(f"[verify-graph] kv={kv}", flush=True)
    spec = MODELS["q8_hd128"]
    model = S.make_model(spec, seed=21)
    prompt = S.random_tokens(121, 30, spec.vocab)
    backend.init_gpu_kv_cache(spec, KV[kv])
    backend.upload_weights_to_gpu(model)
    backend.generate(prompt, 1)
    for M, pos in ((8, 30), (5, 30), (8, 33)):
        drafts = S.random_tokens(200 + M + pos, M, spec.vocab)
        monkeypatch.setenv("FLARE_NO_VERIFY_GRAPH", "1")
        want, wv = backend.verify(drafts, pos)
        monkeypatch.delenv("FLARE_NO_VERIFY_GRAPH")
        for rep in range(3):
            got, gv = backend.verify(drafts, pos)
            assert got.tolist() == want.tolist(), (M, pos, rep)
            assert np.array_equal(gv, wv), (M, pos, rep)
            # eager work between replays (rewrites the first slots it verified)
            backend.forward_greedy(int(drafts[0]), pos)
            backend.sync()
