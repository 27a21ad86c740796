"""GPU parity of the quantized KV caches (Q8, KIVI 2-bit) against the CPU
oracle: attention read straight from the cache (grouped_query_attention_from_
gpu_cache, model.rs:311) after rows written in batches and one at a time, and
whole-model greedy decode where the decode step itself quantizes the new
token (and, for KIVI, each group that leaves the fp16 window).

Bar: attention output within 1e-3 relative (fp32 accumulate) of
or_gqa_attention over the oracle's view of the cache (or_kv_view); greedy
token streams identical for 64 tokens.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_KV_KIVI2, FL_KV_Q8, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

REL = 1e-3


def _close(got, want, rel=REL, floor=1e-6, absb=None):
    """err <= rel*|want| (|want| floored at 1e-3 of the output scale) plus an
    absolute allowance: floor * scale, or the per-element bound absb."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    bound = rel * np.maximum(np.abs(want), 1e-3 * scale) + (floor * scale if absb is None else absb)
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}, scale {scale:.3e}"


def _attention_f64(q, K, V, nh, with_abs=False):
    """Textbook softmax(q k / sqrt(D)) v in float64 over token-major K, V;
    with_abs also returns sum_t p_t |v_t| per output (the magnitude of the
    terms an output sums)."""
    T, nkv, D = K.shape
    G = nh // nkv
    qh = q.reshape(nh, D).astype(np.float64)
    out = np.empty((nh, D))
    mag = np.empty((nh, D))
    for h in range(nh):
        k = K[:, h // G, :].astype(np.float64)
        v = V[:, h // G, :].astype(np.float64)
        s = k @ qh[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v
        mag[h] = p @ np.abs(v)
    return (out.ravel(), mag.ravel()) if with_abs else out.ravel()


# Outputs that cancel to near zero carry the rounding of every p*v term they
# sum.  The MFMA kernel forms q and p as f16 high + f16 residual (~22 bits:
# relative error <= 2^-22 per product) and accumulates in fp32, so an output
# over T tokens is allowed ATTN_C * sqrt(T) * 2^-22 * sum_t p_t |v_t| on top of
# the relative bar (random-sign accumulation of T per-term errors), and at
# least ATTN_FLOOR of the output scale.
ATTN_FLOOR = 1e-5
ATTN_C = 4.0


def _attn_abs_bound(mag, T):
    return ATTN_C * np.sqrt(T) * 2.0 ** -22 * mag


def _mode(oracle, fmt):
    return {FL_KV_F32: oracle.OR_KV_F32, FL_KV_F16: oracle.OR_KV_F16, FL_KV_Q8: oracle.OR_KV_Q8,
            FL_KV_KIVI2: oracle.OR_KV_KIVI32}[fmt]


def _write(backend, layer, K, V, single_tail=3):
    """Rows in three batches and the last few one at a time."""
    T = K.shape[0]
    flat = lambda a: a.reshape(a.shape[0], -1)  # noqa: E731
    cut = [0, T // 3, (2 * T) // 3, max((2 * T) // 3, T - single_tail), T]
    for a, b in zip(cut[:-2], cut[1:-1]):
        if b > a:
            backend.gpu_kv_write_batch(layer, a, flat(K[a:b]), flat(V[a:b]))
    for t in range(cut[-2], T):
        backend.gpu_kv_write(layer, t, K[t].ravel(), V[t].ravel())


FMTS = {"q8": FL_KV_Q8, "kivi": FL_KV_KIVI2, "f16": FL_KV_F16}
SHAPES = [  # (head_dim, heads, kv_heads, T)
    (64, 4, 2, 1), (64, 4, 2, 33), (64, 9, 3, 129), (64, 4, 2, 161), (64, 32, 8, 200),
    (128, 8, 8, 160), (128, 32, 8, 193), (128, 32, 8, 1000), (128, 32, 8, 8192),
    # C4 contexts at Llama-3-8B heads
    (128, 32, 8, 32768), (128, 32, 8, 131072),
]


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("hd,nh,nkv,T", SHAPES)
def test_attention_from_quantized_cache(backend, oracle, fmt, hd, nh, nkv, T):
    print(f"[kv-attn] {fmt} hd={hd} nh={nh} nkv={nkv} T={T}", flush=True)
    spec = S.tiny_spec(FL_Q8_0, heads=nh, kv_heads=nkv, head_dim=hd, max_seq=max(T, 32), layers=2 if T < 32768 else 1)
    backend.init_gpu_kv_cache(spec, FMTS[fmt])
    rng = np.random.default_rng(T * 7 + hd)
    K = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    V = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    layer = spec.layers - 1
    _write(backend, layer, K, V)
    got = backend.grouped_query_attention_from_gpu_cache(q, layer, T)
    Kv, Vv = oracle.kv_view(_mode(oracle, FMTS[fmt]), K, V)
    want64, mag = _attention_f64(q, Kv, Vv, nh, with_abs=True)
    _close(got, want64, absb=np.maximum(_attn_abs_bound(mag, T), ATTN_FLOOR * np.abs(want64).max()))
    # the oracle's fp32 online-softmax form agrees with the float64 form too
    _close(oracle.gqa_attention(q, Kv, Vv, nh, nkv, hd, T), want64, floor=ATTN_FLOOR)


@pytest.mark.parametrize("fmt", ["q8", "kivi", "f16"])
@pytest.mark.parametrize("T", [32768, 131072])
def test_attention_quantized_cache_properties_long(backend, oracle, fmt, T):
    """C4 contexts: softmax weights sum to one, so with V rows all equal to a
    constant vector c the output is c; with uniform keys the output is the
    mean of the (cache-form) V rows."""
    hd, nh, nkv = 128, 32, 8
    print(f"[kv-long] {fmt} T={T}", flush=True)
    spec = S.tiny_spec(FL_Q8_0, heads=nh, kv_heads=nkv, head_dim=hd, max_seq=T, layers=1)
    backend.init_gpu_kv_cache(spec, FMTS[fmt])
    rng = np.random.default_rng(11)
    K = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    # a V row the cache form stores exactly: Q8 -> multiples of 1/128 with
    # +-127/128 in every 32-block (step exactly 1/128); KIVI -> the four
    # levels -0.75, -0.25, 0.25, 0.75 with both ends in every 32-group
    if fmt in ("q8", "f16"):  # multiples of 1/128 are exact binary16 too
        m = rng.integers(-127, 128, (1, nkv, hd)).astype(np.float32)
        m[..., ::32] = 127.0
        c = m / 128.0
    else:
        lv = np.array([-0.75, -0.25, 0.25, 0.75], np.float32)
        idx = rng.integers(0, 4, (1, nkv, hd))
        idx[..., ::32] = 0
        idx[..., 1::32] = 3
        c = lv[idx]
    V = np.broadcast_to(c, (T, nkv, hd)).copy()
    backend.gpu_kv_write_batch(0, 0, K.reshape(T, -1), V.reshape(T, -1))
    q = rng.standard_normal(nh * hd).astype(np.float32)
    got = backend.grouped_query_attention_from_gpu_cache(q, 0, T).reshape(nh, hd)
    want = np.repeat(c[0], nh // nkv, axis=0)
    _close(got, want, rel=1e-5)
    # uniform keys: mean of V (cache form)
    K2 = np.zeros_like(K)
    V2 = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    backend.gpu_kv_write_batch(0, 0, K2.reshape(T, -1), V2.reshape(T, -1))
    got = backend.grouped_query_attention_from_gpu_cache(q, 0, T).reshape(nh, hd)
    _, Vv = oracle.kv_view(_mode(oracle, FMTS[fmt]), K2, V2)
    want = np.repeat(Vv.astype(np.float64).mean(axis=0), nh // nkv, axis=0)
    # the means of T unit-variance values sit near zero (~T^-1/2), so the
    # absolute floor is taken from the V magnitude, not the output's
    _close(got, want, rel=1e-3, absb=1e-6 * np.abs(Vv).mean())


@pytest.mark.parametrize("fmt", ["q8", "kivi"])
def test_greedy_tokens_quantized_kv(backend, oracle, fmt):
    """The decode step quantizes the new token itself (and, for KIVI, the
    groups leaving the window at T = 161, 193); 150-token prompt + 64 tokens
    on the Q8_0 tiny model: identical streams."""
    spec = S.tiny_spec(FL_Q8_0, max_seq=256)
    print(f"[kv-greedy] {fmt}", flush=True)
    model = S.make_model(spec, seed=4)
    prompt = S.random_tokens(104, 150, spec.vocab)
    backend.init_gpu_kv_cache(spec, FMTS[fmt])
    backend.upload_weights_to_gpu(model)
    got = backend.generate(prompt, 64)
    want = oracle.OracleModel(model, _mode(oracle, FMTS[fmt])).generate(prompt, 64)
    assert got.tolist() == want.tolist()


# Q4_K layers quantize the RMS-normed activations to Q8_0 before every
# matvec (model.rs:2040-2095): one int8 rounding flip (from a last-ulp
# difference in a row sum) moves the tiny model's logits by ~0.5 % at a
# 150-token context, enough to flip a near-tie.  Checked teacher-forced: the
# graph-replayed decode step must pick the oracle's token wherever the
# oracle's top-2 gap exceeds this margin (relative to the top logit).
Q4K_MARGIN = 2e-2


@pytest.mark.parametrize("fmt", ["q8", "kivi", "f16"])
def test_greedy_q4k_quantized_kv_teacher_forced(backend, oracle, fmt):
    spec = S.tiny_spec(FL_Q4K, max_seq=256, embed_fmt=FL_Q6K, output_fmt=FL_Q6K)
    print(f"[kv-teacher-forced] q4k {fmt}", flush=True)
    model = S.make_model(spec, seed=4)
    prompt = S.random_tokens(104, 150, spec.vocab)
    backend.init_gpu_kv_cache(spec, FMTS[fmt])
    backend.upload_weights_to_gpu(model)
    mode = _mode(oracle, FMTS[fmt])
    om, ol = oracle.OracleModel(model, mode), oracle.OracleModel(model, mode)
    toks = list(prompt)
    checked = 0
    for pos in range(len(prompt) + 63):
        t, v = backend.forward_greedy(int(toks[pos]), pos)
        ot, ov = om.forward_greedy(int(toks[pos]), pos)
        logits = ol.forward_logits(int(toks[pos]), pos)
        top2 = np.sort(logits)[-2:]
        assert abs(v - ov) <= 2e-2 * abs(ov), (pos, v, ov)
        if top2[1] - top2[0] > Q4K_MARGIN * abs(top2[1]):
            assert t == ot, (pos, t, ot)
            checked += 1
        if pos >= len(prompt) - 1:
            toks.append(ot)
    assert checked >= 100
