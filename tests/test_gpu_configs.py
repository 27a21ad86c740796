"""Production-mode parity at the BASELINE model shapes (not tiny stand-ins).

The production kernels sum rows, squares and softmax terms in tree order; the
reference sums them sequentially.  On these random-weight models that
difference alone is amplified (one flipped int8 code of a requantized
activation moves the logits by ~1 %), so the bar is set by a measuring stick
run in the same test: the CPU oracle with pairwise instead of sequential sums
(or_set_order(1) -- the reference's own arithmetic in another valid order).
The GPU's teacher-forced logits must stay within DRIFT_FACTOR times the
stick's drift from the reference, and its greedy token must equal the
reference's wherever the reference's top-2 gap exceeds that band.  Equality
with the reference is shown separately by the reference-order mode
(tests/test_gpu_exact.py: identical streams, bit-identical logits at C2/C3).

* C2 -- Llama-3.2-1B, Q8_0, tied embedding, fp16 KV (the benchmarked config).
* C3 -- Llama-3-8B, Q4_K layers, Q6_K embedding/output, fp16 KV.
* C5 -- the M=8 verify pass on the C3 model: against the oracle at a short
  context, against the GPU's sequential decode at context 1024 (fused and
  unfused GEMM epilogues identical).

The reference path: forward_greedy / forward_layers (flare-core/src/model.rs:
1872-1942, 1955-2561); speculative_step (flare-core/src/generate.rs:244-312).
"""
import time

import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_KV_Q8
from flarellm_amd import _lib as L
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

DRIFT_FACTOR = 2.0
DRIFT_FLOOR = 2e-3
# Verify against sequential decode at context 1024 (both GPU, two tree
# orders): no oracle at that length in test time.  The pairwise-vs-sequential
# oracle drift on the Llama-3-8B shape, measured on the CPU over 31
# teacher-forced positions, is up to 12.6 % (median 10 %) of the top logit;
# this band is twice the median.
VERIFY_BAND = 0.20


def _now():
    return time.perf_counter()


@pytest.fixture(scope="module")
def c3_model():
    t = _now()
    m = S.make_model(S.LLAMA3_8B, seed=2)
    print(f"[c3] model built in {_now() - t:.1f} s", flush=True)
    return m


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def _teacher_forced(backend, oracle, spec, model, prompt, n_steps, tag):
    """Teacher-forced on the reference's tokens: GPU, oracle (sequential) and
    oracle (pairwise) logits at every position."""
    backend.init_gpu_kv_cache(spec, FL_KV_F16)
    backend.upload_weights_to_gpu(model)
    ref, stick = oracle.OracleModel(model, oracle.OR_KV_F16), oracle.OracleModel(model, oracle.OR_KV_F16)
    toks = list(prompt)
    rows = []
    try:
        for pos in range(len(prompt) + n_steps - 1):
            t = int(toks[pos])
            got = backend.forward_single_token_gpu(t, pos)
            want = ref.forward_logits(t, pos)
            oracle.set_order(1)
            alt = stick.forward_logits(t, pos)
            oracle.set_order(0)
            rows.append((pos, got, want, alt))
            if pos >= len(prompt) - 1:
                toks.append(int(np.argmax(want)))
    finally:
        oracle.set_order(0)
    gdev = [_rel(g, w) for _, g, w, _ in rows]
    sdev = [_rel(a, w) for _, _, w, a in rows]
    band = DRIFT_FACTOR * max(sdev) + DRIFT_FLOOR
    print(f"[{tag}] gpu drift max {max(gdev):.3e} median {np.median(gdev):.3e}; pairwise-oracle drift max "
          f"{max(sdev):.3e} median {np.median(sdev):.3e}; band {band:.3e}", flush=True)
    assert max(gdev) <= band
    checked = 0
    for pos, g, w, _ in rows:
        top2 = np.sort(w)[-2:]
        if top2[1] - top2[0] > band * abs(top2[1]):
            assert int(np.argmax(g)) == int(np.argmax(w)), pos
            checked += 1
    flips = sum(int(np.argmax(g)) != int(np.argmax(w)) for _, g, w, _ in rows)
    sflips = sum(int(np.argmax(a)) != int(np.argmax(w)) for _, _, w, a in rows)
    print(f"[{tag}] argmax differs from the reference at {flips} / {len(rows)} positions (pairwise oracle: "
          f"{sflips}); {checked} positions outside the band agree", flush=True)
    return ref


@pytest.mark.timeout(900)
def test_c2_llama32_1b_production(backend, oracle):
    spec = S.LLAMA32_1B
    print("[c2] Llama-3.2-1B Q8_0 tied fp16-KV: 32-token prompt, 32 steps teacher-forced", flush=True)
    model = S.make_model(spec, seed=1)
    prompt = S.random_tokens(101, 32, spec.vocab)
    ref = _teacher_forced(backend, oracle, spec, model, prompt, 32, "c2")
    backend.reset()
    ref.reset()
    g, w = backend.generate(prompt, 64), ref.generate(prompt, 64)
    print(f"[c2] free-running identical prefix {int(np.cumprod(g == w).sum())}/64", flush=True)


@pytest.mark.timeout(900)
def test_c3_llama3_8b_production(backend, oracle, c3_model):
    spec = S.LLAMA3_8B
    print("[c3] Llama-3-8B Q4_K/Q6_K fp16-KV: 8-token prompt, 24 steps teacher-forced", flush=True)
    prompt = S.random_tokens(102, 8, spec.vocab)
    ref = _teacher_forced(backend, oracle, spec, c3_model, prompt, 24, "c3")
    backend.reset()
    ref.reset()
    g, w = backend.generate(prompt, 64), ref.generate(prompt, 64)
    print(f"[c3] free-running identical prefix {int(np.cumprod(g == w).sum())}/64", flush=True)


def _seq_logits(backend, drafts, pos0):
    return [backend.forward_single_token_gpu(int(t), pos0 + i) for i, t in enumerate(drafts)]


@pytest.mark.timeout(900)
def test_c5_verify_vs_oracle_short_context(backend, oracle, c3_model):
    """8 drafts after a 16-token context: the greedy token after each draft
    and its logit, against the oracle's forward at the same positions, within
    the pairwise-oracle band."""
    spec = S.LLAMA3_8B
    n_prompt, M = 16, 8
    prompt = S.random_tokens(104, n_prompt, spec.vocab)
    drafts = S.random_tokens(204, M, spec.vocab)
    backend.init_gpu_kv_cache(spec, FL_KV_F16)
    backend.upload_weights_to_gpu(c3_model)
    backend.generate(prompt, 1)
    got, vals = backend.verify(drafts, n_prompt)
    ref, stick = oracle.OracleModel(c3_model, oracle.OR_KV_F16), oracle.OracleModel(c3_model, oracle.OR_KV_F16)
    rows = []
    try:
        for pos, t in enumerate(list(prompt) + list(drafts)):
            w = ref.forward_logits(int(t), pos)
            oracle.set_order(1)
            a = stick.forward_logits(int(t), pos)
            oracle.set_order(0)
            if pos >= n_prompt:
                rows.append((w, a))
    finally:
        oracle.set_order(0)
    band = DRIFT_FACTOR * max(_rel(a, w) for w, a in rows) + DRIFT_FLOOR
    checked = 0
    for i, (w, _) in enumerate(rows):
        top2 = np.sort(w)[-2:]
        assert abs(vals[i] - w[got[i]]) <= band * abs(top2[1]), (i, vals[i], w[got[i]], band)
        if top2[1] - top2[0] > band * abs(top2[1]):
            assert got[i] == int(np.argmax(w)), i
            checked += 1
    print(f"[c5] verify vs oracle: band {band:.3e}; {checked}/{M} positions outside the band agree", flush=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("M,kv", [(8, FL_KV_F16), (5, FL_KV_F16), (8, FL_KV_F32), (8, FL_KV_Q8)])
def test_c5_verify_long_context(backend, oracle, c3_model, M, kv):
    """Context 1024 (several attention splits per query, K split > 1 in every
    GEMM): fused and unfused epilogues identical; verify against the GPU's
    sequential decode of the same drafts."""
    spec = S.LLAMA3_8B
    n_prompt = 1024
    prompt = S.random_tokens(105, n_prompt, spec.vocab)
    drafts = S.random_tokens(205 + M, M, spec.vocab)
    print(f"[c5] ctx {n_prompt} M={M} kv={kv}", flush=True)
    backend.init_gpu_kv_cache(spec, kv)
    backend.upload_weights_to_gpu(c3_model)
    backend.generate(prompt, 1)
    seq = _seq_logits(backend, drafts, n_prompt)
    got, vals = backend.verify(drafts, n_prompt)
    backend.set_option(L.FL_OPT_VERIFY_FUSE, 0)
    try:
        got2, vals2 = backend.verify(drafts, n_prompt)
    finally:
        backend.set_option(L.FL_OPT_VERIFY_FUSE, 1)
    assert got.tolist() == got2.tolist()
    assert vals.tolist() == vals2.tolist()
    checked = 0
    for i in range(M):
        top2 = np.sort(seq[i])[-2:]
        assert abs(vals[i] - seq[i][got[i]]) <= VERIFY_BAND * abs(top2[1]), (i, vals[i], seq[i][got[i]])
        if top2[1] - top2[0] > VERIFY_BAND * abs(top2[1]):
            assert got[i] == int(np.argmax(seq[i])), i
            checked += 1
    print(f"[c5] ctx {n_prompt} M={M}: {checked}/{M} clear positions agree with sequential decode", flush=True)
