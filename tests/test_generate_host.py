"""CPU checks of the generation loop's host parts and of their oracles.

* The sampling oracle (oracle/flare_oracle.c or_sample, a restatement of
  flare-core/src/sampling.rs) against the reference's own known answers
  (sampling.rs tests) and against what the mathematics fixes: the sampler is
  the inverse CDF of the truncated, renormalised distribution, so sweeping the
  uniform draw over [0, 1) must return each candidate for a fraction of the
  sweep equal to its probability.
* The product's n-gram cache (fl_ngram_*, flarellm_amd/csrc/generate.cpp)
  against the Python restatement of NgramCache (oracle/generate.py) and the
  reference's known answers (generate.rs:866-901).
* The Python Generator restatement: speculative generation equals plain
  greedy generation (generate.rs:950, test_speculative_output_matches_greedy)
  on an oracle model.
"""
import ctypes as C

import numpy as np
import pytest

from flarellm_amd import FL_KV_F32, FL_Q8_0
from flarellm_amd import synth as S
from oracle import generate as OG
from oracle import oracle as O


# ---- sampling oracle: known answers of sampling.rs's tests -----------------------
def test_sampling_known_answers():
    # test_greedy (sampling.rs:275), test_greedy_all_equal, test_greedy_negative_logits
    assert O.sample([1.0, 3.0, 2.0, 0.5], temperature=0.0) == 1
    assert O.sample([1.0, 1.0, 1.0, 1.0], temperature=0.0, repeat_penalty=1.0) == 0
    assert O.sample([-5.0, -1.0, -3.0, -0.5], temperature=0.0, repeat_penalty=1.0) == 3
    # test_top_p_deterministic_at_zero, test_top_p_full_considers_all
    assert O.sample([1.0, 10.0, 0.1], temperature=1.0, top_p=0.9, repeat_penalty=1.0, u=0.01) == 1
    assert O.sample([0.1, 10.0, 0.1], temperature=1.0, top_p=1.0, top_k=0, repeat_penalty=1.0, u=0.01) == 1
    # test_top_k, test_top_k_one_always_argmax, test_top_k_two_returns_one_of_top_two
    assert O.sample([1.0, 10.0, 0.1, 0.01], temperature=1.0, top_p=1.0, top_k=2, repeat_penalty=1.0,
                    u=0.01) in (0, 1)
    assert O.sample([1.0, 5.0, 2.0, 0.5], temperature=1.0, top_p=1.0, top_k=1, repeat_penalty=1.0, u=0.5) == 1
    for u in (0.01, 0.5, 0.99):
        assert O.sample([0.1, 10.0, 5.0, 0.01], temperature=1.0, top_p=1.0, top_k=2, repeat_penalty=1.0,
                        u=u) in (1, 2)
    # test_min_p_keeps_high_prob_tokens
    assert O.sample([0.01, 10.0, 0.01, 0.01], temperature=1.0, top_p=1.0, min_p=0.1, repeat_penalty=1.0,
                    u=0.01) == 1


def test_repeat_penalty_closed_form():
    """apply_repeat_penalty divides positive and multiplies negative logits,
    once per occurrence (sampling.rs:83-96; test_repeat_penalty_reduces_positive_logit)."""
    # token 2 (3.0) penalised twice by 2 -> 0.75 < token 1 (2.0): greedy picks 1
    assert O.sample([1.0, 2.0, 3.0], temperature=0.0, repeat_penalty=2.0, prev=[2, 2]) == 1
    # once: 1.5 < 2.0 as well; with penalty 1.2 once: 2.5 > 2.0 keeps token 2
    assert O.sample([1.0, 2.0, 3.0], temperature=0.0, repeat_penalty=1.2, prev=[2]) == 2
    # a negative logit becomes more negative: -1 * 3 = -3 < -2
    assert O.sample([-2.0, -1.0], temperature=0.0, repeat_penalty=3.0, prev=[1]) == 0
    # out-of-range previous tokens are ignored
    assert O.sample([1.0, 2.0], temperature=0.0, repeat_penalty=5.0, prev=[7]) == 1


def _sweep(logits, n_u=20000, **kw):
    us = (np.arange(n_u) + 0.5) / n_u
    counts = np.zeros(len(logits))
    for u in us:
        counts[O.sample(logits, u=float(u), **kw)] += 1
    return counts / n_u


def _probs(logits, temperature):
    x = np.asarray(logits, np.float64) / temperature
    e = np.exp(x - x.max())
    return e / e.sum()


@pytest.mark.parametrize("mode", ["top_p", "top_k", "min_p", "full"])
def test_sampler_is_inverse_cdf_of_truncated_distribution(mode):
    rng = np.random.default_rng(7)
    logits = rng.normal(0, 2.0, 40).astype(np.float32)
    T = 0.8
    p = _probs(logits, T)
    order = np.argsort(-p, kind="stable")
    keep = np.zeros_like(p, bool)
    if mode == "top_p":
        kw = dict(top_p=0.7, top_k=0, min_p=0.0)
        cum = np.cumsum(p[order])
        keep[order[:int(np.searchsorted(cum, 0.7)) + 1]] = True
    elif mode == "top_k":
        kw = dict(top_p=1.0, top_k=5, min_p=0.0)
        keep[order[:5]] = True
    elif mode == "min_p":
        kw = dict(top_p=1.0, top_k=0, min_p=0.1)
        keep = p >= 0.1 * p.max()
    else:
        kw = dict(top_p=1.0, top_k=0, min_p=0.0)
        keep[:] = True
    want = np.where(keep, p, 0.0)
    want /= want.sum()
    got = _sweep(logits, temperature=T, repeat_penalty=1.0, **kw)
    assert np.abs(got - want).max() < 3e-4, (mode, np.abs(got - want).max())
    assert (got[~keep] == 0).all()


def test_top_p_candidate_cap_512():
    """sample_top_p keeps at most INITIAL_K = 512 candidates (sampling.rs:143):
    with 2000 equal logits and top_p = 1 only the first 512 indices can be drawn."""
    logits = np.zeros(2000, np.float32)
    got = {O.sample(logits, temperature=1.0, top_p=1.0, top_k=0, repeat_penalty=1.0, u=float(u))
           for u in np.linspace(0.0005, 0.9995, 3000)}
    assert max(got) < 512 and len(got) > 500


# ---- n-gram cache: product vs restatement -------------------------------------------
def _lib():
    from flarellm_amd import _lib as L

    return L.load()


def _lookup(lib, h, toks):
    arr = np.ascontiguousarray(toks, np.uint32)
    out = np.zeros(8, np.uint32)
    n = lib.fl_ngram_lookup(h, arr.ctypes.data if arr.size else None, arr.size, out.ctypes.data)
    return [int(x) for x in out[:n]]


def test_ngram_known_answer():
    """test_ngram_cache_record_and_lookup (generate.rs:866-882)."""
    lib = _lib()
    h = lib.fl_ngram_create()
    try:
        toks = np.array([1, 2, 3, 4, 5], np.uint32)
        for i in range(1, 6):
            lib.fl_ngram_record(h, toks.ctypes.data, i)
        assert 5 in _lookup(lib, h, [3, 4])
        assert _lookup(lib, h, [4, 5]) == []
    finally:
        lib.fl_ngram_destroy(h)


def test_ngram_eviction():
    """test_ngram_cache_eviction (generate.rs:885-901)."""
    lib = _lib()
    h = lib.fl_ngram_create()
    try:
        toks = np.arange(10_000 + 101, dtype=np.uint32)
        for i in range(1, toks.size + 1):
            lib.fl_ngram_record(h, toks.ctypes.data, i)
        assert lib.fl_ngram_entries(h) <= 10_000
    finally:
        lib.fl_ngram_destroy(h)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ngram_matches_restatement(seed):
    """Random repetitive streams (small alphabet): every lookup of the
    product's cache equals the restatement's, across prompt seeding,
    incremental records and evictions."""
    lib = _lib()
    rng = np.random.default_rng(seed)
    h = lib.fl_ngram_create()
    ref = OG.NgramCache()
    try:
        prompt = rng.integers(0, 6, 40).tolist()
        arr = np.array(prompt, np.uint32)
        lib.fl_ngram_record_all(h, arr.ctypes.data, arr.size)
        ref.record_all(prompt)
        toks = list(prompt)
        for step in range(4000):
            assert _lookup(lib, h, toks) == ref.lookup(toks), step
            toks.append(int(rng.integers(0, 6 if step % 500 < 400 else 4000)))
            arr = np.array(toks, np.uint32)
            lib.fl_ngram_record(h, arr.ctypes.data, arr.size)
            ref.record(toks)
            assert lib.fl_ngram_entries(h) == ref.total_entries
    finally:
        lib.fl_ngram_destroy(h)


def test_params_default():
    """SamplingParams::default (sampling.rs:56-70)."""
    from flarellm_amd import _lib as L

    p = L.SamplingParams()
    _lib().fl_sampling_params_default(C.byref(p))
    assert (p.temperature, p.top_k, p.speculative) == (pytest.approx(0.7), 40, 1)
    assert p.top_p == pytest.approx(0.9) and p.repeat_penalty == pytest.approx(1.1) and p.min_p == 0.0


# ---- Generator restatement ---------------------------------------------------------
def test_speculative_restatement_matches_greedy():
    """test_speculative_output_matches_greedy (generate.rs:950) on the oracle:
    the speculative loop's tokens equal plain greedy's, and drafts were tried."""
    spec = S.tiny_spec(FL_Q8_0, max_seq=128)
    model = S.make_model(spec, seed=11)
    prompt = S.random_tokens(3, 6, spec.vocab).tolist()
    outs, stats = [], []
    for speculative in (False, True):
        om = O.OracleModel(model, O.OR_KV_F32)
        g = OG.Generator(om, OG.Params(temperature=0.0, repeat_penalty=1.0, speculative=speculative))
        outs.append(g.generate(prompt, 48))
        stats.append(g.stats)
        om.close()
    assert outs[0] == outs[1]
    assert stats[1].attempts > 0 and stats[1].accepted <= stats[1].drafted
