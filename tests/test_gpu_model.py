"""End-to-end greedy decode parity on the GPU against the CPU oracle.

Bar (north star): greedy token streams identical for the first 64 tokens.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

# Output projections taking the f32 final_normed vector (tied embedding,
# Q6_K output: matvec_argmax_f32, model.rs:1917-1931) -- the paths of every
# BASELINE config.  Streams must be identical.
TINY = {
    "q8_tied": (S.tiny_spec(FL_Q8_0), None),
    "q4k_q6k_out": (S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K), None),
    "q8_gqa3_hd128": (S.tiny_spec(FL_Q8_0, heads=6, kv_heads=2, head_dim=128, hidden=512, inter=768), None),
}
# Raw Q8_0 / Q4_K output weights take the Q8-quantized final_normed
# (model.rs:1899-1916).  One rounding flip of that quantization (caused by a
# last-ulp difference in x, since the GPU sums row terms in a different order)
# moves a logit by ~1e-3 relative, so these are checked teacher-forced: the
# GPU argmax must equal the oracle's wherever the oracle's top-2 gap exceeds
# QOUT_MARGIN (relative to the top logit).
QOUT = {
    "q8_untied_q8out": S.tiny_spec(FL_Q8_0, output_fmt=FL_Q8_0),
    "q4k_q4k_out": S.tiny_spec(FL_Q4K, output_fmt=FL_Q4K),
}
QOUT_MARGIN = 5e-3


def _run(backend, oracle, spec, kv, seed, n_prompt, n_gen):
    model = S.make_model(spec, seed=seed)
    prompt = S.random_tokens(seed + 100, n_prompt, spec.vocab)
    backend.init_gpu_kv_cache(spec, kv)
    backend.upload_weights_to_gpu(model)
    got = backend.generate(prompt, n_gen)
    om = oracle.OracleModel(model, oracle.OR_KV_F16 if kv == FL_KV_F16 else oracle.OR_KV_F32)
    want = om.generate(prompt, n_gen)
    return got, want, model, prompt


@pytest.mark.parametrize("name", list(TINY))
@pytest.mark.parametrize("kv", [FL_KV_F32, FL_KV_F16])
def test_greedy_tokens_tiny(backend, oracle, name, kv):
    spec, _ = TINY[name]
    print(f"[greedy] {name} kv={kv}", flush=True)
    got, want, _, _ = _run(backend, oracle, spec, kv, seed=3, n_prompt=12, n_gen=64)
    assert got.tolist() == want.tolist()


@pytest.mark.parametrize("name", list(QOUT))
def test_greedy_quantized_output_teacher_forced(backend, oracle, name):
    spec = QOUT[name]
    print(f"[teacher-forced] {name}", flush=True)
    model = S.make_model(spec, seed=3)
    prompt = S.random_tokens(103, 12, spec.vocab)
    backend.init_gpu_kv_cache(spec, FL_KV_F32)
    backend.upload_weights_to_gpu(model)
    om = oracle.OracleModel(model)
    ol = oracle.OracleModel(model)
    toks = list(prompt)
    checked = 0
    for pos in range(len(prompt) + 63):
        t, v = backend.forward_greedy(int(toks[pos]), pos)
        ot, ov = om.forward_greedy(int(toks[pos]), pos)
        logits = ol.forward_logits(int(toks[pos]), pos)
        top2 = np.sort(logits)[-2:]
        assert abs(v - ov) <= 1e-2 * abs(ov)
        if top2[1] - top2[0] > QOUT_MARGIN * abs(top2[1]):
            assert t == ot, (pos, t, ot)
            checked += 1
        if pos >= len(prompt) - 1:
            toks.append(ot)
    assert checked >= 40


def test_decode_step_matches_generate(backend, oracle):
    spec = TINY["q8_tied"][0]
    model = S.make_model(spec, seed=9)
    prompt = S.random_tokens(10, 5, spec.vocab)
    backend.init_gpu_kv_cache(spec, FL_KV_F32)
    backend.upload_weights_to_gpu(model)
    gen = backend.generate(prompt, 20)
    backend.reset()
    om = oracle.OracleModel(model)
    toks = list(prompt)
    steps = []
    for pos in range(len(prompt) + 19):
        t, v = backend.forward_greedy(int(toks[pos]), pos)
        ot, ov = om.forward_greedy(int(toks[pos]), pos)
        assert t == ot
        assert abs(v - ov) <= 1e-3 * abs(ov)
        if pos >= len(prompt) - 1:
            steps.append(t)
            toks.append(t)
    assert steps == gen.tolist()


def test_logits_match_oracle(backend, oracle):
    spec = TINY["q4k_q6k_out"][0]
    model = S.make_model(spec, seed=12)
    backend.init_gpu_kv_cache(spec, FL_KV_F32)
    backend.upload_weights_to_gpu(model)
    om = oracle.OracleModel(model)
    for pos, tok in enumerate([5, 77, 300, 2]):
        got = backend.forward_single_token_gpu(tok, pos)
        want = om.forward_logits(tok, pos)
        err = np.abs(got - want).max() / np.abs(want).max()
        assert err < 1e-3, err


def test_smollm2_config_c1_tokens(backend, oracle):
    """SmolLM2-135M shape, Q8_0, 32-token prompt, greedy 128."""
    spec = S.SMOLLM2_135M
    print("[greedy] SmolLM2-135M C1", flush=True)
    got, want, _, _ = _run(backend, oracle, spec, FL_KV_F32, seed=0, n_prompt=32, n_gen=128)
    assert got[:64].tolist() == want[:64].tolist()
    print(f"[greedy] C1 identical tokens: {int(np.cumprod(got == want).sum())}/128", flush=True)


def test_errors_are_reported(backend):
    from flarellm_amd import FlareError

    spec = TINY["q8_tied"][0]
    backend.init_gpu_kv_cache(spec, FL_KV_F32)
    with pytest.raises(FlareError, match="weights not uploaded"):
        backend.forward_greedy(1, 0)
    model = S.make_model(spec, seed=1)
    backend.upload_weights_to_gpu(model)
    with pytest.raises(FlareError, match="outside the KV cache"):
        backend.forward_greedy(1, spec.max_seq)
    with pytest.raises(FlareError, match="exceeds max_seq_len"):
        backend.generate(np.zeros(spec.max_seq, np.uint32), 4)
