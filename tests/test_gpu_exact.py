"""Reference-order mode (FL_OPT_EXACT): bit-identical to the CPU oracle.

With FL_OPT_EXACT the decode step folds every row sum block by block, sums
squares sequentially, runs the online softmax token by token and evaluates
expf as the host C library does -- the x86 reference's floating-point order
(flare-core/src/model.rs:5610-5640, 7456-7477, 8067-8102, 8969-9025,
9914-9966, 8668-8689).  The quantized matvecs are the production streaming
kernels (same tiles, loads, integer dots and per-block terms) with an in-order
fold.  So the bar here is equality: logits bit-identical and greedy streams
identical, at the BASELINE model shapes.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import _lib as L
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture
def exact(backend):
    backend.set_option(L.FL_OPT_EXACT, 1)
    yield backend
    backend.set_option(L.FL_OPT_EXACT, 0)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_silu_expf_bit_exact(backend, oracle):
    """silu_mul_into (model.rs:9783-9796) with the device expf against the
    oracle's (the host C library's expf): every element bit-identical over
    4M random inputs spanning the whole exp range, plus specials."""
    rng = np.random.default_rng(7)
    n = 1 << 22
    g = np.concatenate([
        rng.standard_normal(n // 4) * 4.0,
        rng.uniform(-110.0, 110.0, n // 4),
        rng.standard_normal(n // 4) * 1e-3,
        (rng.integers(0, 1 << 32, n // 4, dtype=np.uint64).astype(np.uint32)).view(np.float32),
    ]).astype(np.float32)
    g[:8] = [0.0, -0.0, np.inf, -np.inf, 88.72283, -103.97208, -87.33655, 1e-30]
    g = np.where(np.isnan(g), np.float32(1.0), g).astype(np.float32)
    u = np.ones_like(g)
    got = backend.silu_mul(_t(g), _t(u)).cpu().numpy()
    want = oracle.silu_mul(g, u)
    same = (_bits(got) == _bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} differ, first at g={g[~same][:4]}"


# (fmt, rows, cols): BASELINE matvec shapes (C2 Q8_0; C3 / C5 Q4_K)
EXACT_MATVECS = [
    (FL_Q8_0, 3072, 2048), (FL_Q8_0, 16384, 2048), (FL_Q8_0, 2048, 2048), (FL_Q8_0, 2048, 8192),
    (FL_Q4K, 6144, 4096), (FL_Q4K, 28672, 4096), (FL_Q4K, 4096, 4096), (FL_Q4K, 4096, 14336),
    (FL_Q8_0, 960, 576), (FL_Q8_0, 576, 1536),
]


@pytest.mark.parametrize("fmt,rows,cols", EXACT_MATVECS)
def test_exact_matvec_bit_exact(exact, oracle, fmt, rows, cols):
    """The streaming matvec with the in-order fold equals the oracle's
    matvec_q8_0_preq_into / matvec_q4k_q8_into bit for bit, so every
    per-block integer dot and per-block float term of the kernel is exact."""
    print(f"[exact-matvec] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows + cols, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = exact.upload(S.QWeight(w, fmt, rows, cols))
    q, s = oracle.quantize_q8(S.normal(cols + 1, 0, cols, 0.0, 1.0))
    su = q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32)
    got = exact.matvec_q8in(W, _t(q), _t(s), _t(su)).cpu().numpy()
    want = oracle.matvec(w, fmt, rows, cols, q, s)
    assert np.array_equal(_bits(got), _bits(want)), f"{(_bits(got) != _bits(want)).sum()} rows differ"


@pytest.mark.parametrize("n,order", [(576, 0), (2048, 0), (4096, 1), (14336, 1)])
def test_exact_rmsnorm_quantize_bit_exact(exact, oracle, n, order):
    x = S.normal(3 + n, 0, n, 0.0, 0.5)
    w = S.normal(5 + n, 0, n, 1.0, 0.1)
    q, s, _ = exact.rmsnorm_quantize_q8(_t(x), _t(w), 1e-5, order)
    if order == 0:
        qo, so = oracle.rmsnorm_quantize_q8(x, w, 1e-5)
    else:
        qo, so = oracle.quantize_q8(oracle.rmsnorm(x, w, 1e-5))
        assert np.array_equal(_bits(exact.rmsnorm(_t(x), _t(w), 1e-5).cpu().numpy()),
                              _bits(oracle.rmsnorm(x, w, 1e-5)))
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(_bits(s.cpu().numpy()), _bits(so))


def _ess_vectors(n, seed):
    """Vectors that stress the exact sum of squares: scales over 80 decades,
    zero runs, heavy tails, integer values (frequent ties), a constant, a
    tiny leading element, growing magnitudes."""
    rng = np.random.default_rng(seed)
    out = [rng.standard_normal(n) * 10.0 ** rng.uniform(-18, 18) for _ in range(6)]
    v = rng.standard_normal(n)
    v[: n // 3] = 0.0
    out.append(v)
    out.append(np.where(rng.random(n) < 0.01, rng.standard_normal(n) * 1e5, rng.standard_normal(n)))
    out.append(np.round(rng.standard_normal(n) * 8.0))
    out.append(np.ldexp(1.0, rng.integers(-10, 10, n)).astype(np.float64))
    out.append(np.full(n, 1.0 + 2.0 ** -20))
    v = rng.standard_normal(n)
    v[0] = 1e-30
    out.append(v)
    out.append(rng.standard_normal(n) * np.arange(1, n + 1))
    return [np.ascontiguousarray(v, np.float32) for v in out]


@pytest.mark.parametrize("n", [576, 1024, 2048, 3072, 4096])
def test_exact_sum_of_squares_stress(exact, oracle, n):
    """rmsnorm_into in reference order (the exact sum of squares of ess.h,
    workgroup form) over adversarial vectors: every output bit-identical to
    the oracle's sequential fold."""
    w = np.ones(n, np.float32)
    for i, x in enumerate(_ess_vectors(n, 100 + n)):
        got = exact.rmsnorm(_t(x), _t(w), 1e-5).cpu().numpy()
        want = oracle.rmsnorm(x, w, 1e-5)
        assert np.array_equal(_bits(got), _bits(want)), f"vector {i}: {(_bits(got) != _bits(want)).sum()} differ"


TINY = {
    "q8_tied": S.tiny_spec(FL_Q8_0),
    "q4k_q6k_out": S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K),
    "q8_untied_q8out": S.tiny_spec(FL_Q8_0, output_fmt=FL_Q8_0),
    "q4k_q4k_out": S.tiny_spec(FL_Q4K, output_fmt=FL_Q4K),
    "q8_gqa3_hd128": S.tiny_spec(FL_Q8_0, heads=6, kv_heads=2, head_dim=128, hidden=512, inter=768),
}


def _omode(oracle, kv):
    return oracle.OR_KV_F16 if kv == FL_KV_F16 else oracle.OR_KV_F32


@pytest.mark.parametrize("name", list(TINY))
@pytest.mark.parametrize("kv", [FL_KV_F32, FL_KV_F16])
def test_exact_tiny_logits_and_tokens(exact, oracle, name, kv):
    spec = TINY[name]
    print(f"[exact] {name} kv={kv}", flush=True)
    model = S.make_model(spec, seed=3)
    prompt = S.random_tokens(103, 12, spec.vocab)
    exact.init_gpu_kv_cache(spec, kv)
    exact.upload_weights_to_gpu(model)
    om = oracle.OracleModel(model, _omode(oracle, kv))
    for pos in range(20):
        tok = int(prompt[pos]) if pos < len(prompt) else int(np.argmax(want))
        got = exact.forward_single_token_gpu(tok, pos)
        want = om.forward_logits(tok, pos)
        assert np.array_equal(_bits(got), _bits(want)), (pos, int((_bits(got) != _bits(want)).sum()))
    exact.reset()
    om.reset()
    assert exact.generate(prompt, 64).tolist() == om.generate(prompt, 64).tolist()


def _stream_and_logits(exact, oracle, spec, model, prompt, n_gen, kv, check_pos):
    exact.init_gpu_kv_cache(spec, kv)
    exact.upload_weights_to_gpu(model)
    got = exact.generate(prompt, n_gen)
    om = oracle.OracleModel(model, _omode(oracle, kv))
    want = om.generate(prompt, n_gen)
    same = int(np.cumprod(got == want).sum())
    print(f"[exact] {spec.name}: identical prefix {same}/{n_gen}", flush=True)
    assert got.tolist() == want.tolist()
    # logits of the next step after the stream, bit for bit
    exact.reset()
    om.reset()
    toks = list(prompt) + want.tolist()
    for pos in range(check_pos):
        t = int(toks[pos])
        if pos < check_pos - 2:
            exact.forward_greedy(t, pos)
            om.forward_greedy(t, pos)
            continue
        g = exact.forward_single_token_gpu(t, pos)
        w = om.forward_logits(t, pos)
        assert np.array_equal(_bits(g), _bits(w)), (pos, int((_bits(g) != _bits(w)).sum()))


@pytest.mark.timeout(900)
def test_exact_c1_smollm2(exact, oracle):
    spec = S.SMOLLM2_135M
    model = S.make_model(spec, seed=0)
    prompt = S.random_tokens(100, 32, spec.vocab)
    _stream_and_logits(exact, oracle, spec, model, prompt, 128, FL_KV_F32, 40)


@pytest.mark.timeout(900)
def test_exact_c2_llama32_1b(exact, oracle):
    """BASELINE C2 (the benchmarked config): 64 greedy tokens after a
    32-token prompt identical to the oracle, logits bit-identical."""
    spec = S.LLAMA32_1B
    model = S.make_model(spec, seed=1)
    prompt = S.random_tokens(101, 32, spec.vocab)
    _stream_and_logits(exact, oracle, spec, model, prompt, 64, FL_KV_F16, 40)


@pytest.mark.timeout(900)
def test_exact_c3_llama3_8b(exact, oracle):
    """BASELINE C3 (Llama-3-8B Q4_K / Q6_K output): 64 greedy tokens
    identical to the oracle, logits bit-identical."""
    spec = S.LLAMA3_8B
    model = S.make_model(spec, seed=2)
    prompt = S.random_tokens(102, 8, spec.vocab)
    _stream_and_logits(exact, oracle, spec, model, prompt, 64, FL_KV_F16, 12)
