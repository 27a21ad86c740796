"""Pins the CPU oracle (oracle/flare_oracle.c) before it is trusted as the
parity reference of the HIP path.

Every function of the oracle is checked against at least one of:
  * the reference's own golden vectors / known-answer tests (cited file:line),
  * an independent formulation (numpy float64 matrix form, numpy's IEEE
    binary16 conversion, closed forms),
  * invariants the mathematics fixes (RoPE at position 0, norm preservation,
    softmax of equal scores, GQA head mapping, round-half-away ties).
A plausible mistake (a dropped min term, a swapped nibble, an interleaved
RoPE pairing, a wrong GQA group) fails one of these.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f16bits(v: float) -> tuple:
    b = int(np.array(v, np.float16).view(np.uint16))
    return b & 0xFF, b >> 8


# ---------------------------------------------------------------- f16 ------
def test_f16_to_f32_exhaustive(oracle):
    """or_f16_to_f32 (quantize.rs f16_to_f32) vs numpy binary16 for all 65536
    bit patterns; NaN stays NaN (quantize.rs:887-960)."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # incl. -0.0


def test_f16_known_answers(oracle):
    """quantize.rs:887-960 known answers."""
    v = oracle.f16_to_f32(np.array([0x3C00, 0x0000, 0xBC00, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x0001, 0x7BFF,
                                    0x4000, 0x3800], np.uint16))
    assert v[0] == 1.0 and v[1] == 0.0 and v[2] == -1.0
    assert v[3] == 0.0 and np.signbit(v[3])
    assert np.isposinf(v[4]) and np.isneginf(v[5]) and np.isnan(v[6])
    assert 0 < v[7] < 1e-4 and v[8] == 65504.0 and v[9] == 2.0 and v[10] == 0.5


def test_f32_to_f16_rne(oracle):
    """or_f32_to_f16_rne vs numpy (IEEE round-to-nearest-even) on random,
    tie, overflow and subnormal inputs."""
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000), rng.normal(0, 3e4, 5000),
        # exact ties between two f16 neighbours
        (np.arange(1024, 2048, dtype=np.float64) + 0.5) / 1024.0,
        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 2.9e-8, np.inf, -np.inf],
    ]).astype(np.float32)
    ours = oracle.f32_to_f16(vals)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------- dequant --------
def test_q4k_real_block_golden(oracle):
    """flare-loader/tests/q4k_real_model.rs: a real SmolLM2 Q4_K block and
    llama.cpp-computed values (fixture written by tests/golden/make_golden.py)."""
    g = json.load(open(os.path.join(GOLDEN, "q4k_real_block.json")))
    out = oracle.dequant(np.array(g["block"], np.uint8), oracle.OR_Q4K, 1, 256).ravel()
    assert np.all(np.abs(out[0:8] - g["expected_0_8"]) < g["tolerance"])
    assert np.all(np.abs(out[128:136] - g["expected_128_136"]) < g["tolerance"])


# (format, block bytes set {offset: value}, output index, expected) from
# flare-loader/src/quantize.rs:1259-1490 and 1608-1690.
KNOWN = [
    ("q8_0", {0: 0x00, 1: 0x3C, 2: 42}, 0, 42.0),
    ("q8_0", {0: 0x00, 1: 0x3C, 2: 0x80}, 0, -128.0),
    ("q8_0", {0: 0x00, 1: 0x3C, 3: 0xFF}, 1, -1.0),
    ("q8_0", {0: 0x00, 1: 0xC0, 2: 0x02}, 0, -4.0),
    ("q8_0", {0: 0x00, 1: 0x00, 2: 0x7F}, 0, 0.0),
    ("q4k", {1: 0x3C, 4: 0x02, 16: 0x04}, 0, 8.0),
    ("q4k", {1: 0x3C, 3: 0x3C, 4: 0x02, 8: 0x03}, 0, -3.0),
    ("q4k", {1: 0x3C, 4: 0x40, 12: 0x01, 16: 0x30}, 128, 15.0),
    ("q4k", {1: 0xBC, 4: 0x03, 16: 0x02}, 0, -6.0),
    ("q4k", {1: 0x3C, 5: 0x04, 48: 0x05}, 32, 20.0),
    ("q6k", {209: 0x3C, 192: 0x01, 0: 0x01}, 0, -31.0),
    ("q6k", {209: 0x3C, 192: 0x01, 128: 0x03}, 0, 16.0),
    ("q6k", {209: 0x3C, 192: 0xFF, 0: 0x01}, 0, 31.0),
    ("q6k", {209: 0x3C, 200: 0x02, 64: 0x01}, 128, -62.0),
]


@pytest.mark.parametrize("case", range(len(KNOWN)))
def test_dequant_known_answers(oracle, case):
    fmt, sets, idx, want = KNOWN[case]
    f, size, n = {"q8_0": (oracle.OR_Q8_0, 34, 32), "q4k": (oracle.OR_Q4K, 144, 256),
                  "q6k": (oracle.OR_Q6K, 210, 256)}[fmt]
    blk = np.zeros(size, np.uint8)
    for k, v in sets.items():
        blk[k] = v
    out = oracle.dequant(blk, f, 1, n).ravel()
    assert abs(out[idx] - want) < 1e-4


def test_dequant_zero_blocks(oracle):
    for f, size in ((oracle.OR_Q8_0, 34), (oracle.OR_Q4K, 144), (oracle.OR_Q6K, 210)):
        n = 32 if f == oracle.OR_Q8_0 else 256
        assert np.all(oracle.dequant(np.zeros(size, np.uint8), f, 1, n) == 0.0)


def test_q8_0_values_ramp(oracle):
    """quantize.rs test_dequant_q8_0: scale 1.0, values 0..31."""
    blk = np.concatenate([[0x00, 0x3C], np.arange(32)]).astype(np.uint8)
    assert np.array_equal(oracle.dequant(blk, oracle.OR_Q8_0, 1, 32).ravel(), np.arange(32, dtype=np.float32))


def test_unpack_q4k_scales_bitfields(oracle):
    """flarellm's 6-bit scale/min packing: sc[i] = raw[i] & 63, mn[i] =
    raw[i+4] & 63, sc[i+4] = raw[i] >> 6 | (raw[i+8] & 15) << 2, mn[i+4] =
    raw[i+4] >> 6 | (raw[i+8] >> 4) << 2 (the quantize.rs:1440-1462 known
    answer: raw[0]=0x40, raw[8]=0x01 -> sc[4]=5)."""
    sc, mn = oracle.unpack_q4k_scales(bytes([0x40, 0, 0, 0, 0, 0, 0, 0, 0x01, 0, 0, 0]))
    assert sc[4] == 5 and sc[0] == 0
    rng = np.random.default_rng(3)
    for _ in range(50):
        raw = rng.integers(0, 256, 12).astype(np.uint8)
        sc, mn = oracle.unpack_q4k_scales(bytes(raw))
        for j in range(8):
            assert 0 <= sc[j] < 64 and 0 <= mn[j] < 64
        # sub-blocks 0..3 and 4..7 use disjoint bits: flipping raw[8..12]
        # changes only sc/mn 4..7
        raw2 = raw.copy()
        raw2[8:12] ^= 0xFF
        sc2, mn2 = oracle.unpack_q4k_scales(bytes(raw2))
        assert sc2[:4] == sc[:4] and mn2[:4] == mn[:4]
        for i in range(4):
            assert sc[i + 4] == (raw[i] >> 6) | ((raw[i + 8] & 15) << 2)
            assert mn[i + 4] == (raw[i + 4] >> 6) | ((raw[i + 8] >> 4) << 2)


# ------------------------------------------------------- quantize ----------
def test_quantize_q8_closed_form(oracle):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 32 * 64).astype(np.float32)
    x[32:64] = 0.0  # all-zero block
    q, s = oracle.quantize_q8(x)
    xb, qb = x.reshape(-1, 32), q.reshape(-1, 32).astype(np.int32)
    amax = np.abs(xb).max(1)
    assert s[1] == 0.0 and np.all(qb[1] == 0)
    nz = amax > 0
    assert np.allclose(s[nz], amax[nz] / 127.0, rtol=1e-7)
    # the largest-magnitude element maps to +-127
    i = np.abs(xb).argmax(1)
    assert np.all(np.abs(qb[nz, i[nz]]) == 127)
    # error <= half a step
    assert np.all(np.abs(qb * s[:, None] - xb) <= s[:, None] * 0.5 * (1 + 1e-5) + 1e-12)


def test_quantize_q8_round_half_away(oracle):
    """model.rs:5557-5570 rounds with f32::round (half away from zero): with
    amax = 127 the step is exactly 1 and +-2.5 -> +-3, +-0.5 -> +-1."""
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49]
    q, s = oracle.quantize_q8(x)
    assert s[0] == 1.0
    assert list(q[:6]) == [127, 3, -3, 1, -1, 1]


def test_rmsnorm_reference_case(oracle):
    """model.rs:10219-10232: rmsnorm([1,2,3,4], ones)."""
    out = oracle.rmsnorm(np.array([1, 2, 3, 4] * 8, np.float32), np.ones(32, np.float32), 1e-5)
    rms = np.sqrt(30.0 / 4.0 + 1e-5)
    assert np.allclose(out[:4], np.arange(1, 5) / rms, atol=1e-4)


def test_rmsnorm_vs_float64(oracle):
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, 2048).astype(np.float32)
    w = rng.normal(1, 0.1, 2048).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w
    assert np.allclose(oracle.rmsnorm(x, w, 1e-5), ref, rtol=1e-5, atol=1e-6)


def test_rmsnorm_quantize_matches_two_step(oracle):
    """model.rs:12302 test_rmsnorm_quantize_q8_0_matches_two_step: fused
    norm+quantize equals rmsnorm then quantize within one quantum."""
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, 1024).astype(np.float32)
    w = rng.normal(1, 0.2, 1024).astype(np.float32)
    q1, s1 = oracle.rmsnorm_quantize_q8(x, w, 1e-5)
    q2, s2 = oracle.quantize_q8(oracle.rmsnorm(x, w, 1e-5))
    assert np.allclose(s1, s2, rtol=1e-5)
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1


# --------------------------------------------------- dots / matvec --------
def _q8_weights(rng, rows, cols):
    from flarellm_amd import synth as S

    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    return S.quantize(w, 1)


def _q8_ints(data, rows, cols):
    b = data.reshape(rows, cols // 32, 34)
    return b[:, :, 2:].view(np.int8).astype(np.int64).reshape(rows, cols)


def test_block_dots_q8_0_bruteforce(oracle):
    rng = np.random.default_rng(5)
    rows, cols = 7, 256
    w = _q8_weights(rng, rows, cols)
    q = rng.integers(-128, 128, cols).astype(np.int8)
    got = oracle.block_dots(w, oracle.OR_Q8_0, rows, cols, q)
    ref = (_q8_ints(w, rows, cols) * q.astype(np.int64)).reshape(rows, cols // 32, 32).sum(2)
    assert np.array_equal(got, ref)


def test_block_dots_q4k_vs_unit_scale_dequant(oracle):
    """With d = 1, dmin = 0 and every 6-bit scale 1, dequant returns the raw
    nibble of each weight (layout pinned by the known answers above); the
    per-sub-block int dots must equal nibble . q8 over that sub-block."""
    rng = np.random.default_rng(6)
    rows, nsb = 3, 2
    blk = np.zeros((rows, nsb, 144), np.uint8)
    blk[:, :, 1] = 0x3C  # d = 1.0
    blk[:, :, 4:8] = 0x41  # sc[0..3] = 1 (low 6 bits), sc[4..7] = 1 (top 2 bits)
    blk[:, :, 16:] = rng.integers(0, 256, (rows, nsb, 128))
    data = blk.ravel()
    cols = nsb * 256
    nib = oracle.dequant(data, oracle.OR_Q4K, rows, cols).astype(np.int64)
    assert nib.min() >= 0 and nib.max() <= 15 and np.all(nib == np.round(nib))
    q = rng.integers(-128, 128, cols).astype(np.int8)
    got = oracle.block_dots(data, oracle.OR_Q4K, rows, cols, q)
    sub = (nib * q.astype(np.int64)).reshape(rows, nsb, 8, 32).sum(3)
    # per super-block the dots are stored as (sub c, sub c+4) pairs:
    # low nibbles of qs[32c..32c+32], then their high nibbles
    ref = np.stack([sub[:, :, :4], sub[:, :, 4:]], axis=3).reshape(rows, nsb * 8)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("fmt", ["q8_0", "q4k"])
def test_matvec_vs_dequant_float64(oracle, fmt):
    """Quantized matvec == dequant(W) @ dequant(x_q8) in float64 (the
    reference's own test_matvec_q8_0_vs_dequant_f32 / q4k_q8_matches_f32_path,
    model.rs:11668, 12038), including the Q4_K min term."""
    from flarellm_amd import synth as S

    rng = np.random.default_rng(7)
    f = oracle.OR_Q8_0 if fmt == "q8_0" else oracle.OR_Q4K
    rows, cols = 64, 1024
    w = S.quantize(rng.normal(0, 0.02, (rows, cols)).astype(np.float32), f)
    x = rng.normal(0, 1, cols).astype(np.float32)
    q, s = oracle.quantize_q8(x)
    got = oracle.matvec(w, f, rows, cols, q, s)
    xd = (q.astype(np.float64).reshape(-1, 32) * s[:, None]).ravel()
    ref = oracle.dequant(w, f, rows, cols).astype(np.float64) @ xd
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("fmt", ["q8_0", "q4k"])
def test_matvec_argmax_matches_full_matvec(oracle, fmt):
    """model.rs:11949 / 12075: fused argmax == argmax of the full matvec."""
    from flarellm_amd import synth as S

    rng = np.random.default_rng(8)
    f = oracle.OR_Q8_0 if fmt == "q8_0" else oracle.OR_Q4K
    rows, cols = 500, 512
    w = S.quantize(rng.normal(0, 0.02, (rows, cols)).astype(np.float32), f)
    q, s = oracle.quantize_q8(rng.normal(0, 1, cols).astype(np.float32))
    full = oracle.matvec(w, f, rows, cols, q, s)
    idx, val = oracle.matvec_argmax(w, f, rows, cols, q, s)
    assert idx == int(np.argmax(full)) and val == full[idx]


def test_matvec_f32_and_argmax_first_max(oracle):
    rng = np.random.default_rng(9)
    m = rng.normal(0, 1, (300, 96)).astype(np.float32)
    v = rng.normal(0, 1, 96).astype(np.float32)
    assert np.allclose(oracle.matvec_f32(m, v), m.astype(np.float64) @ v, rtol=1e-5, atol=1e-5)
    m[17] = m[5] = m[200] = 10.0  # three identical maximal rows
    idx, val = oracle.matvec_argmax_f32(m, np.abs(v))
    assert idx == 5


# ----------------------------------------------------------- rope ---------
def test_rope_position_zero_identity(oracle):
    """model.rs:10934 test_rope_zero_position."""
    d = np.arange(1, 9, dtype=np.float32)
    assert np.array_equal(oracle.apply_rope(d, 2, 4, 0, 10000.0), d)


def test_rope_preserves_norm(oracle):
    """model.rs:10354 test_rope_preserves_magnitude, per head."""
    rng = np.random.default_rng(10)
    d = rng.normal(0, 1, 4 * 64).astype(np.float32)
    for pos in (1, 7, 1000, 4095):
        r = oracle.apply_rope(d, 4, 64, pos, 500000.0).reshape(4, 64)
        assert np.allclose(np.linalg.norm(r, axis=1), np.linalg.norm(d.reshape(4, 64), axis=1), rtol=1e-5)


def test_rope_rotate_half_pairing(oracle):
    """Rotate-half convention (model.rs:7283-7296): element i pairs with
    i + D/2 at frequency theta^(-2i/D).  A unit vector on element 0 at
    position p becomes (cos p, ..., sin p at D/2)."""
    D = 8
    for pos in (1, 3, 10):
        e = np.zeros(D, np.float32)
        e[0] = 1.0
        r = oracle.apply_rope(e, 1, D, pos, 10000.0)
        ref = np.zeros(D)
        ref[0], ref[D // 2] = np.cos(pos), np.sin(pos)
        assert np.allclose(r, ref, atol=1e-6)
        # element 1 rotates with frequency theta^(-2/D)
        e = np.zeros(D, np.float32)
        e[1 + D // 2] = 1.0
        r = oracle.apply_rope(e, 1, D, pos, 10000.0)
        a = pos * 10000.0 ** (-2.0 / D)
        ref = np.zeros(D)
        ref[1], ref[1 + D // 2] = -np.sin(a), np.cos(a)
        assert np.allclose(r, ref, atol=1e-6)


def test_silu_mul_closed_form(oracle):
    rng = np.random.default_rng(11)
    g = rng.normal(0, 3, 4096).astype(np.float32)
    u = rng.normal(0, 1, 4096).astype(np.float32)
    g64 = g.astype(np.float64)
    assert np.allclose(oracle.silu_mul(g, u), g64 / (1 + np.exp(-g64)) * u, rtol=1e-5, atol=1e-7)


# ------------------------------------------------------- attention --------
def attention_f64(q, k, v, nh, nkv, D, T):
    """Multi-pass softmax attention in float64 (the structure of
    model.rs:10369 reference_attention)."""
    q = q.reshape(nh, D).astype(np.float64)
    k = k.reshape(-1, nkv, D)[:T].astype(np.float64)
    v = v.reshape(-1, nkv, D)[:T].astype(np.float64)
    out = np.zeros((nh, D))
    g = nh // nkv
    for h in range(nh):
        s = k[:, h // g, :] @ q[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, h // g, :]
    return out.ravel()


@pytest.mark.parametrize("nh,nkv,D,T", [(4, 2, 64, 1), (4, 2, 64, 37), (8, 8, 32, 100), (6, 2, 128, 300),
                                         (32, 8, 64, 513)])
def test_gqa_attention_vs_float64(oracle, nh, nkv, D, T):
    rng = np.random.default_rng(nh * 1000 + T)
    S = T + 5
    q = rng.normal(0, 1, nh * D).astype(np.float32)
    k = rng.normal(0, 1, S * nkv * D).astype(np.float32)
    v = rng.normal(0, 1, S * nkv * D).astype(np.float32)
    got = oracle.gqa_attention(q, k, v, nh, nkv, D, T)
    assert np.allclose(got, attention_f64(q, k, v, nh, nkv, D, T), rtol=1e-4, atol=1e-5)


def test_gqa_attention_invariants(oracle):
    nh, nkv, D, T = 6, 3, 16, 9
    rng = np.random.default_rng(12)
    q = rng.normal(0, 1, nh * D).astype(np.float32)
    v = rng.normal(0, 1, (T, nkv, D)).astype(np.float32)
    # all-zero keys: uniform softmax -> mean of the values of the head's group
    out = oracle.gqa_attention(q, np.zeros(T * nkv * D, np.float32), v.ravel(), nh, nkv, D, T).reshape(nh, D)
    for h in range(nh):
        assert np.allclose(out[h], v[:, h // 2, :].mean(0), atol=1e-6)
    # one token: output is that token's value row
    out = oracle.gqa_attention(q, rng.normal(0, 1, T * nkv * D).astype(np.float32), v.ravel(), nh, nkv, D, 1)
    assert np.allclose(out.reshape(nh, D), v[0][np.arange(nh) // 2], atol=1e-7)


# ------------------------------------------------------------- KIVI -------
def test_kivi_pack_round_trip(oracle):
    """kv_cache.rs:813 / 924 (packing round trip): 2-bit codes, 4 per byte,
    low bits first; decoded value = code * scale + min, within half a step."""
    rng = np.random.default_rng(13)
    v = rng.normal(0, 1, 130).astype(np.float32)
    packed, s, m = oracle.kivi_quantize_to_packed(v)
    assert packed.size == 33
    codes = np.array([(packed[i // 4] >> ((i % 4) * 2)) & 3 for i in range(v.size)])
    assert m == v.min() and np.isclose(s, (v.max() - v.min()) / 3.0)
    assert np.all(np.abs(codes * s + m - v) <= s * 0.5 * (1 + 1e-5))
    assert codes[v.argmin()] == 0 and codes[v.argmax()] == 3


def test_kivi_constant_values_no_nan(oracle):
    """kv_cache.rs:902: constant input gives scale 0 and code 0, no NaN."""
    packed, s, m = oracle.kivi_quantize_to_packed(np.full(16, 0.75, np.float32))
    assert s == 0.0 and m == 0.75 and np.all(packed == 0)


# ------------------------------------------------------ whole model -------
def numpy_forward(model, tokens):
    """Independent float64 restatement of the decode loop on dequantized
    weights (no activation quantization): embed, per layer rmsnorm -> QKV ->
    rotate-half RoPE -> causal GQA softmax -> Wo residual -> rmsnorm ->
    SiLU(gate)*up -> down residual, final rmsnorm, output projection."""
    from oracle import oracle as O

    sp = model.spec
    H, D, nh, nkv = sp.hidden, sp.head_dim, sp.heads, sp.kv_heads
    dq = lambda w: O.dequant(w.data, w.fmt, w.rows, w.cols).astype(np.float64)  # noqa: E731
    emb = dq(model.embedding)
    out_w = emb if model.output is None else dq(model.output)
    layers = [[dq(w) for w in ws] for ws in model.layers]
    norm = lambda x, w: x / np.sqrt((x * x).mean() + sp.eps) * w  # noqa: E731
    half = D // 2
    inv = sp.theta ** (-np.arange(half) * 2.0 / D)

    def rope(x, n, pos):
        x = x.reshape(n, D).copy()
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        a, b = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half], x[:, half:] = a * c - b * s, a * s + b * c
        return x

    K = [[] for _ in layers]
    V = [[] for _ in layers]
    logits = []
    for pos, t in enumerate(tokens):
        x = emb[t].copy()
        for l, (wq, wk, wv, wo, wg, wu, wd) in enumerate(layers):
            h = norm(x, model.attn_norms[l])
            q = rope(wq @ h, nh, pos)
            K[l].append(rope(wk @ h, nkv, pos))
            V[l].append((wv @ h).reshape(nkv, D))
            k, v = np.stack(K[l]), np.stack(V[l])
            a = np.zeros((nh, D))
            for hh in range(nh):
                g = hh // (nh // nkv)
                sc = k[:, g, :] @ q[hh] / np.sqrt(D)
                p = np.exp(sc - sc.max())
                a[hh] = (p / p.sum()) @ v[:, g, :]
            x = x + wo @ a.ravel()
            h = norm(x, model.ffn_norms[l])
            gt, up = wg @ h, wu @ h
            x = x + wd @ (gt / (1 + np.exp(-gt)) * up)
        logits.append(out_w @ norm(x, model.output_norm))
    return np.array(logits)


@pytest.mark.parametrize("which", ["q8_tied", "q4k_q6k"])
def test_model_logits_vs_float64_forward(oracle, which):
    """Whole decode step of the oracle vs the independent float64 forward.
    The oracle quantizes activations to Q8_0 before every matvec (as the
    reference does), so logits agree to ~1 % of their spread, not bit-wise."""
    from flarellm_amd import synth as S

    if which == "q8_tied":
        spec = S.tiny_spec(S.FL_Q8_0, hidden=128, inter=256, vocab=300, max_seq=16, heads=4, kv_heads=2,
                           head_dim=32)
    else:
        spec = S.tiny_spec(S.FL_Q4K, embed_fmt=S.FL_Q6K, output_fmt=S.FL_Q6K, hidden=256, inter=512,
                           vocab=300, max_seq=16, heads=4, kv_heads=1, head_dim=64)
    spec = S.replace(spec, std=0.08)
    model = S.make_model(spec, seed=21)
    toks = S.random_tokens(3, 6, spec.vocab)
    ref = numpy_forward(model, toks)
    om = oracle.OracleModel(model, oracle.OR_KV_F32)
    got = np.array([om.forward_logits(int(t), i) for i, t in enumerate(toks)])
    om.close()
    for i in range(len(toks)):
        err = np.linalg.norm(got[i] - ref[i]) / np.linalg.norm(ref[i] - ref[i].mean())
        assert err < 0.03, (i, err)


def test_model_greedy_consistency(oracle):
    """forward_greedy returns argmax(forward_logits); generate == a loop of
    forward_greedy; F16 KV stays close to F32 KV; reset restarts."""
    from flarellm_amd import synth as S

    spec = S.tiny_spec(S.FL_Q8_0, vocab=256, max_seq=40)
    model = S.make_model(spec, seed=5)
    prompt = S.random_tokens(1, 5, spec.vocab)
    om = oracle.OracleModel(model, oracle.OR_KV_F32)
    gen = om.generate(prompt, 8)
    om.reset()
    tok = 0
    for i, t in enumerate(prompt):
        tok, _ = om.forward_greedy(int(t), i)
    seq = [tok]
    for j in range(7):
        tok, _ = om.forward_greedy(int(tok), len(prompt) + j)
        seq.append(tok)
    assert list(gen) == seq
    om.reset()
    for i, t in enumerate(prompt[:-1]):
        om.forward_greedy(int(t), i)
    lg = om.forward_logits(int(prompt[-1]), len(prompt) - 1)
    assert int(np.argmax(lg)) == gen[0]
    om.close()
    om16 = oracle.OracleModel(model, oracle.OR_KV_F16)
    om16.reset()
    for i, t in enumerate(prompt[:-1]):
        om16.forward_greedy(int(t), i)
    lg16 = om16.forward_logits(int(prompt[-1]), len(prompt) - 1)
    om16.close()
    assert np.max(np.abs(lg16 - lg)) < 1e-2 * np.abs(lg).max()


def test_q6k_layout_probes(oracle):
    """Q6_K positions beyond the reference's four known answers, from the
    llama.cpp layout flare-loader/src/quantize.rs:343-384 follows: within each
    128-weight half, weight l (l < 32) takes ql[l] low nibble + qh[l] bits
    0-1, weight l+32 ql[l+32] low + bits 2-3, weight l+64 ql[l] high + bits
    4-5, weight l+96 ql[l+32] high + bits 6-7; scale index = l/16 + 2k."""
    def block(**sets):
        b = np.zeros(210, np.uint8)
        b[209] = 0x3C  # d = 1.0
        b[192:208] = 1  # all 16 scales = 1
        for k, v in sets.items():
            b[int(k[1:])] = v
        return oracle.dequant(b, oracle.OR_Q6K, 1, 256).ravel()

    base = block()
    assert np.all(base == -32.0)
    probes = [  # (byte offset, value, changed weight, expected)
        (32, 0x0F, 32, -17.0), (0, 0xF0, 64, -17.0), (32, 0xF0, 96, -17.0),
        (128, 0x0C, 32, 16.0), (128, 0x30, 64, 16.0), (128, 0xC0, 96, 16.0),
        (64 + 5, 0x01, 128 + 5, -31.0), (64 + 32 + 5, 0x10, 128 + 96 + 5, -31.0),
        (128 + 32 + 7, 0x30, 128 + 64 + 7, 16.0),
    ]
    for off, val, idx, want in probes:
        out = block(**{f"b{off}": val})
        changed = np.nonzero(out != base)[0]
        assert list(changed) == [idx] and out[idx] == want, (off, val, changed)
    # scales: 16 per block, scale s covers weights 16*s .. 16*s+16 in order
    for sidx in range(16):
        out = block(**{f"b{192 + sidx}": 3})
        changed = np.nonzero(out != base)[0]
        half, k = divmod(sidx, 8)
        start = half * 128 + (k // 2) * 32 + (k % 2) * 16
        assert list(changed) == list(range(start, start + 16)), sidx


# ---- KV forms of the long-context attention benchmark (Q8, KIVI 2-bit) ------
# No reference implementation exists for these forms; they are pinned by
# closed forms, the quantize_to_packed known answers of kv_cache.rs's own
# tests (exact codes 0..3, constant input -> no NaN) and error bounds.

def test_kivi32_qlen_closed_form(oracle):
    assert [oracle.kivi32_qlen(T) for T in (1, 128, 129, 130, 160, 161, 192, 193)] == [0, 0, 0, 0, 0, 32, 32, 64]
    for T in range(1, 2000):
        Q = oracle.kivi32_qlen(T)
        assert Q % 32 == 0 and Q <= T
        if T > 128:
            assert 129 <= T - Q <= 160  # the fp16 window always holds the newest 128 tokens (+ <= 32)


def _kv_rows(seed, T, nkv, D, std=1.0):
    from flarellm_amd import synth as S

    K = S.normal(seed, 0, T * nkv * D, 0.0, std).reshape(T, nkv, D)
    V = S.normal(seed, 1 << 40, T * nkv * D, 0.0, std).reshape(T, nkv, D)
    return K, V


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def test_kv_view_identity_forms(oracle):
    K, V = _kv_rows(3, 40, 2, 64)
    Ko, Vo = oracle.kv_view(oracle.OR_KV_F32, K, V)
    assert np.array_equal(Ko, K) and np.array_equal(Vo, V)
    Ko, Vo = oracle.kv_view(oracle.OR_KV_F16, K, V)
    assert np.array_equal(Ko, _f16(K)) and np.array_equal(Vo, _f16(V))


def test_kv_view_q8_closed_forms(oracle):
    T, nkv, D = 9, 2, 64
    K, V = _kv_rows(4, T, nkv, D)
    K[0, 0, :32] = 0.0                    # zero block -> zeros (d = 0, id = 0)
    K[1, 0, :32] = 0.75                   # constant block -> 127 * f16(0.75/127)
    K[2, 1, 32:] = np.linspace(-1, 1, 32)  # amax element -> +-127 codes
    Ko, Vo = oracle.kv_view(oracle.OR_KV_Q8, K, V)
    assert np.all(Ko[0, 0, :32] == 0.0)
    assert np.all(Ko[1, 0, :32] == np.float32(127.0) * _f16(np.float32(0.75) / np.float32(127.0)))
    d = _f16(np.float32(1.0) / np.float32(127.0))
    assert Ko[2, 1, 32] == -127 * d and Ko[2, 1, 63] == 127 * d
    # every value within half a step (+ the binary16 rounding of the step)
    for X, Xo in ((K, Ko), (V, Vo)):
        blk = X.reshape(-1, 32)
        amax = np.abs(blk).max(axis=1, keepdims=True)
        step = _f16(amax / 127.0)
        err = np.abs(Xo.reshape(-1, 32) - blk)
        assert np.all(err <= step / 2 + 127 * np.abs(step - amax / 127.0) + 1e-7)
        # the values are integer multiples of the stored step
        k = Xo.reshape(-1, 32) / np.where(step == 0, 1, step)
        assert np.allclose(k, np.round(k), atol=1e-4) and np.abs(np.round(k)).max() <= 127


def test_kv_view_kivi_window_and_groups(oracle):
    for T in (100, 160, 161, 200, 300):
        K, V = _kv_rows(5, T, 2, 64)
        Ko, Vo = oracle.kv_view(oracle.OR_KV_KIVI32, K, V)
        Q = oracle.kivi32_qlen(T)
        # the fp16 window is exact binary16
        assert np.array_equal(Ko[Q:], _f16(K[Q:])) and np.array_equal(Vo[Q:], _f16(V[Q:]))
        for g in range(Q // 32):
            kg = _f16(K[32 * g:32 * g + 32])       # [32 tokens, nkv, D]
            ko = Ko[32 * g:32 * g + 32]
            # K per channel: 4 levels spanning [min, max] of the channel's 32 values
            for h in range(2):
                for ch in range(0, 64, 7):
                    col, out = kg[:, h, ch], ko[:, h, ch]
                    assert len(np.unique(out)) <= 4
                    step = (col.max() - col.min()) / 3
                    assert np.abs(out - col).max() <= step / 2 + 2e-3 * (np.abs(col).max() + step)
                    assert abs(out.min() - col.min()) <= 1e-3 * max(1.0, abs(col.min()))
            # V per token over 32-channel groups
            vg = _f16(V[32 * g:32 * g + 32]).reshape(32, -1, 32)
            vo = Vo[32 * g:32 * g + 32].reshape(32, -1, 32)
            for t in range(0, 32, 5):
                for cg in range(vg.shape[1]):
                    row, out = vg[t, cg], vo[t, cg]
                    assert len(np.unique(out)) <= 4
                    step = (row.max() - row.min()) / 3
                    assert np.abs(out - row).max() <= step / 2 + 2e-3 * (np.abs(row).max() + step)


def test_kv_view_kivi_exact_levels_and_constant(oracle):
    # kv_cache.rs test_quantized_value_per_token_dequant_accuracy: values
    # 0,1,2,3 map to codes 0..3 exactly; test_quantized_constant_values_no_nan:
    # a constant group (range 0, scale 0) dequantizes to the constant.
    T, nkv, D = 200, 1, 64
    K = np.zeros((T, nkv, D), np.float32)
    V = np.zeros((T, nkv, D), np.float32)
    levels = np.array([0.0, 1.0, 2.0, 3.0], np.float32)
    K[:32, 0, :] = levels[np.arange(32) % 4][:, None]       # per channel over tokens: 0,1,2,3,...
    V[:32, 0, :] = levels[np.arange(64) % 4][None, :]       # per token over channels
    K[32:64] = 42.0
    V[32:64] = 42.0
    Ko, Vo = oracle.kv_view(oracle.OR_KV_KIVI32, K, V)
    assert oracle.kivi32_qlen(T) == 64
    assert np.array_equal(Ko[:64], K[:64]) and np.array_equal(Vo[:64], V[:64])
    assert not np.isnan(Ko).any() and not np.isnan(Vo).any()


def test_model_kv_quantized_modes_close_to_f32(oracle):
    """Whole-model oracle in Q8 / KIVI32 modes past the first quantized KIVI
    group: the logits stay finite and near the F32-cache logits (the KV
    quantization error is bounded; a dropped or misplaced term would not be)."""
    from flarellm_amd import FL_Q8_0
    from flarellm_amd import synth as S

    spec = S.tiny_spec(FL_Q8_0, max_seq=256)
    model = S.make_model(spec, seed=9)
    prompt = S.random_tokens(19, 170, spec.vocab)

    def last_logits(mode):
        om = oracle.OracleModel(model, mode)
        for pos, t in enumerate(prompt[:-1]):
            om.forward_greedy(int(t), pos)
        return om.forward_logits(int(prompt[-1]), len(prompt) - 1)

    b = last_logits(oracle.OR_KV_F32)
    for mode, tol in ((oracle.OR_KV_Q8, 0.05), (oracle.OR_KV_KIVI32, 0.5)):
        a = last_logits(mode)
        rel = np.linalg.norm(a - b) / np.linalg.norm(b)
        assert np.isfinite(a).all() and 0 < rel < tol, (mode, rel)


def test_thread_count_does_not_change_results(oracle):
    """Row-parallel oracle loops: every row keeps its sequential order, so
    1 thread and many threads give bit-identical outputs."""
    from flarellm_amd import synth as S

    spec = S.tiny_spec(S.FL_Q4K, embed_fmt=S.FL_Q6K, output_fmt=S.FL_Q6K)
    model = S.make_model(spec, seed=21)
    prompt = S.random_tokens(22, 6, spec.vocab)
    outs = []
    for n in (1, 4):
        oracle.set_threads(n)
        om = oracle.OracleModel(model)
        outs.append((om.generate(prompt, 8), om.forward_logits(3, 13)))
    oracle.set_threads()
    assert outs[0][0].tolist() == outs[1][0].tolist()
    assert np.array_equal(outs[0][1], outs[1][1])
