"""The committed fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py) against the CPU oracle and closed forms.

The oracle must reproduce every vector bit for bit (a change to the oracle
that moves any of them fails here); the Q8_0 dequantized values, the Q8
activation codes and the per-block integer dots are also recomputed
independently in numpy (quantize.rs / model.rs formulas), and the matvec
outputs from the dequantized weights in float64."""
import os

import numpy as np
import pytest

from flarellm_amd import FL_Q4K, FL_Q6K, FL_Q8_0

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
FMTS = {"q8_0": FL_Q8_0, "q4k": FL_Q4K, "q6k": FL_Q6K}


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", list(FMTS))
def test_dequant_fixture(oracle, fx, name):
    w, want = fx[f"dq_{name}__bytes"], fx[f"dq_{name}__values"]
    got = oracle.dequant(w, FMTS[name], 2, 512)
    assert np.array_equal(_bits(got), _bits(want))
    if name == "q8_0":
        # closed form: block = f16 scale + 32 int8 (quantize.rs:189-197)
        blk = w.reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        q = blk[:, 2:].view(np.int8).astype(np.float32)
        assert np.array_equal(_bits((d * q).reshape(2, 512)), _bits(want))


@pytest.mark.parametrize("name", ["q8_0", "q4k"])
@pytest.mark.parametrize("rows", [1, 4])
def test_matvec_fixture(oracle, fx, name, rows):
    k = f"mv_{name}_{rows}__"
    fmt, cols = FMTS[name], 512
    w, x = fx[k + "bytes"], fx[k + "x"]
    q, s = oracle.quantize_q8(x)
    assert np.array_equal(q, fx[k + "q"]) and np.array_equal(_bits(s), _bits(fx[k + "s"]))
    # quantize_input_q8_0_into (model.rs:5557-5570) in numpy: round half away, saturate
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(127.0) / np.where(amax == 0, 1, amax), 0).astype(np.float32)
    v = (xb * inv[:, None]).astype(np.float32)
    qn = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -128, 127).astype(np.int8)
    assert np.array_equal(qn.ravel(), fx[k + "q"]) and np.array_equal(_bits(d), _bits(fx[k + "s"]))
    dots = oracle.block_dots(w, fmt, rows, cols, q)
    assert np.array_equal(dots, fx[k + "dots"])
    if name == "q8_0":
        wq = w.reshape(rows, -1, 34)[:, :, 2:].view(np.int8).astype(np.int64)
        brute = (wq * q.reshape(1, -1, 32).astype(np.int64)).sum(2)
        assert np.array_equal(brute.ravel(), fx[k + "dots"].ravel().astype(np.int64))
    out = oracle.matvec(w, fmt, rows, cols, q, s)
    assert np.array_equal(_bits(out), _bits(fx[k + "out"]))
    ref = oracle.dequant(w, fmt, rows, cols).astype(np.float64) @ (q.astype(np.float64) * np.repeat(s, 32))
    np.testing.assert_allclose(fx[k + "out"], ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 4095, 8191, 8192])
def test_rope_fixture(oracle, fx, hd, pos):
    x, want = fx[f"rope_{hd}__x"], fx[f"rope_{hd}_{pos}__y"]
    got = oracle.apply_rope(x, 2, hd, pos, 500000.0)
    assert np.array_equal(_bits(got), _bits(want))
    if pos == 0:
        assert np.array_equal(_bits(want), _bits(x))  # identity at position 0
    # rotations preserve each pair's norm (pairs i, i + hd/2 of each head)
    a, b = x.reshape(2, 2, hd // 2), want.reshape(2, 2, hd // 2)
    np.testing.assert_allclose(np.hypot(b[:, 0], b[:, 1]), np.hypot(a[:, 0], a[:, 1]), rtol=1e-5)


@pytest.mark.parametrize("kv", ["f16", "q8", "kivi"])
def test_attention_fixture(oracle, fx, kv):
    mode = {"f16": oracle.OR_KV_F16, "q8": oracle.OR_KV_Q8, "kivi": oracle.OR_KV_KIVI32}[kv]
    q, K, V = fx["att__q"], fx["att__k"], fx["att__v"]
    Kv, Vv = oracle.kv_view(mode, K, V)
    got = oracle.gqa_attention(q, Kv, Vv, 4, 2, 64, 33)
    assert np.array_equal(_bits(got), _bits(fx[f"att_{kv}__out"]))
    # float64 softmax over the same cache view
    qh = q.reshape(4, 64).astype(np.float64)
    ref = np.empty((4, 64))
    for h in range(4):
        sc = Kv[:, h // 2, :].astype(np.float64) @ qh[h] / 8.0
        p = np.exp(sc - sc.max())
        ref[h] = (p / p.sum()) @ Vv[:, h // 2, :].astype(np.float64)
    np.testing.assert_allclose(fx[f"att_{kv}__out"], ref.ravel(), rtol=1e-4, atol=1e-5)
