"""The HIP kernels against the committed fixtures (tests/golden/fixtures.npz,
the oracle's outputs for seeded inputs; written by
tests/golden/make_fixtures.py).

Bar: dequantized values, activation codes / scales, per-block integer dots
and RoPE bit-exact; matvec outputs within 1e-3 relative; attention over each
cache form within 1e-3 relative plus the rounding allowance of the f16 MFMA
operands (as in test_gpu_kv.py)."""
import os

import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_KIVI2, FL_KV_Q8, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
FMTS = {"q8_0": FL_Q8_0, "q4k": FL_Q4K, "q6k": FL_Q6K}


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", list(FMTS))
def test_golden_dequant(backend, fx, name):
    w = fx[f"dq_{name}__bytes"]
    W = backend.upload(S.QWeight(w, FMTS[name], 2, 512))
    got = backend.dequant(W, 512).cpu().numpy()
    assert np.array_equal(_bits(got), _bits(fx[f"dq_{name}__values"]))


@pytest.mark.parametrize("name", ["q8_0", "q4k"])
@pytest.mark.parametrize("rows", [1, 4])
def test_golden_matvec(backend, fx, name, rows):
    k = f"mv_{name}_{rows}__"
    print(f"[golden] matvec {name} rows={rows}", flush=True)
    W = backend.upload(S.QWeight(fx[k + "bytes"], FMTS[name], rows, 512))
    q, s, su = backend.quantize_q8(_t(fx[k + "x"]))
    assert np.array_equal(q.cpu().numpy(), fx[k + "q"])
    assert np.array_equal(_bits(s.cpu().numpy()), _bits(fx[k + "s"]))
    dots = backend.block_dots(W, q).cpu().numpy()
    assert np.array_equal(dots.ravel(), fx[k + "dots"].ravel())
    got = backend.matvec_q8in(W, q, s, su).cpu().numpy()
    want = fx[k + "out"]
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-3 * np.abs(want).max())


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 4095, 8191, 8192])
def test_golden_rope(backend, fx, hd, pos):
    got = backend.rope(_t(fx[f"rope_{hd}__x"]), 2, hd, pos, 500000.0).cpu().numpy()
    assert np.array_equal(_bits(got), _bits(fx[f"rope_{hd}_{pos}__y"]))


@pytest.mark.parametrize("kv", ["f16", "q8", "kivi"])
def test_golden_attention(backend, fx, kv):
    print(f"[golden] attention {kv}", flush=True)
    q, K, V = fx["att__q"], fx["att__k"], fx["att__v"]
    T, nkv, hd = K.shape
    spec = S.tiny_spec(FL_Q8_0, heads=4, kv_heads=nkv, head_dim=hd, max_seq=64, layers=1)
    backend.init_gpu_kv_cache(spec, {"f16": FL_KV_F16, "q8": FL_KV_Q8, "kivi": FL_KV_KIVI2}[kv])
    backend.gpu_kv_write_batch(0, 0, K.reshape(T, -1)[:20], V.reshape(T, -1)[:20])
    for t in range(20, T):
        backend.gpu_kv_write(0, t, K[t].ravel(), V[t].ravel())
    got = backend.grouped_query_attention_from_gpu_cache(q, 0, T)
    want = fx[f"att_{kv}__out"]
    scale = np.abs(want).max()
    # 1e-3 relative, floored at 1e-3 of the output scale, plus 1e-5 of the scale
    bound = 1e-3 * np.maximum(np.abs(want), 1e-3 * scale) + 1e-5 * scale
    assert (np.abs(got - want) <= bound).all(), float(np.abs(got - want).max())
