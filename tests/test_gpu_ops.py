"""GPU parity of every hot-path op against the CPU oracle (seeded inputs).

Bar (north star): dequantised values, activation quantization and per-block
integer dots bit-exact; matvec and attention outputs within 1e-3 relative
(fp32 accumulate); fused argmax index identical.
"""
import numpy as np
import pytest

from flarellm_amd import FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu

REL = 1e-3  # north-star tolerance for fp32 matvec / attention outputs


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(got, want, rel=REL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    # per element: rel of the element, floored at rel of the vector's scale
    bound = rel * np.maximum(np.abs(want), 1e-3 * scale) + 1e-6 * scale
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}, scale {scale:.3e}"


def _act(seed, n, std=1.0):
    return S.normal(seed, 0, n, 0.0, std)


@pytest.mark.parametrize("n", [32, 576, 2048, 4096, 14336])
def test_quantize_q8_bit_exact(backend, oracle, n):
    print(f"[quantize] n={n}", flush=True)
    x = _act(n, n)
    x[:32] = 0.0  # all-zero block -> d = 0, q = 0
    x[-5] = 1e30  # saturating block
    q, s, su = backend.quantize_q8(_t(x))
    qo, so = oracle.quantize_q8(x)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(su.cpu().numpy(), qo.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32))


@pytest.mark.parametrize("n,order", [(576, 0), (2048, 0), (4096, 1), (2048, 1)])
def test_rmsnorm_quantize(backend, oracle, n, order):
    print(f"[rmsnorm_quant] n={n} order={order}", flush=True)
    x = _act(7 + n, n, 0.5)
    w = S.normal(9, 0, n, 1.0, 0.1)
    q, s, _ = backend.rmsnorm_quantize_q8(_t(x), _t(w), 1e-5, order)
    if order == 0:
        qo, so = oracle.rmsnorm_quantize_q8(x, w, 1e-5)
    else:
        qo, so = oracle.quantize_q8(oracle.rmsnorm(x, w, 1e-5))
    q = q.cpu().numpy().astype(np.int32)
    # the GPU sums x^2 as a tree: inv_rms may differ in the last ulp, which can
    # move a rounding boundary by one step
    assert np.abs(q - qo).max() <= 1
    assert (q != qo).mean() < 0.01
    np.testing.assert_allclose(s.cpu().numpy(), so, rtol=1e-5)


def test_rmsnorm(backend, oracle):
    x = _act(3, 4096, 0.3)
    w = S.normal(4, 0, 4096, 1.0, 0.1)
    got = backend.rmsnorm(_t(x), _t(w), 1e-5).cpu().numpy()
    np.testing.assert_allclose(got, oracle.rmsnorm(x, w, 1e-5), rtol=1e-5)


MV_SHAPES = [
    (FL_Q8_0, 96, 256), (FL_Q8_0, 1001, 2048), (FL_Q8_0, 64, 576), (FL_Q8_0, 200, 8192),
    (FL_Q8_0, 3072, 2048), (FL_Q4K, 96, 256), (FL_Q4K, 130, 4096), (FL_Q4K, 64, 14336),
    (FL_Q4K, 1536, 4096),
]


@pytest.mark.parametrize("fmt,rows,cols", MV_SHAPES)
def test_block_dots_bit_exact(backend, oracle, fmt, rows, cols):
    print(f"[block_dots] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    q, s = oracle.quantize_q8(_act(11, cols))
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    got = backend.block_dots(W, _t(q)).cpu().numpy()
    want = oracle.block_dots(w, fmt, rows, cols, q)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,rows,cols", MV_SHAPES)
def test_matvec_q8in(backend, oracle, fmt, rows, cols):
    print(f"[matvec] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows + 5, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    q, s = oracle.quantize_q8(_act(13, cols))
    sums = q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    got = backend.matvec_q8in(W, _t(q), _t(s), _t(sums)).cpu().numpy()
    want = oracle.matvec(w, fmt, rows, cols, q, s)
    _close(got, want)


@pytest.mark.parametrize("fmt,rows,cols", [(FL_Q8_0, 77, 576), (FL_Q4K, 33, 512), (FL_Q6K, 45, 4096),
                                           (FL_Q6K, 10, 256)])
def test_dequant_bit_exact(backend, oracle, fmt, rows, cols):
    w = S.quantize(S.normal(rows + 9, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    got = backend.dequant(W, cols).cpu().numpy()
    want = oracle.dequant(w, fmt, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt,rows,cols", [(FL_Q8_0, 1000, 2048), (FL_Q6K, 700, 4096), (FL_Q8_0, 300, 576),
                                           (FL_Q6K, 64, 256)])
def test_matvec_f32in(backend, oracle, fmt, rows, cols):
    print(f"[matvec_f32in] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows + 3, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    x = _act(17, cols)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    got = backend.matvec_f32in(W, _t(x)).cpu().numpy()
    want = oracle.matvec_f32(oracle.dequant(w, fmt, rows, cols), x)
    _close(got, want)


@pytest.mark.parametrize("fmt,rows,cols", [(FL_Q8_0, 5000, 2048), (FL_Q4K, 3000, 4096), (FL_Q8_0, 49152, 576)])
def test_matvec_argmax_q8in(backend, oracle, fmt, rows, cols):
    print(f"[argmax_q8in] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows + 21, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    q, s = oracle.quantize_q8(_act(19, cols))
    sums = q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    gi, gv = backend.matvec_argmax(W, q=_t(q), s=_t(s), su=_t(sums))
    oi, ov = oracle.matvec_argmax(w, fmt, rows, cols, q, s)
    full = oracle.matvec(w, fmt, rows, cols, q, s)
    top2 = np.sort(full)[-2:]
    if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
        assert gi == oi
    assert abs(gv - ov) <= 1e-3 * abs(ov)


@pytest.mark.parametrize("fmt,rows,cols", [(FL_Q8_0, 8000, 2048), (FL_Q6K, 4000, 4096)])
def test_matvec_argmax_f32in(backend, oracle, fmt, rows, cols):
    print(f"[argmax_f32in] fmt={fmt} {rows}x{cols}", flush=True)
    w = S.quantize(S.normal(rows + 23, 0, rows * cols, 0, 0.02).reshape(rows, cols), fmt)
    x = _act(29, cols)
    W = backend.upload(S.QWeight(w, fmt, rows, cols))
    gi, gv = backend.matvec_argmax(W, x=_t(x))
    deq = oracle.dequant(w, fmt, rows, cols)
    oi, ov = oracle.matvec_argmax_f32(deq, x)
    full = oracle.matvec_f32(deq, x)
    top2 = np.sort(full)[-2:]
    if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
        assert gi == oi
    assert abs(gv - ov) <= 1e-3 * abs(ov)


def test_argmax_first_max_on_ties(backend, oracle):
    # identical rows 3, 700 and 900: strict '>' keeps the first (model.rs:8551)
    rows, cols = 1024, 256
    wf = S.normal(31, 0, rows * cols, 0, 0.02).reshape(rows, cols)
    x = _act(37, cols)
    wf[700] = wf[3] = wf[900] = np.sign(x) * 0.05
    w = S.quantize(wf, FL_Q8_0)
    W = backend.upload(S.QWeight(w, FL_Q8_0, rows, cols))
    gi, _ = backend.matvec_argmax(W, x=_t(x))
    oi, _ = oracle.matvec_argmax_f32(oracle.dequant(w, FL_Q8_0, rows, cols), x)
    assert oi == 3 and gi == 3


@pytest.mark.parametrize("nh,hd,pos", [(32, 64, 0), (32, 128, 1), (8, 128, 4095), (9, 64, 8191), (8, 64, 8192)])
def test_rope_bit_exact(backend, oracle, nh, hd, pos):
    x = _act(41 + pos, nh * hd)
    got = backend.rope(_t(x), nh, hd, pos, 500000.0).cpu().numpy()
    want = oracle.apply_rope(x, nh, hd, pos, 500000.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_silu_mul(backend, oracle):
    g = _act(43, 14336, 3.0)
    u = _act(47, 14336)
    got = backend.silu_mul(_t(g), _t(u)).cpu().numpy()
    _close(got, oracle.silu_mul(g, u), rel=1e-5)


ATTN_CASES = [
    # nh, nkv, hd, T, kv dtype, splits
    (32, 8, 128, 1, "f16", 0), (32, 8, 128, 33, "f16", 0), (32, 8, 128, 4096, "f16", 0),
    (32, 8, 64, 768, "f16", 0), (9, 3, 64, 100, "f32", 0), (32, 8, 128, 1000, "f32", 7),
    (8, 8, 64, 257, "f16", 1), (16, 2, 128, 8192, "f16", 0), (4, 1, 64, 5, "f32", 3),
]


@pytest.mark.parametrize("nh,nkv,hd,T,dt,splits", ATTN_CASES)
def test_attention(backend, oracle, nh, nkv, hd, T, dt, splits):
    import torch

    print(f"[attention] nh={nh} nkv={nkv} hd={hd} T={T} {dt} splits={splits}", flush=True)
    q = _act(51, nh * hd)
    k = _act(53, T * nkv * hd).reshape(T, nkv, hd)
    v = _act(59, T * nkv * hd).reshape(T, nkv, hd)
    tdt = torch.float16 if dt == "f16" else torch.float32
    kt = torch.from_numpy(k).to(tdt).cuda()
    vt = torch.from_numpy(v).to(tdt).cuda()
    got = backend.attention(_t(q), kt, vt, nh, nkv, hd, T, splits).cpu().numpy()
    want = oracle.gqa_attention(q, kt.float().cpu().numpy(), vt.float().cpu().numpy(), nh, nkv, hd, T)
    _close(got, want)


@pytest.mark.parametrize("T,splits", [(8192, 0), (3000, 17), (700, 0)])
def test_attention_split_merge_repeatable(backend, oracle, T, splits):
    """Cross-workgroup split merge: repeated launches agree bit-for-bit."""
    import torch

    nh, nkv, hd = 32, 8, 128
    print(f"[attention-merge] T={T} splits={splits}", flush=True)
    q = _act(61, nh * hd)
    k = _act(67, T * nkv * hd).reshape(T, nkv, hd)
    v = _act(71, T * nkv * hd).reshape(T, nkv, hd)
    kt = torch.from_numpy(k).half().cuda()
    vt = torch.from_numpy(v).half().cuda()
    outs = [backend.attention(_t(q), kt, vt, nh, nkv, hd, T, splits).cpu().numpy() for _ in range(20)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    want = oracle.gqa_attention(q, kt.float().cpu().numpy(), vt.float().cpu().numpy(), nh, nkv, hd, T)
    _close(outs[0], want)
