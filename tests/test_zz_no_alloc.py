"""fl_op_batched_matvec_q8in_noalloc: the batched quantized matvec with its
K-split partials in the library's file-scope device array instead of a
per-call allocation.  Called through the C-ABI; its output must equal the
allocating entry point's bit for bit (same kernels, same K split, same
summation order), on two calls in a row, the second smaller."""

import numpy as np
import pytest

from flarellm_amd import FL_Q4K, FL_Q8_0
from flarellm_amd import synth as S
from flarellm_amd._lib import FlareError, check

pytestmark = pytest.mark.gpu


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _inputs(oracle, M, cols, seed):
    qs, ss, sums = [], [], []
    for m in range(M):
        q, s = oracle.quantize_q8(S.normal(seed + m, 0, cols, 0.0, 1.0))
        qs.append(q)
        ss.append(s)
        sums.append(q.reshape(-1, 32).astype(np.int32).sum(1, dtype=np.int32))
    return _t(np.stack(qs)), _t(np.stack(ss)), _t(np.stack(sums))


def _noalloc(backend, W, q, s, su):
    import torch

    M = q.shape[0]
    out = torch.full((M, W.rows), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    check(backend.lib.fl_op_batched_matvec_q8in_noalloc(backend.ctx, W.handle, M, q.data_ptr(), s.data_ptr(),
                                                         su.data_ptr(), out.data_ptr()), backend.ctx)
    backend.sync()
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt,rows,cols,M,rows2,cols2,M2", [
    (FL_Q4K, 6144, 4096, 8, 1024, 4096, 5),     # C5 fused QKV, then a smaller one
    (FL_Q8_0, 16384, 2048, 16, 3072, 2048, 3),  # Llama-3.2-1B gate/up, then QKV
])
def test_noalloc_matches_allocating_entry(backend, oracle, fmt, rows, cols, M, rows2, cols2, M2):
    for r, c, m, seed in ((rows, cols, M, 1), (rows2, cols2, M2, 2)):
        print(f"[noalloc] fmt={fmt} {r}x{c} M={m}", flush=True)
        w = S.quantize(S.normal(r + c + seed, 0, r * c, 0, 0.02).reshape(r, c), fmt)
        W = backend.upload(S.QWeight(w, fmt, r, c))
        q, s, su = _inputs(oracle, m, c, 40 * seed)
        want = backend.batched_matvec_q8in(W, q, s, su).cpu().numpy()
        got = _noalloc(backend, W, q, s, su)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        W.free()


def test_noalloc_rejects_oversize(backend):
    rows, cols = 300000, 32  # 16 tokens x 300000 rows of partials > 4 Mi floats
    w = S.quantize(np.zeros((rows, cols), np.float32), FL_Q8_0)
    W = backend.upload(S.QWeight(w, FL_Q8_0, rows, cols))
    import torch

    q = torch.zeros((16, cols), dtype=torch.int8, device="cuda")
    s = torch.zeros((16, 1), dtype=torch.float32, device="cuda")
    su = torch.zeros((16, 1), dtype=torch.int32, device="cuda")
    out = torch.zeros((16, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(FlareError, match="no-alloc scratch"):
        check(backend.lib.fl_op_batched_matvec_q8in_noalloc(backend.ctx, W.handle, 16, q.data_ptr(), s.data_ptr(),
                                                             su.data_ptr(), out.data_ptr()), backend.ctx)
    W.free()
