"""CPU checks of the C-ABI library: it loads, exports every symbol the public
header declares, and its host-only entry points behave (no GPU needed)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flare_hip.h")


def _lib():
    from flarellm_amd import _lib as L

    if not os.path.exists(L.LIB_PATH):
        from flarellm_amd import build

        build.build()
    return L


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(fl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 30
    for must in ("fl_ctx_create", "fl_model_init", "fl_upload_weights", "fl_decode_step", "fl_generate",
                 "fl_op_matvec_q8in", "fl_op_attention", "fl_op_matvec_argmax"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    L = _lib()
    lib = C.CDLL(L.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared in flare_hip.h but not exported: {missing}"


def test_python_signatures_match_header():
    L = _lib()
    syms = set(declared_symbols())
    extra = [s for s in L.SIGNATURES if s not in syms]
    assert not extra, f"bound in _lib.py but not declared in the header: {extra}"
    assert set(L.SIGNATURES) == syms


def test_abi_version_and_name():
    lib = _lib().load()
    assert lib.fl_abi_version() == 1
    assert b"gfx950" in lib.fl_backend_name()


def test_format_row_bytes():
    """GGUF block sizes (flare-loader/src/gguf.rs block tables): Q8_0 34 B / 32,
    Q4_K 144 B / 256, Q6_K 210 B / 256; misaligned widths are rejected (0)."""
    lib = _lib().load()
    from flarellm_amd import FL_F32, FL_Q4K, FL_Q6K, FL_Q8_0

    assert lib.fl_format_row_bytes(FL_F32, 100) == 400
    assert lib.fl_format_row_bytes(FL_Q8_0, 2048) == 64 * 34
    assert lib.fl_format_row_bytes(FL_Q4K, 4096) == 16 * 144
    assert lib.fl_format_row_bytes(FL_Q6K, 4096) == 16 * 210
    assert lib.fl_format_row_bytes(FL_Q8_0, 33) == 0
    assert lib.fl_format_row_bytes(FL_Q4K, 128) == 0
    assert lib.fl_format_row_bytes(99, 256) == 0


def test_ctx_create_without_gpu_reports_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = _lib().load()
    h = C.c_void_p()
    rc = lib.fl_ctx_create(0, C.byref(h))
    assert rc != 0 and not h.value
    assert lib.fl_last_error(None)


def test_backend_raises_without_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from flarellm_amd._lib import FlareError
    from flarellm_amd.backend import HipBackend

    with pytest.raises((FlareError, RuntimeError)):
        HipBackend(0)


def test_synth_normal_is_seeded_and_standard():
    from flarellm_amd import synth as S

    a = S.normal(5, 0, 1 << 16)
    b = S.normal(5, 0, 1 << 16)
    c = S.normal(6, 0, 1 << 16)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    # stream offsets address the same sequence
    assert np.array_equal(S.normal(5, 1000, 10), a[1000:1010])
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1.0) < 0.02


@pytest.mark.parametrize("fmt", ["q8_0", "q4k", "q6k"])
def test_synth_quantize_round_trip(oracle, fmt):
    """Host block encoders vs the oracle's dequantizers (which are pinned by
    the reference's known-answer tests in test_oracle.py): the decoded
    weights are within the format's quantization step of the input."""
    from flarellm_amd import FL_Q4K, FL_Q6K, FL_Q8_0
    from flarellm_amd import synth as S

    f = {"q8_0": FL_Q8_0, "q4k": FL_Q4K, "q6k": FL_Q6K}[fmt]
    rows, cols = 8, 512
    w = S.normal(11, 0, rows * cols, 0.0, 0.02).reshape(rows, cols)
    data = S.quantize(w, f)
    back = oracle.dequant(data, f, rows, cols).reshape(rows, cols)
    err = np.abs(back - w)
    if fmt == "q8_0":
        # per 32-block: step d = amax/127 (f16-rounded), error <= d/2 (+ f16 rounding of d)
        amax = np.abs(w.reshape(-1, 32)).max(1)
        bound = (amax / 127.0) * 0.5 * 1.01 + 1e-7
        assert np.all(err.reshape(-1, 32) <= bound[:, None])
    else:
        # 6-bit / 4-bit sub-block quantizers: error well below the weight scale
        limit = {"q4k": 0.25, "q6k": 0.06}[fmt]
        assert err.max() < limit * np.abs(w).max()
        rel = np.linalg.norm(back - w) / np.linalg.norm(w)
        assert rel < {"q4k": 0.12, "q6k": 0.03}[fmt]
