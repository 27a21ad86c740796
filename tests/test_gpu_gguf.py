"""A model loaded from a GGUF file (fl_model_load_gguf) on the GPU: the
weights stream from the memory-mapped file into the same device layout as
fl_upload_weights from memory, so greedy streams are identical to the
in-memory upload and to the CPU oracle (flare-loader/src/weights.rs:30-66,
gguf.rs:616-688)."""
import time

import numpy as np
import pytest

from flarellm_amd import FL_KV_F16, FL_KV_F32, FL_Q4K, FL_Q6K, FL_Q8_0
from flarellm_amd import _lib as L
from flarellm_amd import synth as S
from flarellm_amd.gguf import write_gguf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("spec", [S.tiny_spec(FL_Q8_0), S.tiny_spec(FL_Q4K, embed_fmt=FL_Q6K, output_fmt=FL_Q6K),
                                  S.SMOLLM2_135M], ids=["q8_tied", "q4k_q6k", "smollm2"])
def test_gguf_load_matches_memory_upload_and_oracle(backend, oracle, tmp_path, spec):
    print(f"[gguf] {spec.name}", flush=True)
    model = S.make_model(spec, seed=4)
    path = str(tmp_path / "m.gguf")
    write_gguf(path, model)
    prompt = S.random_tokens(8, 12, spec.vocab)
    got_spec = backend.load_gguf(path, FL_KV_F32, spec.max_seq)
    assert (got_spec.hidden, got_spec.layers, got_spec.vocab, got_spec.layer_fmt) == \
        (spec.hidden, spec.layers, spec.vocab, spec.layer_fmt)
    from_file = backend.generate(prompt, 32)
    backend.init_gpu_kv_cache(spec, FL_KV_F32)
    backend.upload_weights_to_gpu(model)
    from_mem = backend.generate(prompt, 32)
    assert from_file.tolist() == from_mem.tolist()
    if spec.layer_fmt == FL_Q8_0 and spec.output_fmt is None:
        # reference-order mode: the file-loaded model's stream is the oracle's
        backend.load_gguf(path, FL_KV_F32, spec.max_seq)
        backend.set_option(L.FL_OPT_EXACT, 1)
        try:
            exact = backend.generate(prompt, 32)
        finally:
            backend.set_option(L.FL_OPT_EXACT, 0)
        want = oracle.OracleModel(model, oracle.OR_KV_F32).generate(prompt, 32)
        assert exact.tolist() == want.tolist()


@pytest.mark.timeout(600)
def test_gguf_load_c2_time(backend, tmp_path):
    """Llama-3.2-1B Q8_0 (1.3 GB file): load time and the first greedy tokens
    against the in-memory upload."""
    spec = S.replace(S.CONFIGS["Llama-3.2-1B"], max_seq=256)
    model = S.make_model(spec, seed=1)
    path = str(tmp_path / "c2.gguf")
    write_gguf(path, model)
    t0 = time.perf_counter()
    backend.load_gguf(path, FL_KV_F16, 256)
    t_load = time.perf_counter() - t0
    prompt = S.random_tokens(7, 16, spec.vocab)
    a = backend.generate(prompt, 8)
    backend.init_gpu_kv_cache(spec, FL_KV_F16)
    t0 = time.perf_counter()
    backend.upload_weights_to_gpu(model)
    t_mem = time.perf_counter() - t0
    b = backend.generate(prompt, 8)
    print(f"[gguf c2] file load {t_load:.2f} s, in-memory upload {t_mem:.2f} s", flush=True)
    assert a.tolist() == b.tolist()
