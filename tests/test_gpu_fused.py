"""The fused QKV + attention launch of the decode step (FL_OPT_FUSE_ATTN,
off by default: measured slower on MI355X).

With an fp16 KV cache each layer's QKV matvec and attention run as one
launch: the attention workgroups stream the K / V cache while the QKV
workgroups compute, wait for them, then read q and the new token's K / V row
from what those published.  The values and the order of every operation are
those of the two separate kernels, so the decode step's outputs must be
bit-identical with the option on and off -- logits, greedy tokens, and the
cache the following steps read.  Checked at the C2 and C3 model widths
(2 layers), at contexts of one split, a few, and more than 8 per kv head,
through the graph-replayed greedy loop and the logits-returning step.

The reference path: forward_layers (flare-core/src/model.rs:1955-2561),
cpu_grouped_query_attention_into 9849-9966.
"""
import numpy as np
import pytest

from flarellm_amd import FL_KV_F16
from flarellm_amd import _lib as L
from flarellm_amd import synth as S

pytestmark = pytest.mark.gpu


def _run(backend, prompt, n_gen, n_logit, fuse):
    backend.set_option(L.FL_OPT_FUSE_ATTN, fuse)
    backend.reset()
    gen = backend.generate(prompt, n_gen)
    pos = len(prompt) + n_gen - 1
    tok = int(gen[-1])
    logits = []
    for i in range(n_logit):
        lg = backend.forward_single_token_gpu(tok, pos + i)
        logits.append(lg)
        tok = int(np.argmax(lg))
    backend.sync()
    return gen, np.stack(logits)


@pytest.mark.timeout(600)
# contexts: one split, a few, and more than 8 per kv head (the split merge's
# batched form; C2 128-slot and C3 256-slot chunks)
@pytest.mark.parametrize("width,n_prompt", [("c2", 5), ("c2", 300), ("c2", 1100), ("c3", 7), ("c3", 600),
                                            ("c3", 2200)])
def test_fused_step_identical(backend, width, n_prompt):
    base = S.LLAMA32_1B if width == "c2" else S.LLAMA3_8B
    spec = S.replace(base, layers=2, max_seq=n_prompt + 48)
    print(f"[fused] {width} prompt {n_prompt}", flush=True)
    model = S.make_model(spec, seed=23)
    backend.init_gpu_kv_cache(spec, FL_KV_F16)
    backend.upload_weights_to_gpu(model)
    prompt = S.random_tokens(31 + n_prompt, n_prompt, spec.vocab)
    try:
        g1, l1 = _run(backend, prompt, 24, 6, 1)
        g0, l0 = _run(backend, prompt, 24, 6, 0)
    finally:
        backend.set_option(L.FL_OPT_FUSE_ATTN, 0)
    assert g1.tolist() == g0.tolist()
    assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32)), float(np.abs(l1 - l0).max())
