"""Write tests/golden/fixtures.npz: small input/output vectors of the hot-path
operations, computed in this container by the CPU oracle (oracle/, the C
restatement of flare-core's x86 path) on seeded inputs.

    python tests/golden/make_fixtures.py

Contents (every array named <case>__<field>):
  * dq_<fmt>:    GGUF block bytes of 2 x 512 weights and their dequantized
                 values (dequant_q8_0_block / dequant_q4k_block /
                 dequant_q6k_block)
  * mv_<fmt>_<rows>: a 1-row and a 4-row matvec with Q8 input: block bytes,
                 the input vector, its Q8_0 codes / scales, the per-block
                 integer dots and the matvec output
                 (matvec_q8_0_preq_into / matvec_q4k_q8_into)
  * rope_<hd>_<pos>: one row of 2 heads rotated at positions 0, 1, 4095,
                 8191, 8192 (apply_rope_with_table, inline past the table)
  * att:         one GQA head group (4 query heads, 2 kv heads, head_dim 64)
                 at T = 33: q, and K, V as written into the cache; att_<kv>:
                 the attention output over the cache form's values (f16, Q8,
                 KIVI2: or_kv_view, then or_gqa_attention)

The GPU tests compare the HIP kernels with these vectors; the CPU tests check
that the oracle still reproduces them.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flarellm_amd import FL_Q4K, FL_Q6K, FL_Q8_0  # noqa: E402
from flarellm_amd import synth as S  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz")
FMTS = {"q8_0": FL_Q8_0, "q4k": FL_Q4K, "q6k": FL_Q6K}
ROPE_THETA = 500000.0


def cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for name, fmt in FMTS.items():
        rows, cols = 2, 512
        w = S.quantize(S.normal(101, 0, rows * cols, 0.0, 0.02).reshape(rows, cols), fmt)
        out[f"dq_{name}__bytes"] = w
        out[f"dq_{name}__values"] = O.dequant(w, fmt, rows, cols)
    for name in ("q8_0", "q4k"):
        fmt = FMTS[name]
        for rows in (1, 4):
            cols = 512
            w = S.quantize(S.normal(200 + rows, 0, rows * cols, 0.0, 0.02).reshape(rows, cols), fmt)
            x = S.normal(300 + rows, 0, cols, 0.0, 1.0)
            q, s = O.quantize_q8(x)
            key = f"mv_{name}_{rows}"
            out[key + "__bytes"] = w
            out[key + "__x"] = x
            out[key + "__q"] = q
            out[key + "__s"] = s
            out[key + "__dots"] = O.block_dots(w, fmt, rows, cols, q)
            out[key + "__out"] = O.matvec(w, fmt, rows, cols, q, s)
    for hd in (64, 128):
        x = S.normal(400 + hd, 0, 2 * hd, 0.0, 1.0)
        out[f"rope_{hd}__x"] = x
        for pos in (0, 1, 4095, 8191, 8192):
            out[f"rope_{hd}_{pos}__y"] = O.apply_rope(x, 2, hd, pos, ROPE_THETA)
    rng = np.random.default_rng(33)
    T, nh, nkv, hd = 33, 4, 2, 64
    K = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    V = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    out["att__q"] = q
    out["att__k"] = K
    out["att__v"] = V
    for kv, mode in (("f16", O.OR_KV_F16), ("q8", O.OR_KV_Q8), ("kivi", O.OR_KV_KIVI32)):
        Kv, Vv = O.kv_view(mode, K, V)
        out[f"att_{kv}__out"] = O.gqa_attention(q, Kv, Vv, nh, nkv, hd, T)
    return out


def main() -> None:
    data = cases()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(data)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
