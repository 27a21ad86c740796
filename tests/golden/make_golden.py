"""Writes the golden fixtures of this directory from the reference's own tests.

Reads (as text, never runs) flare-loader/tests/q4k_real_model.rs: the raw
144-byte Q4_K block taken from SmolLM2-135M-Instruct-Q4_K_M.gguf and the
llama.cpp-computed values of weights 0..8 and 128..136.  Run it in a
container where the reference is mounted:

    python tests/golden/make_golden.py /root/reference
"""
import json
import os
import re
import sys


def _array(text: str, name: str):
    m = re.search(r"let\s+" + name + r"\s*:\s*\[[^\]]*\]\s*=\s*\[(.*?)\];", text, re.S)
    if not m:
        raise SystemExit(f"{name} not found")
    return [float(v) if "." in v else int(v) for v in re.findall(r"-?\d+(?:\.\d+)?", m.group(1))]


def main(ref_root: str) -> None:
    src = os.path.join(ref_root, "flare-loader", "tests", "q4k_real_model.rs")
    text = open(src).read()
    block = _array(text, "block")
    assert len(block) == 144
    out = {
        "source": "flare-loader/tests/q4k_real_model.rs (test_q4k_real_block)",
        "tolerance": 0.01,
        "block": block,
        "expected_0_8": _array(text, "expected_0_8"),
        "expected_128_136": _array(text, "expected_128_136"),
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4k_real_block.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", dst)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
