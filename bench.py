"""Decode benchmark: batch-1 greedy decode tok/s + quant-matvec HBM GB/s.

Default workload: Llama-3.2-1B architecture,
random N(0, 0.02) weights in Q8_0 with tied embeddings, fp16 KV cache of 2048
slots, greedy decode after a 512-token uniform-random prompt.  One "step" is
one decoded token (a HIP-graph replay of the whole forward + fused argmax);
the prompt is fed through the same step before the timed region.

Prints ONE JSON line (the driver's contract) with the roofline of the
dominant kernel measured live with HIP events, and a CPU baseline: the C
restatement of flarellm's x86 decode path (oracle/) timed single-threaded on a
bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
METRIC = "decode tok/s (batch 1) + quant-matvec HBM GB/s vs peak, Llama-3.2-1B Q8_0"

WORKLOADS = {
    "c2": dict(spec="Llama-3.2-1B", prompt=512, kv="f16",
               desc="Llama-3.2-1B arch, Q8_0 tied embeddings, batch-1 greedy decode after a 512-token "
                    "random prompt, fp16 KV cache 2048 slots"),
    "c3": dict(spec="Llama-3-8B", prompt=4096, kv="f16",
               desc="Llama-3-8B arch, Q4_K layers + Q6_K output/embedding, batch-1 greedy decode at "
                    "context 4096, fp16 KV cache"),
    "c4": dict(spec="Llama-3-8B", prompt=0, kv="all",
               desc="decode attention kernel alone at Llama-3-8B heads (32 q / 8 kv, head_dim 128), one query "
                    "token, KV cache of 8k / 32k / 128k tokens in fp16, Q8 (per-32 fp16 scale) and KIVI 2-bit "
                    "(group 32, fp16 residual window); q, K, V ~ N(0, 1)"),
    "c5": dict(spec="Llama-3-8B", prompt=4096, kv="f16",
               desc="speculative verify on the Llama-3-8B Q4_K / Q6_K-output shape: k=8 uniform-random draft "
                    "tokens through the model in one pass (M=8 int8-MFMA quantized GEMMs, causal attention over "
                    "the 8 new tokens) at context 4096, fp16 KV"),
    "c1": dict(spec="SmolLM2-135M", prompt=32, kv="f32",
               desc="SmolLM2-135M arch, Q8_0 tied, greedy decode after a 32-token prompt"),
}
KERNEL_NAMES = {0: "qkv", 1: "wo", 2: "gate_up", 3: "down", 4: "output+argmax", 5: "attention"}
# Calibrated HBM traffic per launch, from rocprofv3 --pmc FETCH_SIZE /
# WRITE_SIZE runs of this script (summaries committed under profiles/):
# lines "traffic <config> <kernel> <bytes>".
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")


def measured_traffic(config: str) -> dict:
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                p = line.strip().strip("`").split()
                if len(p) == 4 and p[0] == "traffic" and p[1] == config:
                    out[p[2]] = int(float(p[3]))
    except OSError:
        pass
    return out


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, spec, n_prompt: int, n_decode: int, n_decode_par: int) -> dict:
    """flarellm's x86 decode path restated in C (oracle/, -O3 -march=x86-64-v3):
    single thread (the reference's quantized x86 path is single-threaded), and
    an OpenMP row-parallel variant on this host's cores (reported beside it)."""
    from oracle import oracle as O

    from flarellm_amd import synth as S

    def run(threads: int, steps: int):
        O.set_threads(threads)
        om = O.OracleModel(model, O.OR_KV_F32)
        prompt = S.random_tokens(77, n_prompt, spec.vocab)
        tok = 0
        for i, t in enumerate(prompt):
            tok, _ = om.forward_greedy(int(t), i)
        t0 = time.perf_counter()
        pos = n_prompt
        for _ in range(steps):
            tok, _ = om.forward_greedy(int(tok), pos)
            pos += 1
        dt = time.perf_counter() - t0
        om.close()
        return steps / dt, dt

    v1, dt1 = run(1, n_decode)
    ncores = min(16, len(os.sched_getaffinity(0)))
    vp, dtp = run(ncores, n_decode_par)
    O.set_threads(1)
    cpu = _cpu_model()
    return {"value": round(v1, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n_decode} greedy decode steps after a {n_prompt}-token prompt (context {n_prompt}.."
                      f"{n_prompt + n_decode}; the GPU line runs at context 512+, where attention is <3 % of the "
                      f"CPU step) on the same synthetic model, f32 KV, C restatement of flare-core's x86 scalar "
                      f"path, {dt1:.1f} s on {cpu}",
            "parallel": {"value": round(vp, 4), "unit": "tok/s", "cores": ncores, "kind": "port",
                         "sample": f"{n_decode_par} steps, OpenMP row-parallel matvecs / heads, {dtp:.1f} s"}}


def bench_attention_c4(args) -> int:
    """the decode attention kernel alone.  For each KV
    form and context, the cache is filled with N(0,1) rows and enough layers
    (>= 1 GB of K+V in total) that consecutive launches stream from HBM, not
    the 256 MB MALL; HIP events on the context stream time `iters` launches."""
    import numpy as np
    import torch

    from flarellm_amd import FL_KV_F16, FL_KV_KIVI2, FL_KV_Q8
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    base = S.CONFIGS["Llama-3-8B"]
    nh, nkv, hd = base.heads, base.kv_heads, base.head_dim
    kvd = nkv * hd
    forms = {"f16": FL_KV_F16, "q8": FL_KV_Q8, "kivi2": FL_KV_KIVI2}
    ctxs = [8192, 32768, 131072]
    rng = np.random.default_rng(3)
    rows_k = rng.standard_normal((max(ctxs), kvd), dtype=np.float32)
    rows_v = rng.standard_normal((max(ctxs), kvd), dtype=np.float32)
    q = rng.standard_normal(nh * hd, dtype=np.float32)
    b = HipBackend(0)
    stream = torch.cuda.ExternalStream(b.stream)
    cases = {}
    tot_bytes = tot_us = 0.0
    for name, fmt in forms.items():
        for T in ctxs:
            # bytes of one launch decide the layer count (>= 1 GB rotated)
            spec = S.replace(base, layers=1, max_seq=T)
            b.init_gpu_kv_cache(spec, fmt)
            nbytes = b.bench_attention(T, 0)
            L = int(min(256, max(2, -(-1.0e9 // nbytes))))
            spec = S.replace(base, layers=L, max_seq=T)
            b.init_gpu_kv_cache(spec, fmt)
            t0 = time.time()
            for l in range(L):
                b.gpu_kv_write_batch(l, 0, rows_k[:T], rows_v[:T])
            out = b.grouped_query_attention_from_gpu_cache(q, 0, T)  # also stages q
            assert np.isfinite(out).all()
            b.bench_attention(T, 3)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            iters = args.kernel_iters
            e0.record(stream)
            nbytes = b.bench_attention(T, iters)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / iters
            cases[f"{name}@{T // 1024}k"] = {"us": round(us, 2), "bytes": int(nbytes), "layers": L,
                                            "GB_s": round(nbytes / us / 1e3, 1),
                                            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
            tot_bytes += nbytes
            tot_us += us
            log(f"[bench c4] {name:6s} T={T:6d} L={L:3d} fill {time.time() - t0:.1f}s  {us:9.2f} us  "
                f"{nbytes / 1e6:8.2f} MB  {nbytes / us / 1e3:7.1f} GB/s")
    b.close()
    dom = max(cases, key=lambda k: cases[k]["us"])
    d = cases[dom]
    out = {
        "metric": "decode attention HBM GB/s (one query token, Llama-3-8B heads, KV 8k/32k/128k in fp16/Q8/KIVI2)",
        "value": round(tot_bytes / tot_us / 1e3, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.kernel_iters,
        "warmup": 3, "ms_per_step": round(tot_us / len(cases) / 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (fp16 / int8 / 2-bit KV)",
        "data": "synthetic (q, K, V ~ N(0,1))",
        "config": {"workload": WORKLOADS["c4"]["desc"], "model": "Llama-3-8B heads", "global_batch": 1,
                   "seq_len": max(ctxs), "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": d["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d["frac"], "traffic": None, "kernel": f"k_attm {dom}", "bytes_per_launch": d["bytes"],
                     "avg_launch_us": d["us"]},
        "cpu_baseline": None,
        "cases": cases,
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_verify_c5(args) -> int:
    """one verify pass of k=8 drafts at context 4096.

    Acceptance: the pass's greedy tokens must match sequential decode's
    (fl_decode_step) for the same drafts.  On this random-weight 8B model two
    valid decode orders (different attention chunking / matvec tiling) differ
    by ~5 % in their logits after a 4096-token context: fp32 rounding-order
    and Q8-requantization differences are amplified through 32 layers.  So the
    token check runs after a 64-token context, where the orders agree to
    ~1e-3, and the timing runs at context 4096 (each pass rewrites the same 8
    cache slots)."""
    import numpy as np
    import torch

    from flarellm_amd import FL_KV_F16
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    wl = WORKLOADS["c5"]
    spec = S.replace(S.CONFIGS[wl["spec"]], max_seq=max(wl["prompt"], args.prompt or 0) + 64)
    n_prompt, k = (wl["prompt"] if args.prompt is None else max(64, args.prompt)), 8
    t0 = time.time()
    model = S.make_model(spec, seed=2)
    log(f"[bench c5] synthetic {spec.name} built in {time.time() - t0:.1f}s")
    b = HipBackend(0)
    b.init_gpu_kv_cache(spec, FL_KV_F16)
    b.upload_weights_to_gpu(model)
    drafts = S.random_tokens(9, k, spec.vocab)

    # ---- acceptance vs sequential decode (64-token context) ------------------
    n_short = 64
    b.generate(S.random_tokens(7, n_short, spec.vocab), 1)
    got, vvals = b.verify(drafts, n_short)
    got = [int(x) for x in got]
    seq, gaps, vdiff = [], [], []
    for i, t in enumerate(drafts):
        lg = b.forward_single_token_gpu(int(t), n_short + i)
        top2 = np.sort(lg)[-2:]
        seq.append(int(np.argmax(lg)))
        gaps.append(float((top2[1] - top2[0]) / abs(top2[1])))
        vdiff.append(float(abs(vvals[i] - lg[got[i]]) / abs(top2[1])))
    # a position is decided when its top-2 gap exceeds twice the largest
    # verify-vs-sequential logit difference of this run (relative to the top
    # logit): two tree orders of the same arithmetic move logits by that much
    margin = max(2e-2, 2.0 * max(vdiff))
    decided = [i for i in range(k) if gaps[i] > margin]
    accepted = all(got[i] == seq[i] for i in decided)
    agree = sum(g == s_ for g, s_ in zip(got, seq))
    log(f"[bench c5] context {n_short}: verify {got} sequential {seq}; top-2 gaps {[round(g, 4) for g in gaps]}; "
        f"|verify - sequential logit| / top {[round(v, 4) for v in vdiff]}; agree {agree}/{k}, "
        f"positions with gap > {margin}: {len(decided)}, all agree={accepted}")

    # ---- timing at context 4096 --------------------------------------------------
    b.reset()
    b.generate(S.random_tokens(7, n_prompt, spec.vocab), 1)
    for _ in range(max(1, args.warmup // 4)):
        b.verify(drafts, n_prompt)
    torch.cuda.synchronize()
    steps = max(1, args.steps // 16)
    t1 = time.perf_counter()
    for _ in range(steps):
        b.verify(drafts, n_prompt)
    ms = (time.perf_counter() - t1) * 1000.0 / steps
    t1 = time.perf_counter()
    for i, t in enumerate(drafts):
        b.forward_greedy(int(t), n_prompt + i)
    seq_ms = (time.perf_counter() - t1) * 1000.0
    log(f"[bench c5] context {n_prompt}: verify pass {ms:.3f} ms ({k} tokens); 8 sequential steps {seq_ms:.3f} ms")
    b.close()
    bytes_pass = spec.weight_bytes_per_token()
    out = {
        "metric": "speculative verify tokens/s (k=8 drafts per pass, Llama-3-8B Q4_K, context 4096)",
        "value": round(k * 1000.0 / ms, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": max(1, args.warmup // 4), "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8 (MFMA i32 16x16x32)",
        "data": "synthetic (random N(0,0.02) weights quantized to GGUF blocks; uniform-random tokens)",
        "config": {"workload": wl["desc"], "model": spec.name, "global_batch": k, "seq_len": n_prompt,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(bytes_pass / ms / 1e6, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(bytes_pass / ms / 1e6 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole verify pass (weight bytes once per pass)", "bytes_per_launch": bytes_pass,
                     "avg_launch_us": round(ms * 1000.0, 1)},
        "cpu_baseline": None,
        "acceptance": {"context": n_short, "agree_positions": agree, "decided_positions": len(decided),
                       "decided_all_agree": accepted, "max_logit_rel_diff": round(max(vdiff), 5),
                       "decided_margin": round(margin, 5)},
        "sequential_8_steps_ms": round(seq_ms, 3),
    }
    print(json.dumps(out), flush=True)
    return 0 if accepted else 1


def run_decode(args, config: str, with_cpu: bool) -> dict:
    """One decode workload (c1 / c2 / c3): synthetic model, the prompt fed
    through the decode step (untimed), warmup steps, then args.steps greedy
    steps timed with HIP events on the context stream; per-kernel HBM rates
    (HIP events around back-to-back launches); a timed fl_prefill of the same
    prompt; optionally the CPU baseline.  Returns the JSON fields."""
    import numpy as np
    import torch

    from flarellm_amd import FL_KV_F16, FL_KV_F32
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    wl = WORKLOADS[config]
    spec = S.CONFIGS[wl["spec"]]
    n_prompt = wl["prompt"] if args.prompt is None else max(1, args.prompt)
    need = n_prompt + args.warmup + args.steps
    if need > spec.max_seq:
        spec = S.replace(spec, max_seq=need)
    t0 = time.time()
    model = S.make_model(spec, seed=1)
    log(f"[bench {config}] synthetic {spec.name} built in {time.time() - t0:.1f}s")
    b = HipBackend(0)
    b.init_gpu_kv_cache(spec, FL_KV_F16 if wl["kv"] == "f16" else FL_KV_F32)
    t0 = time.time()
    b.upload_weights_to_gpu(model)
    log(f"[bench {config}] uploaded in {time.time() - t0:.1f}s")
    prompt = S.random_tokens(7, n_prompt, spec.vocab)

    stream = torch.cuda.ExternalStream(b.stream)
    # prompt (untimed), then warmup steps
    t0 = time.time()
    b.generate(prompt, 1)
    log(f"[bench {config}] prompt of {n_prompt} tokens through the decode step in {time.time() - t0:.2f}s")
    b.decode_continue(args.warmup)
    b.sync()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    ev0.record(stream)
    b.decode_continue(args.steps)
    ev1.record(stream)
    b.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms_total = ev0.elapsed_time(ev1)
    ms_per_step = ms_total / args.steps
    tok_s = 1000.0 / ms_per_step
    toks = b.read_tokens(n_prompt, 8)
    log(f"[bench {config}] {args.steps} steps: {ms_total:.2f} ms (wall {wall * 1e3:.2f} ms) -> {tok_s:.1f} tok/s; "
        f"first tokens {toks.tolist()}")

    # per-kernel HBM bandwidth: HIP events on the context stream around
    # back-to-back launches; launch i uses layer i % L, so consecutive
    # launches stream distinct weights from HBM
    kernels = {}
    for which, name in KERNEL_NAMES.items():
        b.bench_layer_kernel(which, 3)  # warm
        b.sync()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        nbytes = b.bench_layer_kernel(which, args.kernel_iters)
        e1.record(stream)
        b.sync()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / args.kernel_iters
        kernels[name] = {"kernel": b.bench_kernel_name(which), "us": round(us, 2), "bytes": int(nbytes),
                         "GB_s": round(nbytes / us / 1e3, 1)}
    for k, v in kernels.items():
        log(f"[bench {config}] {k:14s} {v['kernel']:12s} {v['us']:8.2f} us  {v['bytes'] / 1e6:8.2f} MB  "
            f"{v['GB_s']:7.1f} GB/s")
    # dominant kernel: largest total time per token
    per_token = {"qkv": spec.layers, "wo": spec.layers, "gate_up": spec.layers, "down": spec.layers,
                 "output+argmax": 1, "attention": spec.layers}
    dom = max(kernels, key=lambda k: kernels[k]["us"] * per_token[k])
    d = kernels[dom]
    bytes_per_token = spec.weight_bytes_per_token()
    traffic = measured_traffic(config).get(dom)
    roofline = {"bound": "hbm", "achieved": d["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(d["GB_s"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": "calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, read from "
                                  "profiles/hbm_traffic.md (not measured in this run)",
                "kernel": f"{dom} ({d['kernel']})", "bytes_per_launch": d["bytes"],
                "avg_launch_us": d["us"]}

    # time to first token through fl_prefill (64-token int8-MFMA passes) of
    # the same prompt, against the decode-step path above
    prefill = None
    if n_prompt > 1:
        b.reset()
        b.forward_prefill(prompt[:32], logits=False)  # capture the pass graphs
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, ptok, _ = b.forward_prefill(prompt, logits=False)
        pms = (time.perf_counter() - t0) * 1000.0
        # the same prefill with logits: the top-2 gap of the last token (a
        # first token that differs from the decode path's is a near-tie of
        # two tree orders when this gap is small)
        b.reset()
        plg, _, _ = b.forward_prefill(prompt, logits=True)
        top2 = np.sort(plg)[-2:]
        prefill = {"tokens": n_prompt, "ms": round(pms, 2), "tok_s": round(n_prompt * 1000.0 / pms, 1),
                   "pass_tokens": 64, "first_token": ptok, "decode_path_first_token": int(toks[0]),
                   "top2_gap_rel": round(float((top2[1] - top2[0]) / abs(top2[1])), 5),
                   "decode_path_token_rank": int((plg > plg[int(toks[0])]).sum())}
        log(f"[bench {config}] prefill of {n_prompt} tokens: {pms:.2f} ms ({n_prompt * 1000.0 / pms:.0f} tok/s); "
            f"first token {ptok} (decode path {int(toks[0])})")
    b.close()
    if args.calibrate_copy:
        # a plain device copy of known size: its FETCH_SIZE / WRITE_SIZE
        # counters calibrate the per-kernel HBM traffic readings
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {src.numel() * 4} bytes read, {dst.numel() * 4} bytes written")
        del src, dst

    cpu = None
    if with_cpu:
        log("[bench] CPU baseline ...")
        cpu = cpu_baseline(model, spec, 4, args.cpu_tokens, 2 * args.cpu_tokens)
        log(f"[bench] CPU baseline {cpu['value']} tok/s (1 thread), {cpu['parallel']['value']} tok/s "
            f"({cpu['parallel']['cores']} threads)")
    return {
        "value": round(tok_s, 2), "ms_per_step": round(ms_per_step, 4), "spec": spec, "n_prompt": n_prompt,
        "wl": wl, "roofline": roofline, "cpu_baseline": cpu, "kernels": kernels, "prefill": prefill, "model": model,
        "decode_weight_roofline": {"bytes_per_token": bytes_per_token,
                                   "achieved_GB_s": round(bytes_per_token * tok_s / 1e9, 1),
                                   "frac": round(bytes_per_token * tok_s / 1e9 / HBM_PEAK_GBS, 4)},
    }


def run_exact(args, config: str, model=None) -> dict:
    """The same decode workload in the reference-order mode (FL_OPT_EXACT:
    logits bit-identical to the CPU reference's): the prompt through exact
    decode steps (untimed), then args.steps steps timed with HIP events."""
    import torch

    from flarellm_amd import FL_KV_F16
    from flarellm_amd import _lib as L
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    wl = WORKLOADS[config]
    spec = S.CONFIGS[wl["spec"]]
    n_prompt = wl["prompt"] if args.prompt is None else max(1, args.prompt)
    need = n_prompt + args.warmup + args.steps
    if need > spec.max_seq:
        spec = S.replace(spec, max_seq=need)
    if model is None or model.spec != spec:
        model = S.make_model(spec, seed=1)
    b = HipBackend(0)
    b.init_gpu_kv_cache(spec, FL_KV_F16)
    b.upload_weights_to_gpu(model)
    b.set_option(L.FL_OPT_EXACT, 1)
    stream = torch.cuda.ExternalStream(b.stream)
    t0 = time.time()
    b.generate(S.random_tokens(7, n_prompt, spec.vocab), 1)
    b.decode_continue(args.warmup)
    b.sync()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    b.decode_continue(args.steps)
    ev1.record(stream)
    b.sync()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    toks = b.read_tokens(n_prompt, 8)
    b.close()
    log(f"[bench {config} exact] {args.steps} steps: {1000.0 / ms:.1f} tok/s ({ms:.4f} ms/token; prompt "
        f"{time.time() - t0:.1f}s); first tokens {toks.tolist()}")
    return {"value": round(1000.0 / ms, 2), "unit": "tok/s", "ms_per_step": round(ms, 4), "steps": args.steps,
            "context": n_prompt,
            "mode": "FL_OPT_EXACT: logits bit-identical to the x86 reference's (reference summation order)"}


def c4_128k(args) -> dict:
    """BASELINE configs[3] at its longest context only (the default line's
    extra_configs): the decode attention kernel over 128k cached tokens in the
    three cache forms, from HBM (>= 1 GB of K+V rotated across layers)."""
    import numpy as np
    import torch

    from flarellm_amd import FL_KV_F16, FL_KV_KIVI2, FL_KV_Q8
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    base = S.CONFIGS["Llama-3-8B"]
    nh, nkv, hd = base.heads, base.kv_heads, base.head_dim
    T = 131072
    rng = np.random.default_rng(3)
    rows_k = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    rows_v = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    q = rng.standard_normal(nh * hd, dtype=np.float32)
    b = HipBackend(0)
    stream = torch.cuda.ExternalStream(b.stream)
    out = {}
    for name, fmt in (("f16", FL_KV_F16), ("q8", FL_KV_Q8), ("kivi2", FL_KV_KIVI2)):
        spec = S.replace(base, layers=1, max_seq=T)
        b.init_gpu_kv_cache(spec, fmt)
        nbytes = b.bench_attention(T, 0)
        L = int(min(256, max(2, -(-1.0e9 // nbytes))))
        b.init_gpu_kv_cache(S.replace(base, layers=L, max_seq=T), fmt)
        for layer in range(L):
            b.gpu_kv_write_batch(layer, 0, rows_k, rows_v)
        b.grouped_query_attention_from_gpu_cache(q, 0, T)
        b.bench_attention(T, 3)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        nbytes = b.bench_attention(T, args.kernel_iters)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / args.kernel_iters
        out[name] = {"us": round(us, 2), "bytes": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"[bench c4 128k] {name:6s} {us:8.2f} us  {nbytes / 1e6:8.2f} MB  {nbytes / us / 1e3:7.1f} GB/s")
    b.close()
    return {"workload": "decode attention alone, Llama-3-8B heads, 131072 cached tokens", "unit": "us per launch",
            "cases": out}


def c5_verify(args, model) -> dict:
    """one 8-draft verify pass at context 4096 on the
    Llama-3-8B model (the prompt through fl_prefill, untimed); ms per pass
    timed with HIP events over repeated passes at the same positions."""
    import torch

    from flarellm_amd import FL_KV_F16
    from flarellm_amd import synth as S
    from flarellm_amd.backend import HipBackend

    spec = model.spec
    n_prompt, k = 4096, 8
    b = HipBackend(0)
    b.init_gpu_kv_cache(spec, FL_KV_F16)
    b.upload_weights_to_gpu(model)
    b.forward_prefill(S.random_tokens(7, n_prompt, spec.vocab), logits=False)
    drafts = S.random_tokens(9, k, spec.vocab)
    for _ in range(3):
        b.verify(drafts, n_prompt)
    stream = torch.cuda.ExternalStream(b.stream)
    torch.cuda.synchronize()
    n = 16
    t1 = time.perf_counter()
    for _ in range(n):
        b.verify(drafts, n_prompt)
    ms = (time.perf_counter() - t1) * 1000.0 / n
    b.close()
    log(f"[bench c5] verify pass of {k} drafts at context {n_prompt}: {ms:.3f} ms ({k * 1000.0 / ms:.0f} drafts/s)")
    return {"workload": WORKLOADS["c5"]["desc"], "ms_per_pass": round(ms, 4), "unit": "drafts/s",
            "value": round(k * 1000.0 / ms, 1), "passes": n,
            "weight_roofline_frac": round(spec.weight_bytes_per_token() / ms / 1e6 / HBM_PEAK_GBS, 4),
            "timing": "host wall clock per fl_verify call (each call synchronizes for the 8 tokens)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-c3", action="store_true",
                    help="default run: skip the Llama-3-8B (C3) decode line reported under extra_configs")
    ap.add_argument("--no-extra", action="store_true",
                    help="default run: skip the exact-mode, C4 128k and C5 lines under extra_configs")
    ap.add_argument("--cpu-tokens", type=int, default=40)
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--prompt", type=int, default=None,
                    help="override the workload's prompt length (profiling runs of the weight-streaming kernels, "
                         "whose bytes do not depend on the context; the reported line names the length used)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB device copy (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the decode path "
              "would shard by output rows / KV heads, which is not built here.", file=sys.stderr)
        return 2
    if args.config == "c4":
        return bench_attention_c4(args)
    if args.config == "c5":
        return bench_verify_c5(args)
    r = run_decode(args, args.config, not args.no_cpu_baseline)
    spec, wl = r["spec"], r["wl"]
    out = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random N(0,0.02) weights quantized to GGUF blocks; uniform-random prompt)",
        "config": {"workload": wl["desc"], "model": spec.name, "global_batch": 1, "seq_len": r["n_prompt"],
                   "parallelism": "none (1 GPU)"},
        "roofline": r["roofline"],
        "cpu_baseline": r["cpu_baseline"],
        "decode_weight_roofline": r["decode_weight_roofline"],
        "prefill": r["prefill"],
        "kernels": r["kernels"],
    }
    if args.config == "c2" and not args.no_c3 and args.prompt is None:
        # the north-star shape and the other BASELINE configs, driver-timed in
        # the same run
        c3 = run_decode(args, "c3", False)
        extra = {"c3": {
            "workload": c3["wl"]["desc"], "value": c3["value"], "unit": "tok/s", "ms_per_step": c3["ms_per_step"],
            "steps": args.steps, "decode_weight_roofline": c3["decode_weight_roofline"],
            "roofline": c3["roofline"], "prefill": c3["prefill"], "kernels": c3["kernels"]}}
        if not args.no_extra:
            extra["c2_exact"] = run_exact(args, "c2")
            extra["c3_exact"] = run_exact(args, "c3", c3["model"])
            extra["c4_128k"] = c4_128k(args)
            extra["c5"] = c5_verify(args, c3["model"])
        out["extra_configs"] = extra
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
