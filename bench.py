#!/usr/bin/env python3
"""Benchmark of the decoder hot path on one MI355X.

Workload (the headline "decode ms/token"): full 28-layer greedy decode of a
random-init Qwen3-0.6B-shaped model (d=1024, 16Q/8KV heads x 128, FFN 3072,
vocab 151936), FP16 layer weights, INT8 lm_head with per-column fp32 scales,
RoPE theta 1e6 split-half, fp16 KV cache prefilled to 512 positions with
N(0,1) values; each timed step decodes one token with the argmax fed back on
the device.  A "step" is one token, which is one launch of the whole-step
kernel k_persist_step (all 28 layers, the lm_head and the argmax).  value =
tokens/s over the timed steps (host wall clock around the whole timed loop,
GPU synchronised on both sides).

Also reported: the roofline of that kernel (algorithmic bytes of a step over
its average duration, HIP events on the decoder's stream), with the HBM
traffic measured by rocprofv3 counters when its summary is present under
profiles/; the per-stage kernels of the general path (the fallback for other
shapes); and the oracle (the scalar C restatement of the reference CPU path)
timed on this host on a bounded sample of the same decode workload.  The
other workloads of the metric each get their own object under "configs":
  1  one INT8 GEMV tile 1 x 1024 x 4096 with per-column scales, 1024
     back-to-back launches over 128 rotated weight copies (541 MB), replayed
     from a captured graph of 128 launches;
  2  one fp16 layer's seven projections with their RMSNorms at M = 1 (four
     launches), cycling through the 28 layers of the decode model (a captured
     graph of the 28 layers' 112 launches, replayed);
  4  the M=60 INT8 batch prefill (28 layers, 60 tokens from an empty cache);
  5  W4A16 greedy decode at KV 4096 -> 4224 (128 steps), int4 layer weights
     with fp16 scales, INT8 lm_head.

Usage: python bench.py [--gpus 1] [--steps 64] [--warmup 8]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "rknn-matmul-parallel_amd")
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
KV_PREFILL = 512
START_TOKEN = 151644


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_dir(mdx, tag: str, cfg, quant: int, seed: int) -> str:
    base = os.environ.get("MDX_BENCH_DIR") or os.path.join(tempfile.gettempdir(), "mdx_bench")
    path = os.path.join(base, tag)
    marker = os.path.join(path, ".complete")
    if not os.path.exists(marker):
        t0 = time.time()
        os.makedirs(base, exist_ok=True)
        mdx.write_model(path, cfg, quant, seed)
        open(marker, "w").close()
        log(f"wrote {tag} in {time.time() - t0:.1f}s")
    return path


def step_bytes(d: dict, positions: list[int], quant: int = 0) -> float:
    """Algorithmic HBM bytes of one decode step (weights + lm_head + KV), mean over positions.
    quant 0: fp16 layer weights; 2: int4 weights plus fp32 per-row scales."""
    h, qd, kvd, F, L, V = d["hidden_dim"], d["num_q_heads"] * d["head_dim"], \
        d["num_kv_heads"] * d["head_dim"], d["ffn_dim"], d["num_layers"], d["vocab_size"]
    elems = h * (qd + 2 * kvd) + qd * h + 2 * h * F + F * h
    rows = (qd + 2 * kvd) + h + 2 * F + h
    layer_w = 2.0 * elems if quant == 0 else 0.5 * elems + 4.0 * rows
    norms = 4.0 * (2 * h + 2 * d["head_dim"])
    lm = V * h * 1.0 + V * 4.0
    kv = np.mean([L * (p + 1) * kvd * 2 * 2.0 for p in positions])
    return L * (layer_w + norms) + lm + kv + 4.0 * h


def cpu_info() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count()}


def run_cpu_baseline(path: str, d: dict, budget_s: float) -> dict:
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    t0 = time.time()
    m = orc.Model(path, d, 0, KV_PREFILL + 64, kv_fp16=True)
    m.kv_fill_normal(KV_PREFILL, 1003)
    log(f"oracle loaded in {time.time() - t0:.1f}s")
    n, tok, t_start = 0, START_TOKEN, time.perf_counter()
    while True:
        tok, _ = m.step(tok)
        n += 1
        el = time.perf_counter() - t_start
        if el >= budget_s or n >= 64:
            break
    m.close()
    info = cpu_info()
    return {"value": round(n / el, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "ms_per_token": round(el / n * 1000, 2),
            "sample": f"{n} greedy decode steps of the same 28-layer fp16/int8-lm_head model at KV "
                      f"{KV_PREFILL}..{KV_PREFILL + n} (oracle: scalar C restatement of the reference "
                      f"CPU path, gcc -O3, 1 thread), {el:.1f} s",
            **info}


def run_sampling(mdx, cfg, max_seq: int, args) -> int:
    """Per-step time of device-side sampling (matmul_decoder_step_sample,
    logits left on the device) against greedy steps (mdx_step_token), each
    over `--steps` steps after two untimed ones, KV refilled to 512 first."""
    path16 = model_dir(mdx, "decode_fp16_seed1003", cfg, 0, 1003)
    dec = mdx.Decoder(path16, cfg, "fp16", max_seq + 64)
    lib = mdx.lib()
    n = max(4, args.steps)

    def per_step(fn):
        dec.kv_fill_normal(KV_PREFILL, 1003)
        fn()
        fn()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return (time.perf_counter() - t0) * 1000.0 / n

    res = {"greedy_ms": round(per_step(lambda: dec.step_token(5)), 4)}
    hist = list(range(100, 164))
    for k in (40, 64, 1024):
        p, toks = mdx.sampling_params(k, 0.9, 0.8, 1.1, hist)
        res[f"top_k_{k}_ms"] = round(per_step(
            lambda: lib.matmul_decoder_step_sample(dec.h, 5, None, mdx.C.byref(p), 0.37, None)), 4)
    dec.close()
    print(json.dumps({"workload": "sampled decode step, fp16 layers, KV 512, T 0.8, top-p 0.9, "
                                  "64 penalised tokens", "steps": n, **res}), flush=True)
    return 0


def profile_traffic(name: str) -> dict | None:
    """HBM traffic of a kernel or launch sequence from the committed rocprofv3
    counter summary profiles/<name>_traffic.json (FETCH_SIZE and WRITE_SIZE
    passes scaled by a copy kernel's counts), or None."""
    path = os.path.join(ROOT, "profiles", name + "_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def layer_stage_split(traces, n_layers: int) -> dict:
    """Stage times (us) of one layer inside the one-launch step, from traced
    steps ([workgroups][events] of 100 MHz device timestamps, 16 events per
    layer): the four projection stages (input staged -> result published),
    the exchange waits before them, and the whole layer.  Medians over the 256
    workgroups, means over layers 2 .. L-3 and over the traced steps."""
    seg = {"qkv": (1, 2), "o": (6, 7), "gate_up": (8, 9), "down": (10, 11),
           "wait_h_before_qkv": (11, 17), "wait_attn_before_o": (5, 6),
           "wait_h_before_gate_up": (7, 8), "wait_act_before_down": (9, 10), "layer": (0, 16)}
    acc = {k: [] for k in seg}
    for tr in traces:
        x = np.asarray(tr, np.int64) * 0.01
        for lay in range(2, n_layers - 2):
            base = 16 * lay
            for k, (a, b) in seg.items():
                acc[k].append(float(np.median(x[:, base + b] - x[:, base + a])))
    out = {k: round(float(np.mean(v)), 3) for k, v in acc.items()}
    out["projections_sum"] = round(out["qkv"] + out["o"] + out["gate_up"] + out["down"], 3)
    out["source"] = ("mdx_trace_step: medians over 256 workgroups, mean over layers 2..25 of 3 "
                     "traced steps; wait_h_before_qkv spans the previous layer's last event to "
                     "this layer's staged input")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of oracle decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-w4", action="store_true", help="skip the W4A16 KV 4096 decode (config 5)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="counter runs: the calibration copy, then the M=60 INT8 prefill only")
    ap.add_argument("--workload", default="fp16_kv512", choices=["fp16_kv512", "w4a16_kv4096"],
                    help="decode workload: fp16 layers at KV 512 (the default line), or W4A16 at "
                         "KV 4096 (decode only)")
    ap.add_argument("--sampling", action="store_true",
                    help="sampled decode: matmul_decoder_step_sample at top-k 40, 64 and 1024 (T 0.8, "
                         "top-p 0.9, 64 penalised tokens) against greedy steps, fp16 layers at KV 512")
    ap.add_argument("--probe", action="store_true",
                    help="counter runs: a 256 MiB device copy (the calibration kernel), then the "
                         "decode steps only")
    args = ap.parse_args()
    if args.probe:
        args.no_prefill = args.no_cpu_baseline = True
    w4 = args.workload == "w4a16_kv4096"
    if w4:
        args.no_prefill = args.no_cpu_baseline = True
    kv0 = 4096 if w4 else KV_PREFILL
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decoder runs on a single MI355X and there is no "
              "multi-GPU path (the weights, 881 MB, fit one GPU's HBM many times over: independent "
              "sequences would each run on their own GPU with replicated weights, and a tensor-"
              "parallel split would cost two small all-reduces per layer); use --gpus 1.", file=sys.stderr)
        return 2

    import mdx_lib as mdx
    if mdx.device_count() <= 0:
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1

    d = dict(hidden_dim=1024, num_q_heads=16, num_kv_heads=8, head_dim=128, ffn_dim=3072,
             num_layers=28, vocab_size=151936, max_seq_len=4096, rms_eps=1e-6, rope_theta=1e6,
             tie_word_embeddings=1, has_qk_norm=1, rope_style=1, max_batch_prefill=64)
    if w4:
        d["max_seq_len"] = 4224
    cfg = mdx.qwen3_0_6b_config(name="qwen3-0.6b-synthetic", **d)
    max_seq = kv0 + max(args.steps, args.warmup) + 8

    if args.probe:
        # plain copy of a known size: the scale for the HBM byte counters
        if mdx.lib().mdx_copy_probe(1 << 28, 3) != 0:
            print("bench.py: copy probe failed", file=sys.stderr)
            return 1
        log("probe copy: 3 x 256 MiB device-to-device")

    if args.prefill_only:
        if mdx.lib().mdx_copy_probe(1 << 28, 3) != 0:
            print("bench.py: copy probe failed", file=sys.stderr)
            return 1
        path8 = model_dir(mdx, "prefill_int8_seed1004", cfg, 1, 1004)
        dec8 = mdx.Decoder(path8, cfg, "int8", 128)
        emb = mdx.synth_fill_normal(60 * 1024, mdx.synth_seed(1004, "prefill/emb")).reshape(60, 1024)
        dec8.time_prefill(emb, 2)
        pms = dec8.time_prefill(emb, max(1, args.steps))
        dec8.close()
        print(json.dumps({"workload": "M=60 INT8 prefill, 28 layers", "ms": round(pms, 4)}), flush=True)
        return 0

    if args.sampling:
        return run_sampling(mdx, cfg, max_seq, args)

    # ---- decode (config: 28-layer greedy, FP16 layers + INT8 lm_head, KV 512) ----
    path16 = model_dir(mdx, "decode_int4_seed1005" if w4 else "decode_fp16_seed1003", cfg,
                       2 if w4 else 0, 1005 if w4 else 1003)
    t0 = time.time()
    dec = mdx.Decoder(path16, cfg, "int4" if w4 else "fp16", max_seq)
    log(f"decoder created in {time.time() - t0:.1f}s")
    dec.kv_fill_normal(kv0, 1003)
    dec.generate_greedy(START_TOKEN, args.warmup)
    dec.kv_fill_normal(kv0, 1003)
    t0 = time.perf_counter()
    toks, dev_ms = dec.generate_greedy(START_TOKEN, args.steps)
    wall_s = time.perf_counter() - t0
    ms_per_step = wall_s * 1000.0 / args.steps
    positions = list(range(kv0, kv0 + args.steps))
    bytes_step = step_bytes(d, positions, 2 if w4 else 0)
    log(f"decode: {ms_per_step * 1000:.1f} us/token wall, {dev_ms * 1000 / args.steps:.1f} us/token device")

    # API-level latency: matmul_decoder_step with the logits copied to the host each
    # token, into one caller-owned buffer (a fresh array per step would add the
    # first-touch page faults of 607 KB to every step)
    api_ms = None
    if not args.probe:
        dec.kv_fill_normal(kv0, 1003)
        logits = np.empty(d["vocab_size"], np.float32)
        dec.step_into(START_TOKEN, logits)   # untimed: the first logits copy sets up the copy path
        dec.kv_fill_normal(kv0, 1003)
        tok, t0 = START_TOKEN, time.perf_counter()
        n_api = min(args.steps, 32)
        for _ in range(n_api):
            tok = dec.step_into(tok, logits)
        api_ms = round((time.perf_counter() - t0) * 1000.0 / n_api, 4)

    # per-projection kernels of the per-stage path (each launch cycles through
    # the 28 layers' weights)
    kernels = {}
    for name, per_step in () if args.probe or w4 else (("qkv", 28), ("o", 28), ("gate_up", 28),
                                                 ("down", 28), ("lm_head", 1)):
        iters = 280 if per_step == 28 else 40
        dec.time_projection(name, 28)
        us, b = dec.time_projection(name, iters)
        kernels[name] = {"avg_us": round(us, 3), "bytes": b, "GBps": round(b / us / 1e3, 1),
                         "per_step_us": round(us * per_step, 1)}
    layer_us = layer_bytes = None
    if not args.probe and not w4:
        dec.time_projection("layer", 28)
        layer_us, layer_bytes = dec.time_projection("layer", 280)
    # the same projections inside the one-launch step (the path the decode
    # figure runs): stage times from traced steps
    one_launch_stages = None
    if not args.probe and not w4 and dec.path == 1:
        dec.kv_fill_normal(kv0, 1003)
        dec.trace_step(START_TOKEN)
        one_launch_stages = layer_stage_split([dec.trace_step(START_TOKEN) for _ in range(3)],
                                              d["num_layers"])
    path_kind = dec.path
    dec.close()
    step_us = dev_ms * 1000.0 / args.steps
    traffic = None
    tdoc = None if w4 else profile_traffic("k_persist_step_fp16_decode_kv512")
    if tdoc:
        traffic = tdoc.get("hbm_bytes_per_launch")

    configs = {}
    if not args.probe and not w4:
        # ---- config 2: one fp16 layer's projections at M=1 (per-stage kernels) ----
        us, b = layer_us, layer_bytes
        configs["2_fp16_layer_projections_m1"] = {
            "avg_us": round(us, 3), "bytes": b, "GBps": round(b / us / 1e3, 1),
            "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
            "kernels": "k_gemv: RMSNorm+q|k|v, o+residual, RMSNorm+gate|up+SwiGLU, down+residual",
            "rotation": "28 layers' distinct weights (881 MB), launches replayed from a captured graph",
            "one_launch_stages": one_launch_stages}
        log(f"config 2 layer projections: {us:.2f} us, {b / us / 1e3:.0f} GB/s")
        # ---- config 1: the INT8 lm_head tile GEMV 1 x 1024 x 4096 ----
        us1 = mdx.time_gemv(1, 1024, 4096, 128, 1024)
        b1 = 1024 * 4096 + 4.0 * 4096 + 4.0 * 1024 + 4.0 * 4096
        configs["1_int8_tile_gemv_1x1024x4096"] = {
            "avg_us": round(us1, 3), "bytes": b1, "GBps": round(b1 / us1 / 1e3, 1),
            "hbm_frac": round(b1 / us1 / 1e3 / HBM_PEAK_GBS, 4),
            "kernels": "k_gemv<int8> (fp32 x rounded to fp16, per-column scales)",
            "rotation": "1024 launches over 128 weight copies (541 MB), replayed from a captured graph"}
        log(f"config 1 int8 tile GEMV: {us1:.2f} us, {b1 / us1 / 1e3:.0f} GB/s")
        # ---- the same GEMV kernel where a launch is not dominated by its fixed
        # cost: 1 x 1024 x 151936 (a vocabulary-sized matrix), weights rotated
        # over more than the 256 MB last-level cache ----
        gl = {}
        for kind, name, copies in ((0, "fp16", 2), (1, "int8", 4)):
            usl = mdx.time_gemv(kind, 1024, 151936, copies, 8 * copies)
            # weights + column scales + x + y, as for config 1
            bl = (2 if kind == 0 else 1) * 1024 * 151936 + 4.0 * 151936 + 4.0 * 1024 + 4.0 * 151936
            gl[name] = {"avg_us": round(usl, 2), "bytes": bl, "GBps": round(bl / usl / 1e3, 1),
                        "hbm_frac": round(bl / usl / 1e3 / HBM_PEAK_GBS, 4),
                        "rotation": f"{8 * copies} launches over {copies} weight copies "
                                    f"({copies * bl / 1e6:.0f} MB), replayed from a captured graph"}
            log(f"k_gemv {name} 1x1024x151936: {usl:.2f} us, {bl / usl / 1e3:.0f} GB/s")
        configs["gemv_1x1024x151936"] = gl

    # ---- batch prefill M=60 through 28 INT8 layers ----
    prefill = None
    if not args.no_prefill:
        path8 = model_dir(mdx, "prefill_int8_seed1004", cfg, 1, 1004)
        dec8 = mdx.Decoder(path8, cfg, "int8", 128)
        emb = mdx.synth_fill_normal(60 * 1024, mdx.synth_seed(1004, "prefill/emb")).reshape(60, 1024)
        dec8.time_prefill(emb, 3)
        pms = dec8.time_prefill(emb, 20)
        layer_bytes = 28 * (1.0 * (1024 * 4096 + 2048 * 1024 + 2 * 1024 * 3072 + 3072 * 1024)
                            + 4.0 * (4096 + 1024 + 6144 + 1024) + 4.0 * (2 * 1024 + 256))
        flops = 2.0 * 60 * 28 * (1024 * 4096 + 2048 * 1024 + 2 * 1024 * 3072 + 3072 * 1024)
        dec8.close()
        ptr = profile_traffic("k_gemm_prefill_m60_int8")
        prefill = {"ms": round(pms, 4), "tokens": 60,
                   "hbm_frac_layers": round(layer_bytes / (pms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "mfma_frac_layers": round(flops / (pms * 1e-3) / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4),
                   "algorithmic_bytes": layer_bytes,
                   "traffic": ptr["hbm_bytes_per_prefill"] if ptr else None,
                   "traffic_source": ("profiles/k_gemm_prefill_m60_int8_traffic.json: rocprofv3 FETCH_SIZE "
                                      "and WRITE_SIZE passes over the same prefill, scaled by a copy "
                                      "kernel's counts (not this run)") if ptr else None,
                   "note": "28 INT8 layers, causal GQA over 60 positions, device time (HIP events)"}
        log(f"prefill M=60: {pms:.3f} ms")

    if prefill:
        configs["4_prefill_m60_int8"] = prefill

    # ---- config 5: W4A16 greedy decode at KV 4096 (128 steps) ----
    if not args.probe and not w4 and not args.no_w4:
        d5 = dict(d, max_seq_len=4224)
        cfg5 = mdx.qwen3_0_6b_config(name="qwen3-0.6b-synthetic-w4", **d5)
        path4 = model_dir(mdx, "decode_int4_seed1005", cfg5, 2, 1005)
        n5, w5 = 128, 8
        dec4 = mdx.Decoder(path4, cfg5, "int4", 4096 + n5 + w5)
        dec4.kv_fill_normal(4096, 1005)
        dec4.generate_greedy(START_TOKEN, w5)
        dec4.kv_fill_normal(4096, 1005)
        t0 = time.perf_counter()
        toks5, dev5 = dec4.generate_greedy(START_TOKEN, n5)
        wall5 = time.perf_counter() - t0
        dec4.close()
        b5 = step_bytes(d5, list(range(4096, 4096 + n5)), 2)
        tr5 = profile_traffic("k_persist_step_int4_decode_kv4096")
        us5 = dev5 * 1000.0 / n5
        configs["5_w4a16_decode_kv4096"] = {
            "ms_per_token": round(wall5 * 1000.0 / n5, 5), "tokens_per_s": round(n5 / wall5, 2),
            "steps": n5, "kv": f"4096->{4096 + n5}",
            "roofline": {"bound": "hbm", "kernel": "k_persist_step<i4>", "avg_us": round(us5, 2),
                         "bytes_per_launch": b5, "achieved": round(b5 / (us5 * 1e-6) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(b5 / (us5 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": tr5["hbm_bytes_per_launch"] if tr5 else None,
                         "traffic_source": ("profiles/k_persist_step_int4_decode_kv4096_traffic.json: "
                                            "rocprofv3 FETCH_SIZE and WRITE_SIZE passes over the same "
                                            "kernel at KV 4096..4105, scaled by a copy kernel's counts "
                                            "(not this run)") if tr5 else None},
            "tokens_head": toks5[:8]}
        log(f"config 5 W4A16 KV 4096: {wall5 * 1000.0 / n5 * 1000:.1f} us/token wall, {us5:.1f} us device")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = run_cpu_baseline(path16, d, args.cpu_budget)
        log(f"cpu baseline: {cpu['ms_per_token']} ms/token")

    line = {
        "metric": "decode ms/token + M=60 prefill ms, 0.6B/28L shape; GEMV HBM GB/s",
        "value": round(args.steps / wall_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i4 x f16" if w4 else "f16",
        "data": "synthetic (seeded random-init Qwen3-0.6B-shaped weights and N(0,1) KV)",
        "config": {"workload": f"28-layer greedy decode, {'int4 (W4A16)' if w4 else 'fp16'} layers + "
                               f"int8 lm_head, fp16 KV {kv0}->{kv0 + args.steps}, 1 token per step, "
                               "argmax fed back on device",
                   "hidden": 1024, "heads": "16q/8kv x128", "ffn": 3072, "vocab": 151936,
                   "kv_start": kv0, "start_token": START_TOKEN},
        "roofline": {"bound": "hbm",
                     "kernel": f"k_persist_step<{'i4' if w4 else 'f16'}> (one launch per token: 28 "
                               "layers + INT8 lm_head + argmax)" if path_kind == 1 else
                               "per-stage kernel sequence (one-launch step unavailable)",
                     "achieved": round(bytes_step / (step_us * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes_step / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": ("profiles/k_persist_step_fp16_decode_kv512_traffic.json: "
                                        "rocprofv3 FETCH_SIZE and WRITE_SIZE passes over the same "
                                        "kernel at KV 512..520, scaled by a copy kernel's counts "
                                        "(not this run)") if traffic else None,
                     "bytes_per_launch": bytes_step, "avg_us": round(step_us, 2)},
        "wall_roofline_frac": round(bytes_step / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "api_step_ms": api_ms,
        "per_stage_path_kernels": kernels,
        "prefill_m60": prefill,
        "configs": configs,
        "cpu_baseline": cpu,
        "tokens_head": toks[:8],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
