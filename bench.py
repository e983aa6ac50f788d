#!/usr/bin/env python3
"""Benchmark of the MI355X quantized MoE FFN layer (one GPU).

A step is one MoE FFN layer call (hip_moe_ffn_dev) over one batch of
synthetic tokens whose activations are already resident in HBM.  The default
workload is the OLMoE-1B-7B-shaped decode layer: d_model 2048, 64 experts,
top-8 softmax routing without renormalisation, SwiGLU d_ff 1024, Q8_0 expert
weights drawn N(0, 0.02), fp32 router, one token per call.

The selected experts of one call (~53.5 MB) fit in MI355X's 256 MB
Infinity Cache, so the timed loop rotates over `--layers` copies of the layer
(distinct device allocations, like the 16 layers of the full model) and over
distinct tokens: consecutive calls touch different memory and the figure is
an HBM figure.  Calls are replayed from HIP graphs of one call per layer copy.

The `*_lm_head` workloads time the dense quantized product instead
(hip_moe_qmat_mul_dev: the reference's tensor_mma_transposed_2x2 on a Q8_0 or
Q4_0 matrix, here the lm_head of each model for one token), rotating over
`--layers` copies of the matrix in the same way.

Prints one JSON line on stdout (progress goes to stderr).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "llm.c_amd"))
import hipmoe  # noqa: E402

METRIC = "MoE-layer tokens/s & % of HBM roofline; OLMoE-shaped decode tok/s"
QMAT_METRIC = "dense quantized product tokens/s & % of HBM roofline"
HBM_PEAK_GBS = 8000.0
SEED = 1337

WORKLOADS = {
    "olmoe_q8_decode": dict(wtype=hipmoe.Q8_0, E=2048, EI=1024, NE=64, K=8, renorm=0, T=1,
                            bias_std=None),
    "olmoe_q4_prefill512_skew": dict(wtype=hipmoe.Q4_0, E=2048, EI=1024, NE=64, K=8, renorm=0,
                                     T=512, bias_std=1.0),
    "mixtral_q4_decode": dict(wtype=hipmoe.Q4_0, E=4096, EI=14336, NE=8, K=2, renorm=1, T=1,
                              bias_std=None),
    "mixtral_q4_T16": dict(wtype=hipmoe.Q4_0, E=4096, EI=14336, NE=8, K=2, renorm=1, T=16,
                           bias_std=None),
    "mixtral_q4_T64": dict(wtype=hipmoe.Q4_0, E=4096, EI=14336, NE=8, K=2, renorm=1, T=64,
                           bias_std=None),
    # dense quantized products: N rows of K columns, T tokens
    "olmoe_q8_lm_head": dict(kind="qmat", wtype=hipmoe.Q8_0, N=50304, Kc=2048, T=1),
    "mixtral_q4_lm_head": dict(kind="qmat", wtype=hipmoe.Q4_0, N=32000, Kc=4096, T=1),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(w):
    return 2 * w["EI"] * hipmoe.row_bytes(w["wtype"], w["E"]) + \
        w["E"] * hipmoe.row_bytes(w["wtype"], w["EI"])


def cpu_baseline(lw, w, xs, seconds):
    """The oracle (a C restatement of the reference's AVX2 CPU path) on this
    host, one thread: the reference runs the OLMoE router (T < 64) and the
    expert FFN (2*2048*1024 flops < 16 Mi, thread_pool.c:25,178-185) on one
    thread.  Bounded by `seconds`."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    T = w["T"]
    sample_T = min(T, 8)
    done_tokens = 0
    t0 = time.perf_counter()
    i = 0
    while True:
        x = xs[i % len(xs)][:sample_T]
        oracle.moe_ffn(x, lw, w["K"], bool(w["renorm"]), lw["bias"], nthreads=1)
        done_tokens += sample_T
        i += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return dict(value=done_tokens / el, unit="tokens/s", cores=1, kind="port",
                sample=f"{done_tokens} tokens in {i} layer calls of {sample_T} token(s), "
                       f"{el:.1f} s, 1 thread, oracle/moe_oracle.c built -O3 -mavx2 -mfma")


def traffic_bytes(kernel, workload):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, each divided by the
    factor the same counter reads for a copy of known size), from the
    committed counter summary of this kernel and workload, or None."""
    path = os.path.join(REPO, "profiles", f"{kernel}.{workload}.pmc.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def bench_qmat(args, w, H):
    """Dense quantized product: out[T][N] = x[T][K] . W^T per call, W one of
    `--layers` copies in turn.  Algorithmic bytes per call: the matrix's
    blocks + x + out."""
    wt, N, Kc, T = w["wtype"], w["N"], w["Kc"], w["T"]
    q = hipmoe.synth_quant_matrix(SEED, 0x7700 + wt, 0.02, wt, N, Kc)
    nl = max(1, args.layers)
    mats = [hipmoe.QMat(q, wt, N, Kc) for _ in range(nl)]
    log(f"uploaded {nl} matrix copies ({nl * mats[0].bytes() / 1e9:.2f} GB)")
    ntok = max(1, args.tokens)
    xs = [hipmoe.synth_input(SEED, 2000 + i, T, Kc) for i in range(ntok)]
    d_x = H.upload(np.stack(xs))
    d_out = H.malloc(T * N * 4)
    s = H.stream()
    xbytes = T * Kc * 4
    bytes_per_call = mats[0].bytes() + xbytes + T * N * 4

    def call(i):
        mats[i % nl].mul_dev(d_x + (i % ntok) * xbytes, T, d_out, None, 0, s)

    if args.copy_calib_mb > 0:
        nb = args.copy_calib_mb << 20
        c_src, c_dst = H.malloc(nb), H.malloc(nb)
        for _ in range(4):
            if hipmoe.lib().hip_moe_copy_dev(c_src, c_dst, nb, s) != 1:
                sys.exit("hip_moe_copy_dev: " + hipmoe.last_error())
        H.stream_sync(s)
        H.free(c_src)
        H.free(c_dst)
        log(f"copy calibration: 4 x {nb} bytes")
    for i in range(max(nl, args.warmup)):
        call(i)
    H.stream_sync(s)
    graphs = []
    if not args.eager:
        ngraphs = max(1, min(4, ntok // nl)) if ntok >= nl else 1
        for g in range(ngraphs):
            H.begin_capture(s)
            for i in range(nl):
                call(g * nl + i)
            graphs.append(H.end_capture(s))
        for ge in graphs:
            H.graph_launch(ge, s)
        H.stream_sync(s)
        log(f"captured {len(graphs)} graphs of {nl} calls")
    steps = args.steps
    e0, e1 = H.event(), H.event()
    H.sync()
    H.record(e0, s)
    if graphs:
        full, rem = divmod(steps, nl)
        for r in range(full):
            H.graph_launch(graphs[r % len(graphs)], s)
        for i in range(rem):
            call(i)
    else:
        for i in range(steps):
            call(i)
    H.record(e1, s)
    ms = H.elapsed_ms(e0, e1)
    H.sync()
    ms_per_step = ms / steps
    tokens_per_s = steps * T / (ms / 1e3)
    achieved_gbs = bytes_per_call / (ms_per_step / 1e3) / 1e9
    log(f"{steps} steps in {ms:.2f} ms: {ms_per_step * 1e3:.2f} us/step, "
        f"{tokens_per_s:.1f} tokens/s, {achieved_gbs:.1f} GB/s algorithmic")

    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle
        done, i, t0 = 0, 0, time.perf_counter()
        while True:
            oracle.qmat_mul(xs[i % ntok], q, wt, N, Kc)
            done += T
            i += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds:
                break
        cpu = dict(value=done / el, unit="tokens/s", cores=1, kind="port",
                   sample=f"{done} tokens in {i} calls, {el:.1f} s, 1 thread, "
                          f"oracle/moe_oracle.c orc_qmat_mul built -O3 -mavx2 -mfma")
        log(f"cpu baseline: {cpu['value']:.2f} tokens/s")
    line = {
        "metric": QMAT_METRIC, "value": round(tokens_per_s, 2), "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.workload, "rows": N, "cols": Kc, "tokens_per_call": T,
                   "weights": "Q8_0" if wt == hipmoe.Q8_0 else "Q4_0",
                   "matrix_copies": nl, "distinct_inputs": ntok, "graphs": bool(graphs),
                   "algorithmic_bytes_per_call": int(bytes_per_call)},
        "roofline": {"bound": "hbm", "kernel": "k_qgemv", "achieved": round(achieved_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes("k_qgemv", args.workload)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--workload", default="olmoe_q8_decode", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=16, help="layer copies rotated over")
    ap.add_argument("--tokens", type=int, default=64, help="distinct token batches")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch without HIP graphs")
    ap.add_argument("--copy-calib-mb", type=int, default=0,
                    help="before warmup, run a plain device copy of this many MiB four "
                         "times (its byte counters calibrate the kernels' counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the MoE path here runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    w = WORKLOADS[args.workload]
    H = hipmoe.hip()
    if H.device_count() < 1:
        sys.exit("no HIP device")
    if w.get("kind") == "qmat":
        return bench_qmat(args, w, H)
    E, T, K = w["E"], w["T"], w["K"]

    t0 = time.perf_counter()
    lw = hipmoe.synth_layer(SEED, 0, w["wtype"], E, w["EI"], w["NE"], 0.02, w["bias_std"])
    log(f"generated layer in {time.perf_counter() - t0:.1f} s")
    nl = max(1, args.layers)
    layers = [hipmoe.MoeLayer.from_synth(lw, K, bool(w["renorm"])) for _ in range(nl)]
    log(f"uploaded {nl} layer copies ({nl * layers[0].weight_bytes() / 1e9:.2f} GB)")

    ntok = max(1, args.tokens)
    xs = [hipmoe.synth_input(SEED, 1000 + i, T, E) for i in range(ntok)]
    d_x = H.upload(np.stack(xs))
    d_bias = H.upload(lw["bias"]) if lw["bias"] is not None else None
    d_out = H.malloc(T * E * 4)
    s = H.stream()
    xbytes = T * E * 4

    def call(i):
        layers[i % nl].ffn_dev(d_x + (i % ntok) * xbytes, d_out, T, d_bias, None, None, s)

    # algorithmic bytes: the unique experts each call touches, the router, x and out
    uniq = []
    for i in range(ntok):
        _, _, ids, _ = layers[0].route(xs[i], lw["bias"])
        uniq.append(len(np.unique(ids)))
    router_bytes = w["NE"] * E * 4
    bytes_per_call = float(np.mean(uniq)) * expert_bytes(w) + router_bytes + 2 * xbytes

    if args.copy_calib_mb > 0:
        nb = args.copy_calib_mb << 20
        c_src, c_dst = H.malloc(nb), H.malloc(nb)
        for _ in range(4):
            if hipmoe.lib().hip_moe_copy_dev(c_src, c_dst, nb, s) != 1:
                sys.exit("hip_moe_copy_dev: " + hipmoe.last_error())
        H.stream_sync(s)
        H.free(c_src)
        H.free(c_dst)
        log(f"copy calibration: 4 x {nb} bytes")

    for i in range(nl):  # every copy allocates its scratch before any capture
        call(i)
    for i in range(args.warmup):
        call(i)
    H.stream_sync(s)
    log(f"warmup {args.warmup} calls done")

    graphs = []
    if not args.eager:
        G = nl
        ngraphs = max(1, min(4, ntok // G)) if ntok >= G else 1
        for g in range(ngraphs):
            H.begin_capture(s)
            for i in range(G):
                layers[i].ffn_dev(d_x + ((g * G + i) % ntok) * xbytes, d_out, T, d_bias,
                                  None, None, s)
            graphs.append(H.end_capture(s))
        for ge in graphs:  # warm the graphs
            H.graph_launch(ge, s)
        H.stream_sync(s)
        log(f"captured {len(graphs)} graphs of {G} calls")

    steps = args.steps
    e0, e1 = H.event(), H.event()
    H.sync()
    H.record(e0, s)
    if graphs:
        G = nl
        full, rem = divmod(steps, G)
        for r in range(full):
            H.graph_launch(graphs[r % len(graphs)], s)
        for i in range(rem):
            call(i)
    else:
        for i in range(steps):
            call(i)
    H.record(e1, s)
    ms = H.elapsed_ms(e0, e1)
    H.sync()
    ms_per_step = ms / steps
    tokens_per_s = steps * T / (ms / 1e3)
    achieved_gbs = bytes_per_call / (ms_per_step / 1e3) / 1e9
    log(f"{steps} steps in {ms:.2f} ms: {ms_per_step * 1e3:.2f} us/step, "
        f"{tokens_per_s:.1f} tokens/s, {achieved_gbs:.1f} GB/s algorithmic")

    # the path the library takes for this T: one launch of k_moe_decode, or
    # router, top-k, sort and the grouped GEMMs, or router, top-k, GEMVs
    path = layers[0].path_for(T)
    # (layer_grouped / layer_gemv: the whole call, whose kernels the counter
    # summaries add up)
    kernel = {hipmoe.PATH_DECODE: "k_moe_decode",
              hipmoe.PATH_GROUPED: "layer_grouped",
              hipmoe.PATH_GEMV: "layer_gemv"}[path]

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(lw, w, xs, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.2f} tokens/s")

    line = {
        "metric": METRIC,
        "value": round(tokens_per_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": args.workload,
            "d_model": E, "experts": w["NE"], "topk": K, "d_ff": w["EI"],
            "weights": "Q8_0" if w["wtype"] == hipmoe.Q8_0 else "Q4_0",
            "tokens_per_call": T, "renorm": bool(w["renorm"]),
            "router_bias_std": w["bias_std"], "layer_copies": nl, "distinct_inputs": ntok,
            "graphs": bool(graphs),
            "mean_unique_experts": round(float(np.mean(uniq)), 3),
            "algorithmic_bytes_per_call": int(bytes_per_call),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(kernel, args.workload),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
