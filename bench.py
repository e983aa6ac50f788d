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
(hip_moe_qmat_mul_dev: the reference's tensor_mma_transposed_2x2 on a Q8_0,
Q4_0, Q4_K or Q6_K matrix, here the lm_head of each model for one token),
rotating over `--layers` copies of the matrix in the same way.

`olmoe_full_decode` times the whole OLMoE-1B-7B-shaped model (hip_lm.h: 16
layers, d_model 2048, 16 heads of 128, 64 experts top-8 d_ff 1024, vocab
50304, Q8_0 weights N(0, 0.02), unit norms, fp32 KV cache of context 2048)
decoding greedily after a 16-token random-id prompt: a step is one
generated token, the whole step (embedding to greedy pick) replayed from a
captured HIP graph with the token fed back on the device;
`olmoe_q4km_full_decode` the same model with its tensors' block types mixed as
a Q4_K_M file mixes them (Q4_K; Q6_K output, and attn_v and the experts' down
in 8 of the 16 layers).
`mixtral_full_decode` does the same for the Mixtral-8x7B shape after a
1024-token prompt, and `mixtral_full_decode_b16` for sixteen sequences in
lockstep (hip_lm_batch_*: each step one token of every sequence, their own
KV caches, the MoE layer at T = 16): tokens/s counts all sixteen.

The CPU baseline runs in a process of its own (oracle/cpu_baseline.py): the
oracle with the reference's threading on this host's cores, after the GPU
measurement.

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
    # K-quant experts as a Q4_K_M file mixes them: Q4_K gate/up, Q6_K down
    "olmoe_q4km_decode": dict(wtype=hipmoe.Q4_K | hipmoe.Q6_K << 8, E=2048, EI=1024, NE=64, K=8,
                              renorm=0, T=1, bias_std=None),
    "mixtral_q4km_decode": dict(wtype=hipmoe.Q4_K | hipmoe.Q6_K << 8, E=4096, EI=14336, NE=8,
                                K=2, renorm=1, T=1, bias_std=None),
    # dense quantized products: N rows of K columns, T tokens
    "olmoe_q8_lm_head": dict(kind="qmat", wtype=hipmoe.Q8_0, N=50304, Kc=2048, T=1),
    "mixtral_q4_lm_head": dict(kind="qmat", wtype=hipmoe.Q4_0, N=32000, Kc=4096, T=1),
    # K-quant matrices (the Q8_K path, bit-exact): the lm_head of a Q4_K_M
    # Mixtral file is Q6_K; OLMoE's as Q4_K
    "mixtral_q6k_lm_head": dict(kind="qmat", wtype=hipmoe.Q6_K, N=32000, Kc=4096, T=1),
    "olmoe_q4k_lm_head": dict(kind="qmat", wtype=hipmoe.Q4_K, N=50304, Kc=2048, T=1),
    # the whole model, one generated token per step
    "olmoe_full_decode": dict(kind="model", arch="olmoe", wtype=hipmoe.Q8_0, layers=16, E=2048,
                              H=16, KH=16, V=50304, NE=64, K=8, EI=1024, C=2048, prompt=16),
    # the same model with its tensors' types mixed as a Q4_K_M file mixes
    # them (hiplm.q4_k_m_types): every product through Q8_K activations
    "olmoe_q4km_full_decode": dict(kind="model", arch="olmoe", wtype=hipmoe.Q4_K, q4km=True,
                                   layers=16, E=2048, H=16, KH=16, V=50304, NE=64, K=8,
                                   EI=1024, C=2048, prompt=16),
    "mixtral_full_decode": dict(kind="model", arch="mixtral", wtype=hipmoe.Q4_0, layers=32,
                                E=4096, H=32, KH=8, V=32000, NE=8, K=2, EI=14336, C=4096,
                                prompt=1024, window=0, theta=1e6),
    # sixteen sequences in lockstep (hip_lm_batch_*): each step one token of
    # each, 1024-token prompts
    "mixtral_full_decode_b16": dict(kind="model", arch="mixtral", wtype=hipmoe.Q4_0, layers=32,
                                    E=4096, H=32, KH=8, V=32000, NE=8, K=2, EI=14336, C=4096,
                                    prompt=1024, window=0, theta=1e6, nseq=16),
}
MODEL_METRIC = "full-model decode tok/s & % of HBM roofline"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(w):
    gt, dt = hipmoe.wtypes(w["wtype"])
    return 2 * w["EI"] * hipmoe.row_bytes(gt, w["E"]) + w["E"] * hipmoe.row_bytes(dt, w["EI"])


def type_name(wtype):
    names = {hipmoe.Q8_0: "Q8_0", hipmoe.Q4_0: "Q4_0", hipmoe.Q4_K: "Q4_K", hipmoe.Q6_K: "Q6_K"}
    gt, dt = hipmoe.wtypes(wtype)
    return names[gt] if gt == dt else f"{names[gt]} gate/up, {names[dt]} down"


def cpu_baseline(w, seconds):
    """The oracle (a C restatement of the reference's AVX2 CPU path) timed on
    this host's cores with the reference's threading, in a process of its
    own (oracle/cpu_baseline.py), over a bounded sample of `seconds`."""
    import subprocess
    spec = {k: v for k, v in w.items()}
    spec.setdefault("kind", "moe")
    if spec["kind"] == "model":
        spec["gen"] = 256
    cmd = [sys.executable, os.path.join(REPO, "oracle", "cpu_baseline.py"),
           "--spec", json.dumps(spec), "--seconds", str(seconds)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600 + 4 * seconds)
    if r.returncode != 0:
        log(f"cpu baseline failed ({r.returncode}): {r.stderr.strip()[-400:]}")
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


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
    kquant = wt in (hipmoe.Q4_K, hipmoe.Q6_K)
    # a Q6_K single token of up to 8192 columns (a multiple of 2048) streams
    # through the LDS ring kernel; other K-quant products take the register one
    ring = wt == hipmoe.Q6_K and T == 1 and Kc % 2048 == 0 and Kc <= 8192
    kname = ("k_kq_stream" if ring else "k_kq_gemv") if kquant else "k_qgemv"
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
        log(f"cpu baseline ({args.cpu_seconds:.0f} s, own process)")
        cpu = cpu_baseline(w, args.cpu_seconds)
        if cpu:
            log(f"cpu baseline: {cpu['value']:.2f} tokens/s on {cpu['cores']} threads")
    line = {
        "metric": QMAT_METRIC, "value": round(tokens_per_s, 2), "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8" if kquant else "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "rows": N, "cols": Kc, "tokens_per_call": T,
                   "weights": {hipmoe.Q8_0: "Q8_0", hipmoe.Q4_0: "Q4_0", hipmoe.Q4_K: "Q4_K",
                               hipmoe.Q6_K: "Q6_K"}[wt],
                   "matrix_copies": nl, "distinct_inputs": ntok, "graphs": bool(graphs),
                   "algorithmic_bytes_per_call": int(bytes_per_call)},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes(kname, args.workload)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_model(args, w, H):
    """The whole model: `--steps` greedy tokens after the prompt, every step
    from a replayed graph, timed with HIP events on the model's stream (by
    hip_lm_generate).  Algorithmic bytes per token: per layer the q/k/v and
    output matrices, the router, the unique experts the token's routing
    picked and the KV rows attention reads (k and v, 4 bytes, at the step's
    cache length); then the lm_head and one embedding row."""
    import hiplm
    wt, Lh, E, V, NE, K, EI, Cx = (w["wtype"], w["layers"], w["E"], w["V"], w["NE"], w["K"],
                                   w["EI"], w["C"])
    H, KH = w["H"], w["KH"]
    t0 = time.perf_counter()
    types = hiplm.q4_k_m_types(Lh) if w.get("q4km") else None
    if w["arch"] == "olmoe":
        md = hiplm.synth_olmoe(SEED, Lh, E, H, V, NE, K, EI, wt, types=types)
    else:
        # 32 layers of 8 Mixtral experts are ~26 GB of Q4_0: the layers share
        # one generated set of values on the host, each uploaded to its own
        # device memory (the bytes a step streams are those of 32 layers)
        md = hiplm.synth_mixtral(SEED, Lh, E, H, KH, V, NE, K, EI, wt, theta=w["theta"],
                                 window=w["window"], share_layers=True)
    prompt = hiplm.synth_prompt(SEED, w["prompt"], V)
    nseq = w.get("nseq", 1)
    log(f"generated the model in {time.perf_counter() - t0:.1f} s")
    M = hiplm.LmModel(md, Cx)
    log(f"uploaded ({M.weight_bytes() / 1e9:.2f} GB on the device)")
    steps, warm = args.steps, max(1, args.warmup)
    if w["prompt"] + steps + 1 > Cx:
        sys.exit(f"--steps {steps} runs past the context {Cx}")
    # unique experts per layer and step, from eager steps' routing traces: one
    # token's, or (several sequences) the union over nseq tokens of
    # single-sequence steps
    traces = []
    tok = 0
    for i, t in enumerate(list(prompt[:16]) + [None] * max(8, nseq)):
        tok, _ = M.decode(int(t) if t is not None else tok)
        if t is None:
            traces.append(M.trace()[1])
    if nseq == 1:
        mean_uniq = float(np.mean([[len(np.unique(r)) for r in tr] for tr in traces]))
    else:
        tr = np.stack(traces[:nseq])  # [nseq][layers][K]
        mean_uniq = float(np.mean([len(np.unique(tr[:, l])) for l in range(Lh)]))
    M.reset()
    if nseq == 1 and args.eager:
        # for kernel traces: the same steps launched one kernel at a time,
        # each synchronised by the host-pointer entry point
        log(f"eager: {w['prompt']} prompt steps, then {steps} timed")
        tok = 0
        for t in prompt:
            tok, _ = M.decode(int(t))
        for i in range(warm):
            tok, _ = M.decode(tok)
        t1 = time.perf_counter()
        for i in range(steps):
            tok, _ = M.decode(tok)
        ms = (time.perf_counter() - t1) * 1e3
    elif nseq == 1:
        M.generate(prompt[:16], warm)  # captures the step graphs of short contexts
        M.reset()
        toks, ms = M.generate(prompt, steps)
    else:
        prompts = np.stack([prompt] + [hiplm.synth_prompt(SEED + 1 + q, w["prompt"], V)
                                       for q in range(1, nseq)])
        Bt = hiplm.LmBatch(M, nseq)
        if args.eager:
            # for kernel traces (the profiler's trace of replayed step graphs
            # fails): the same steps launched one kernel at a time, each step
            # synchronised by the host-pointer entry point
            log(f"{nseq} sequences, eager: {w['prompt']} prompt steps, then {steps} timed")
            for i in range(w["prompt"]):
                nxt, _ = Bt.decode(prompts[:, i])
            for i in range(warm):
                nxt, _ = Bt.decode(nxt)
            t1 = time.perf_counter()
            for i in range(steps):
                nxt, _ = Bt.decode(nxt)
            ms = (time.perf_counter() - t1) * 1e3
        else:
            Bt.generate(prompts[:, :16], warm)
            Bt.reset()
            log(f"{nseq} sequences: {w['prompt']} prompt steps, then {steps} timed")
            toks, ms = Bt.generate(prompts, steps)
        Bt.free()
    ms_per_step = ms / steps
    tokens_per_s = nseq * steps / (ms / 1e3)
    EQ, EKV = H * 128, KH * 128
    kv_rows = np.mean([w["prompt"] + s + 1 for s in range(1, steps + 1)])

    def tb(t, rows, cols):  # bytes of a rows x cols matrix of block type t
        return rows * hipmoe.row_bytes(t, cols)
    lt = types["layers"] if types else [(wt,) * 6] * Lh
    et, ot = (types["embd"], types["output"]) if types else (wt, wt)
    # a step reads the weights once for all sequences, and each sequence's
    # own KV rows and embedding row: per layer q, k, v (rows of E columns),
    # the output (E rows of EQ), the router, the unique experts' gate, up
    # and down, the KV rows attention reads
    bytes_per_step = tb(ot, V, E) + nseq * tb(et, 1, E)
    for t in lt:
        bytes_per_step += (tb(t[0], EQ, E) + tb(t[1], EKV, E) + tb(t[2], EKV, E) +
                           tb(t[3], E, EQ) + NE * E * 4 +
                           mean_uniq * (2 * tb(t[4], EI, E) + tb(t[5], E, EI)) +
                           nseq * 2 * kv_rows * EKV * 4)
    achieved_gbs = bytes_per_step / (ms_per_step / 1e3) / 1e9
    log(f"{steps} steps x {nseq} sequences in {ms:.2f} ms: {ms_per_step * 1e3:.1f} us/step, "
        f"{tokens_per_s:.1f} tokens/s, {achieved_gbs:.1f} GB/s algorithmic "
        f"({bytes_per_step / 1e9:.3f} GB/step)")
    M.free()
    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s, own process)")
        # the reference decodes one sequence at a time: sixteen sequences
        # are sixteen sequential runs at the single-sequence rate
        cpu = cpu_baseline({k: v for k, v in w.items() if k != "nseq"}, args.cpu_seconds)
        if cpu:
            log(f"cpu baseline: {cpu['value']:.2f} tokens/s on {cpu['cores']} threads")
    line = {
        "metric": MODEL_METRIC, "value": round(tokens_per_s, 2), "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "layers": Lh, "d_model": E, "heads": H,
                   "kv_heads": KH, "vocab": V, "experts": NE, "topk": K, "d_ff": EI,
                   "context": Cx,
                   "weights": "Q4_K_M" if types else {
                       hipmoe.Q8_0: "Q8_0", hipmoe.Q4_0: "Q4_0", hipmoe.Q4_K: "Q4_K",
                       hipmoe.Q6_K: "Q6_K"}[wt],
                   "prompt_tokens": w["prompt"], "sequences": nseq, "graphs": not args.eager,
                   "mean_unique_experts": round(mean_uniq, 3),
                   "algorithmic_bytes_per_step": int(bytes_per_step)},
        "roofline": {"bound": "hbm", "kernel": "decode_step", "achieved": round(achieved_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes("decode_step", args.workload)},
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
    ap.add_argument("--prompt", type=int, default=0,
                    help="model workloads: prompt length in place of the workload's (for "
                         "profiling runs, whose tracers hold every dispatch)")
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
    if args.prompt > 0:
        if w.get("kind") != "model":
            sys.exit("--prompt applies to the model workloads")
        w = dict(w, prompt=args.prompt)
    H = hipmoe.hip()
    if H.device_count() < 1:
        sys.exit("no HIP device")
    if w.get("kind") == "qmat":
        return bench_qmat(args, w, H)
    if w.get("kind") == "model":
        return bench_model(args, w, H)
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

    # the path the library takes for this T: one launch of k_moe_decode (K-quant
    # experts: routing + gate/up, then down + combine), or router, top-k, sort
    # and the grouped GEMMs, or router, top-k, GEMVs
    path = layers[0].path_for(T)
    kq = hipmoe.wtypes(w["wtype"])[0] in (hipmoe.Q4_K, hipmoe.Q6_K)
    # (layer_*: the whole call, whose kernels the counter summaries add up)
    kernel = {hipmoe.PATH_DECODE: "layer_decode" if kq else "k_moe_decode",
              hipmoe.PATH_GROUPED: "layer_grouped",
              hipmoe.PATH_GEMV: "layer_gemv"}[path]

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s, own process)")
        cpu = cpu_baseline(w, args.cpu_seconds)
        if cpu:
            log(f"cpu baseline: {cpu['value']:.2f} tokens/s on {cpu['cores']} threads")

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
            "weights": type_name(w["wtype"]),
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
