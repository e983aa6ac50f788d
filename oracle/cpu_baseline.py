#!/usr/bin/env python3
"""CPU baseline for bench.py, run as a process of its own.

TEST INFRASTRUCTURE: times the oracle (oracle/moe_oracle.c, lm_oracle.c: a
C restatement of the reference's AVX2 CPU path, bit-identical to it) on this
host with the reference's threading (thread_pool.c): a pool of one thread per
physical core the process may use, each operation on one thread below
16 Mi flops and on the whole pool above (thread_pool.c:25,69-109,178-185).
It never touches the GPU.  Prints one JSON line:

  value, unit          tokens/s over a bounded sample of the workload
  cores                threads of the pool
  kind                 "port" (the oracle, not the reference's own build)
  sample               what was timed
  cpu_model, physical_cores, usable_cores, isa, threads_per_op

Usage: cpu_baseline.py --spec JSON --seconds S
  spec kind "moe"   : {wtype, E, EI, NE, K, renorm, T, bias_std}
       kind "qmat"  : {wtype, N, Kc, T}
       kind "model" : {layers, E, H, V, NE, K, EI, C, wtype, prompt, gen[, q4km]}
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path[:0] = [HERE, os.path.join(REPO, "llm.c_amd")]

import ctypes as C  # noqa: E402

import numpy as np  # noqa: E402

SEED = 1337
MIN_FLOPS_THREADED = 16 * 1024 * 1024


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def isa_flags():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                fl = set(line.split(":", 1)[1].split())
                return [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vnni")
                        if f in fl]
    except OSError:
        pass
    return []


def physical_cores(cpus):
    """Distinct (package, core) pairs among `cpus` (detect_cores,
    thread_pool.c:69-109)."""
    seen = set()
    for c in cpus:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            core = int(open(base + "core_id").read())
            try:
                pkg = int(open(base + "physical_package_id").read())
            except OSError:
                pkg = 0
            seen.add((pkg, core))
        except OSError:
            return len(cpus)
    return len(seen)


def cgroup_cpus():
    """CPUs the cgroup quota allows (cpu.max), or None."""
    try:
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            return max(1, int(int(q) // int(p)))
    except (OSError, ValueError):
        pass
    return None


def pool_size():
    allowed = sorted(os.sched_getaffinity(0))
    machine = physical_cores(range(os.cpu_count() or 1))
    usable = physical_cores(allowed)
    n = usable
    quota = cgroup_cpus()
    if quota:
        n = min(n, quota)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n), machine, usable, quota


def nthreads_for(flops, pool):
    return 1 if flops < MIN_FLOPS_THREADED else pool


def bench_moe(spec, seconds, pool):
    import hipmoe
    import oracle
    wt, E, EI, NE, K, T = spec["wtype"], spec["E"], spec["EI"], spec["NE"], spec["K"], spec["T"]
    lw = hipmoe.synth_layer(SEED, 0, wt, E, EI, NE, 0.02, spec.get("bias_std"))
    sample_T = min(T, 64)
    xs = [hipmoe.synth_input(SEED, 1000 + i, sample_T, E) for i in range(8)]
    done, i, t0 = 0, 0, time.perf_counter()
    while True:
        oracle.moe_ffn(xs[i % len(xs)], lw, K, bool(spec["renorm"]), lw["bias"], nthreads=1)
        done += sample_T
        i += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    ops = {"router": nthreads_for(2 * sample_T * E * NE, pool),
           "expert_ffn": nthreads_for(2 * E * EI, pool)}
    return done / el, f"{done} tokens in {i} layer calls of {sample_T} token(s), {el:.1f} s", ops


def bench_qmat(spec, seconds, pool):
    import hipmoe
    import oracle
    wt, N, Kc, T = spec["wtype"], spec["N"], spec["Kc"], spec["T"]
    q = hipmoe.synth_quant_matrix(SEED, 0x7700 + wt, 0.02, wt, N, Kc)
    xs = [hipmoe.synth_input(SEED, 2000 + i, T, Kc) for i in range(8)]
    done, i, t0 = 0, 0, time.perf_counter()
    while True:
        oracle.qmat_mul(xs[i % len(xs)], q, wt, N, Kc)
        done += T
        i += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return done / el, f"{done} tokens in {i} calls, {el:.1f} s", \
        {"product": nthreads_for(2 * T * Kc * N, pool)}


def bench_model(spec, seconds, pool):
    import hiplm
    import oracle
    if spec.get("arch", "olmoe") == "olmoe":
        # q4km: the tensors' types mixed as a Q4_K_M file mixes them
        types = hiplm.q4_k_m_types(spec["layers"]) if spec.get("q4km") else None
        md = hiplm.synth_olmoe(SEED, spec["layers"], spec["E"], spec["H"], spec["V"],
                               spec["NE"], spec["K"], spec["EI"], spec["wtype"], types=types)
        tab = hiplm.ptr_table(md)
    else:
        md = hiplm.synth_mixtral(SEED, spec["layers"], spec["E"], spec["H"], spec["KH"],
                                 spec["V"], spec["NE"], spec["K"], spec["EI"], spec["wtype"],
                                 theta=spec["theta"], window=spec["window"], share_layers=True)
        tab = hiplm.ptr_table_llama(md)
    # a bounded sample: at most 16 prompt steps (untimed) before the timed ones
    spec = dict(spec, prompt=min(spec["prompt"], 16))
    prompt = hiplm.synth_prompt(SEED, spec["prompt"], spec["V"])
    m = oracle.OlmoeModel(md, spec["C"], tab)
    tok = 0
    for t in prompt:  # the prompt, untimed
        tok, _ = m.decode(int(t))
    done, t0 = 0, time.perf_counter()
    while done < spec["gen"]:
        tok, _ = m.decode(tok)
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    m.free()
    E, V = spec["E"], spec["V"]
    ops = {"attn_products": nthreads_for(2 * E * spec["H"] * 128, pool),
           "expert_ffn": nthreads_for(2 * E * spec["EI"], pool),
           "lm_head": nthreads_for(2 * E * V, pool), "attention": 1}
    return done / el, (f"{done} greedy decode steps after a {spec['prompt']}-token prompt, "
                       f"{el:.1f} s"), ops


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--spec", required=True)
    ap.add_argument("--seconds", type=float, default=10.0)
    args = ap.parse_args()
    spec = json.loads(args.spec)
    import oracle
    pool, machine, usable, quota = pool_size()
    L = oracle.lib()
    L.orc_set_pool.argtypes = [C.c_int]
    L.orc_set_pool.restype = C.c_int
    if pool > 1 and L.orc_set_pool(pool) != pool:
        sys.exit("cpu_baseline: could not start the thread pool")
    kind = spec.get("kind", "moe")
    fn = {"moe": bench_moe, "qmat": bench_qmat, "model": bench_model}[kind]
    value, sample, ops = fn(spec, args.seconds, pool)
    L.orc_set_pool(0)
    print(json.dumps({
        "value": value, "unit": "tokens/s", "cores": pool, "kind": "port",
        "sample": sample + f"; oracle (C restatement of the reference's AVX2 path, "
                           f"-O3 -mavx2 -mfma), reference threading: pool of {pool}",
        "cpu_model": cpu_model(), "physical_cores": machine, "usable_cores": usable,
        "cgroup_cpus": quota, "isa": isa_flags(), "threads_per_op": ops,
    }), flush=True)


if __name__ == "__main__":
    main()
