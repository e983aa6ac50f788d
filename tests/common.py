"""Shared helpers for the tests: configurations, golden fixtures, metrics."""
from __future__ import annotations

import ctypes as C
import functools
import hashlib
import os

import numpy as np

import hipmoe

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
REPO = os.path.abspath(os.path.join(HERE, ".."))
SEED = 1337

# name: (wtype, E, EI, NE, topk, renorm, bias_std)
CONFIGS = {
    "olmoe_q8": (hipmoe.Q8_0, 2048, 1024, 64, 8, 0, None),
    "olmoe_q4_skew": (hipmoe.Q4_0, 2048, 1024, 64, 8, 0, 1.0),
    "mixtral_q4": (hipmoe.Q4_0, 4096, 14336, 8, 2, 1, None),
}

# Output tolerance of the layer (relative L2 against the reference CPU path).
REL_L2_TOL = 1e-3


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@functools.lru_cache(maxsize=2)
def layer(cfg: str, layer_index: int = 0) -> dict:
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    return hipmoe.synth_layer(SEED, layer_index, wt, E, EI, NE, 0.02, bias_std)


def router_inputs(cfg: str, T: int, call: int):
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    L = hipmoe.lib()
    wr = hipmoe.synth_normal(SEED, L.moe_stream_router(0), NE * E, 0.0, 0.02).reshape(NE, E)
    bias = None
    if bias_std is not None:
        bias = hipmoe.synth_normal(SEED, L.moe_stream_bias(0), NE, 0.0, bias_std)
    x = hipmoe.synth_normal(SEED, L.moe_stream_input(call), T * E).reshape(T, E)
    return wr, bias, x


_host_expf = None


def host_expf_lib():
    global _host_expf
    if _host_expf is None:
        path = os.path.join(HERE, "native", "libhost_expf.so")
        L = C.CDLL(path)
        L.host_expf_mismatches.restype = C.c_uint64
        L.host_expf_mismatches.argtypes = [C.c_uint32, C.c_uint64, C.c_uint64, C.c_int,
                                           C.POINTER(C.c_uint32)]
        L.host_moe_expf.restype = None
        L.host_moe_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        _host_expf = L
    return _host_expf


def top_k_closed_form(p: np.ndarray, k: int):
    """The closed form the device evaluates for top_k (nn.c:276-308):
    rank_i = #{j: p_j > p_i or (p_j == p_i and j < i)}, r0 = rank_0; i != 0
    goes to slot k-1-rank_i iff rank_i < min(r0, k); slots 0..k-1-r0 hold
    element 0 when r0 < k."""
    n = p.size
    idx = np.arange(n)
    gt = (p[None, :] > p[:, None]) | ((p[None, :] == p[:, None]) & (idx[None, :] < idx[:, None]))
    rank = gt.sum(axis=1)
    r0 = int(rank[0])
    ids = np.zeros(k, np.uint32)
    w = np.full(k, p[0], np.float32)
    lim = min(r0, k)
    for i in range(1, n):
        if rank[i] < lim:
            ids[k - 1 - rank[i]] = i
            w[k - 1 - rank[i]] = p[i]
    return ids, w


def qmat_cases():
    """The dense quantized-product cases of tests/golden/make_golden.py and
    their seeded input generator (the fixture stores the inputs' digests)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden",
                                                  os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    return mg.QMAT_CASES, mg.qmat_inputs


def qmat_case(i: int, name: str):
    """(wtype, T, N, K, q, x, add, expected out) of fixture case `name`,
    after checking the regenerated inputs are the fixture's bytes."""
    cases, gen = qmat_cases()
    wt, T, N, K, add = cases[name]
    assert list(cases).index(name) == i
    q, x, a = gen(i, wt, T, N, K, add)
    g = golden("qmat.npz")
    assert sha(q) == str(g[f"{name}_sha_w"]) and sha(x) == str(g[f"{name}_sha_x"])
    assert (sha(a) if a is not None else "") == str(g[f"{name}_sha_add"])
    return wt, T, N, K, q, x, a, g[f"{name}_out"]


def kq_case(name: str):
    """(wtype, T, N, K, q, x, add, expected out) of K-quant product case
    `name` (tests/golden/kquant.npz), after checking the regenerated inputs
    are the fixture's bytes."""
    mg = _make_golden_module()
    wt, T, N, K, add = mg.KQ_CASES[name]
    q, x, a = mg.kq_inputs(list(mg.KQ_CASES).index(name), wt, T, N, K, add)
    g = golden("kquant.npz")
    assert sha(q) == str(g[f"{name}_sha_w"]) and sha(x) == str(g[f"{name}_sha_x"])
    assert (sha(a) if a is not None else "") == str(g[f"{name}_sha_add"])
    return wt, T, N, K, q, x, a, g[f"{name}_out"]


def _make_golden_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden",
                                                  os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    return mg


@functools.lru_cache(maxsize=1)
def batch_case(name: str):
    """(model dict, prompts [nseq][n_prompt], batch case, fixture) of the
    lockstep-batch fixture batch_<name>.npz; bc["case"] is the model case
    tuple."""
    mg = _make_golden_module()
    md, _, case = mg.model_case(name)
    g = golden(f"batch_{name}.npz")
    assert mg.model_digest(md) == str(g["sha_model"]), "regenerated model differs from fixture"
    bc = dict(mg.BATCH_CASES[name])
    bc["case"] = case
    return md, mg.batch_prompts(name, case[3]), bc, g


def model_case(name: str):
    """(model dict, prompt, case tuple, fixture) of model fixture `name`,
    after checking the regenerated weights are the fixture's bytes."""
    mg = _make_golden_module()
    md, prompt, case = mg.model_case(name)
    g = golden(f"model_{name}.npz")
    assert np.array_equal(prompt, g["prompt"])
    assert mg.model_digest(md) == str(g["sha_model"]), "regenerated model differs from fixture"
    return md, prompt, case, g


# --------------------------------------------------------------------------
# routing near-ties and generate's picks
# --------------------------------------------------------------------------

# a routing probability moves by ~3e-4 (relative) downstream of a layer on
# the grouped path (f16 operands); gaps under ~7 times that are near-ties
ROUTE_GAP = 2e-3


def routing_margins(md, Cx, seq, n_prompt):
    """The model oracle's (bit for bit the reference's) decode of one
    sequence: for every step from the prompt's last id on, the smallest
    relative gap over the layers between the last selected and the first
    unselected routing probability, (p_K - p_K+1) / p_K."""
    import hiplm
    import oracle
    L, K = md["layers"], md["K"]
    tab = hiplm.ptr_table(md) if md["arch"] == "olmoe" else hiplm.ptr_table_llama(md)
    om = oracle.OlmoeModel(md, Cx, tab)
    gaps = []
    try:
        for i, tok in enumerate(seq):
            _, _, (mi, _, _) = om.decode(int(tok), trace=True)
            if i < n_prompt - 1:
                continue
            gap = 1.0
            for l in range(L):
                b = md["blk"][l]
                lay = dict(router=b["router"], gate=b["gate"], up=b["up"], down=b["down"],
                           wtype=md["wtype"], E=md["E"], EI=md["EI"], NE=md["NE"])
                pr = np.sort(oracle.moe_ffn(mi[l:l + 1], lay, K, md["arch"] != "olmoe",
                                            None)[4][0])[::-1]
                gap = min(gap, float((pr[K - 1] - pr[K]) / pr[K - 1]))
            gaps.append(gap)
    finally:
        om.free()
    return np.asarray(gaps)


def prefill_moe_fp32(md, rows):
    """A prefill launch of `rows` rows keeps its MoE layers in fp32: the
    decode kernel takes them (4 * rows * K <= 3 * NE); past that the grouped
    path's f16 operands move each layer's output by ~5e-4."""
    return 4 * rows * md["K"] <= 3 * md["NE"]


def generate_upto(md, Cx, prompt, ref_tokens, top_logits, rows):
    """How many of generate's picks (one prefill of the prompt, `rows` rows
    per launch, then decode steps) must equal the reference's ref_tokens
    [n_gen + 1]: those before the first whose reference top-two logits are
    within 1e-4 relative (an fp32 prefill) or 2e-3 (a prefill on the grouped
    path).  After a grouped-path prefill, whose f16 layers move the prompt's
    rows (and the cache rows later steps attend to) by ~5e-4, also none past
    a routing near-tie (ROUTE_GAP) of a prompt row, or of the step that makes
    the pick: there the other expert may be picked."""
    t = np.asarray(top_logits, np.float64)
    fp32 = prefill_moe_fp32(md, rows)
    gap = np.abs(t[:, 0] - t[:, 1]) / np.abs(t[:, 0])
    bad = list(np.nonzero(gap <= (1e-4 if fp32 else 2e-3))[0])
    if not fp32:
        n = len(prompt)
        seq = np.concatenate([np.asarray(prompt), np.asarray(ref_tokens)[:-1]])
        rg = routing_margins(md, Cx, seq, 1)
        if n > 1 and rg[:n - 1].min() <= ROUTE_GAP:
            return 0
        bad += list(np.nonzero(rg[n - 1:] <= ROUTE_GAP)[0])
    return int(min(bad)) if bad else t.shape[0]
