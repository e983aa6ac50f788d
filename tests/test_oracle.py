"""Pins the CPU oracle (oracle/moe_oracle.c) and the synthetic-input
quantizers before either is trusted as a checker.

Each function is checked against what fixes it independently:
  * golden vectors from the compiled reference (tests/golden/, written by
    make_golden.py from the reference's own C sources, AVX2 build);
  * the reference's own known-answer test for top_k (test/nn.c:5-33);
  * closed forms: fp16 conversion vs numpy, block dequantization from the
    layout of quant.h:14-26, dots vs float64 sums, brute force on tiny inputs;
  * the exhaustive glibc expf comparison of the device expf algorithm.
"""
import numpy as np
import pytest

import hipmoe
import oracle
from common import (CONFIGS, SEED, bits, golden, host_expf_lib, layer, qmat_case,
                    qmat_cases, rel_l2, router_inputs, sha, top_k_closed_form)
import ctypes as C


# --------------------------------------------------------------------------
# quantizers (input generation) and block layout
# --------------------------------------------------------------------------

def test_quantizers_match_reference_goldens():
    g = golden("quant.npz")
    x = g["x"]
    assert np.array_equal(hipmoe.quantize(x.reshape(-1), hipmoe.Q8_0), g["q8_0"])
    assert np.array_equal(hipmoe.quantize(x.reshape(-1), hipmoe.Q4_0), g["q4_0"])


def test_f16_rne_matches_numpy():
    L = hipmoe.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  1e-10, -3e-8, 0.5, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32)])
    got = np.array([L.moe_f32_to_f16_rne(float(v)) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # f16 -> f32 is exact: all 65536 patterns round trip through numpy
    allh = np.arange(65536, dtype=np.uint16)
    f = np.array([L.moe_f16_to_f32(int(h)) for h in allh[::7]], np.float32)
    ref = allh[::7].view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()


def _decode_blocks(q: np.ndarray, wtype: int, n: int) -> np.ndarray:
    """Closed form of the block layouts (quant.h:14-26): value = d * q with
    Q8_0 q = int8 qs[j]; Q4_0 element j<16 = (qs[j] & 15) - 8 and element
    j>=16 = (qs[j-16] >> 4) - 8."""
    if wtype == hipmoe.Q8_0:
        b = q.reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float64)
        v = b[:, 2:].view(np.int8).astype(np.float64)
    else:
        b = q.reshape(-1, 18)
        d = b[:, :2].copy().view(np.float16).astype(np.float64)
        qs = b[:, 2:].astype(np.int64)
        v = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float64)
    return (d * v).reshape(-1)[:n]


@pytest.mark.parametrize("wtype", [hipmoe.Q8_0, hipmoe.Q4_0])
def test_dequant_closed_form(wtype):
    n = 4096
    q = hipmoe.synth_quant_matrix(SEED, 11, 0.02, wtype, 1, n)
    got = oracle.dequant(q, wtype, n)
    assert np.array_equal(got.astype(np.float64), _decode_blocks(q, wtype, n))


@pytest.mark.parametrize("wtype", [hipmoe.Q8_0, hipmoe.Q4_0])
def test_quantize_roundtrip_error_bound(wtype):
    """|x - dequant(quant(x))| <= scale/2 per element (+ fp16 scale rounding)."""
    x = hipmoe.synth_normal(SEED, 12, 32 * 256, 0.0, 0.02)
    q = hipmoe.quantize(x, wtype)
    y = _decode_blocks(q, wtype, x.size)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    step = amax / (127.0 if wtype == hipmoe.Q8_0 else 7.0)
    err = np.abs(x.astype(np.float64) - y).reshape(-1, 32).max(axis=1)
    assert np.all(err <= step * 0.5 * 1.01 + amax * 2e-3)


# --------------------------------------------------------------------------
# dots
# --------------------------------------------------------------------------

@pytest.mark.parametrize("wtype,name", [(hipmoe.Q8_0, "q8_0"), (hipmoe.Q4_0, "q4_0")])
@pytest.mark.parametrize("n", [256, 1024, 2048, 4096, 14336])
def test_dot_matches_reference_bits(wtype, name, n):
    g = golden("dot.npz")
    rows = 4
    qm = hipmoe.synth_quant_matrix(SEED, 0x7000 + n + wtype, 0.02, wtype, rows, n)
    x = hipmoe.synth_normal(SEED, 0x7100 + n + wtype, rows * n).reshape(rows, n)
    assert sha(qm) == str(g[f"{name}_{n}_sha_w"]) and sha(x) == str(g[f"{name}_{n}_sha_x"])
    rb = hipmoe.row_bytes(wtype, n)
    got = np.array([oracle.dot(x[r], qm[r * rb:(r + 1) * rb], wtype) for r in range(rows)],
                   np.float32)
    assert np.array_equal(bits(got), bits(g[f"{name}_{n}_dot"]))
    # and against a float64 sum of the closed-form dequantization
    for r in range(rows):
        w64 = _decode_blocks(qm[r * rb:(r + 1) * rb], wtype, n)
        d64 = float(np.dot(w64, x[r].astype(np.float64)))
        scale = float(np.dot(np.abs(w64), np.abs(x[r].astype(np.float64))))
        assert abs(float(got[r]) - d64) <= 1e-6 * scale


# --------------------------------------------------------------------------
# dense quantized products (tensor_mma_transposed_2x2 on Q8_0/Q4_0)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("i,name", list(enumerate(qmat_cases()[0])))
def test_qmat_matches_reference_bits(i, name):
    """The oracle's product equals the compiled reference's
    tensor_mma_transposed_2x2 bit for bit (T = 1..9, add NULL / [N] /
    [T][N]), and a float64 product of the closed-form block decoding."""
    wt, T, N, K, q, x, a, want = qmat_case(i, name)
    got = oracle.qmat_mul(x, q, wt, N, K, a)
    assert np.array_equal(bits(got), bits(want))
    rb = hipmoe.row_bytes(wt, K)
    w64 = np.stack([_decode_blocks(q[j * rb:(j + 1) * rb], wt, K) for j in range(N)])
    x64 = x.astype(np.float64)
    ref64 = x64 @ w64.T
    scale = np.abs(x64) @ np.abs(w64).T
    if a is not None:
        a64 = a.astype(np.float64).reshape(-1, N)
        ref64 = ref64 + a64
        scale = scale + np.abs(a64)
    assert np.all(np.abs(got - ref64) <= 1e-6 * scale + 1e-30)


# --------------------------------------------------------------------------
# router / softmax / top-k
# --------------------------------------------------------------------------

@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_routing_matches_reference_bits(cfg):
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    g = golden(f"route_{cfg}.npz")
    T = int(g["T"])
    wr, bias, x = router_inputs(cfg, T, int(g["input_call"]))
    assert sha(wr) == str(g["sha_router"]) and sha(x) == str(g["sha_x"])
    if bias is not None:
        assert sha(bias) == str(g["sha_bias"])
    lg = oracle.router(x, wr, bias)
    keep = g["logits"].shape[0]
    assert np.array_equal(bits(lg[:keep]), bits(g["logits"]))
    ids = np.empty((T, K), np.uint32)
    w = np.empty((T, K), np.float32)
    for t in range(T):
        p = oracle.softmax(lg[t])
        if t < keep:
            assert np.array_equal(bits(p), bits(g["probs"][t])), t
        i, ww = oracle.top_k(p, K)
        if renorm:
            s = np.float32(0)
            for v in ww:
                s = np.float32(s + v)
            ww = (ww / s).astype(np.float32)
        ids[t], w[t] = i, ww
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(bits(w), bits(g["w"]))


def test_router_logits_float64_bound():
    wr, bias, x = router_inputs("olmoe_q4_skew", 64, 5)
    lg = oracle.router(x, wr, bias)
    ref = x.astype(np.float64) @ wr.astype(np.float64).T + bias.astype(np.float64)
    scale = np.abs(x).astype(np.float64) @ np.abs(wr).astype(np.float64).T + np.abs(bias)
    assert np.all(np.abs(lg - ref) <= 1e-6 * scale)


def test_softmax_properties():
    rng = np.random.default_rng(1)
    for n in (8, 64, 13, 1):
        v = rng.standard_normal(n).astype(np.float32) * 5
        p = oracle.softmax(v)
        ref = np.exp(v.astype(np.float64) - v.max())
        ref /= ref.sum()
        assert np.allclose(p, ref, rtol=1e-6, atol=1e-9)
        assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-6


def test_top_k_reference_known_answer():
    """test/nn.c:5-33"""
    x = np.array([0, 1, 7, 2, 9, 3, 6, 4, 5, 8], np.float32)
    ids, w = oracle.top_k(x, 5)
    assert list(ids) == [8, 6, 2, 9, 4]
    assert list(w) == [5.0, 6.0, 7.0, 8.0, 9.0]


def test_top_k_duplicates_element_zero():
    # only one value beats element 0: it takes slot k-1, element 0 fills the rest
    x = np.array([0.5, 0.1, 0.9, 0.2, 0.3], np.float32)
    ids, w = oracle.top_k(x, 3)
    assert list(ids) == [0, 0, 2] and list(w) == [0.5, 0.5, 0.9]
    # all equal: nothing is strictly greater than element 0
    ids, w = oracle.top_k(np.full(64, 1 / 64, np.float32), 8)
    assert list(ids) == [0] * 8


def test_top_k_closed_form_matches_sequential():
    """The device's rank formulation against the sequential insertion on
    inputs with many ties (small integer values)."""
    rng = np.random.default_rng(2)
    for trial in range(3000):
        n = int(rng.integers(1, 70))
        k = int(rng.integers(1, n + 1))
        p = rng.integers(0, 6, n).astype(np.float32)
        a = oracle.top_k(p, k)
        b = top_k_closed_form(p, k)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (p, k)


# --------------------------------------------------------------------------
# expert FFN and whole layers
# --------------------------------------------------------------------------

@pytest.mark.parametrize("wtype,name", [(hipmoe.Q8_0, "q8_0"), (hipmoe.Q4_0, "q4_0")])
def test_fused_ffn_matches_reference_bits(wtype, name):
    g = golden(f"ffn_{name}.npz")
    E, EI = 2048, 1024
    gm = hipmoe.synth_quant_matrix(SEED, 0x9001, 0.02, wtype, EI, E)
    um = hipmoe.synth_quant_matrix(SEED, 0x9002, 0.02, wtype, EI, E)
    dm = hipmoe.synth_quant_matrix(SEED, 0x9003, 0.02, wtype, E, EI)
    x = hipmoe.synth_normal(SEED, 0x9004, E)
    assert sha(gm) == str(g["sha_gate"]) and sha(dm) == str(g["sha_down"])
    out = oracle.fused_ffn(x, gm, um, dm, wtype, E, EI)
    assert np.array_equal(bits(out), bits(g["out"]))
    # float64 closed form: down . (silu(gate . x) * (up . x))
    Wg = _decode_blocks(gm, wtype, EI * E).reshape(EI, E)
    Wu = _decode_blocks(um, wtype, EI * E).reshape(EI, E)
    Wd = _decode_blocks(dm, wtype, E * EI).reshape(E, EI)
    gg, uu = Wg @ x.astype(np.float64), Wu @ x.astype(np.float64)
    ref = Wd @ (gg / (1 + np.exp(-gg)) * uu)
    assert rel_l2(out, ref) < 1e-5


@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_moe_layer_matches_reference_bits(cfg):
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    g = golden(f"moe_{cfg}.npz")
    T = int(g["T"])
    lay = layer(cfg)
    x = hipmoe.synth_input(SEED, 0, T, E)
    assert sha(lay["router"]) == str(g["sha_router"])
    assert sha(lay["gate"]) == str(g["sha_gate"]) and sha(lay["down"]) == str(g["sha_down"])
    assert sha(x) == str(g["sha_x"])
    out, ids, w, lg, pr = oracle.moe_ffn(x, lay, K, bool(renorm), lay["bias"])
    assert np.array_equal(bits(out), bits(g["out"]))


def test_moe_threads_do_not_change_bits():
    lay = layer("olmoe_q8")
    x = hipmoe.synth_input(SEED, 3, 6, 2048)
    a = oracle.moe_ffn(x, lay, 8, False, None, nthreads=1)[0]
    b = oracle.moe_ffn(x, lay, 8, False, None, nthreads=4)[0]
    assert np.array_equal(bits(a), bits(b))


# --------------------------------------------------------------------------
# expf: the device algorithm vs glibc, on the host
# --------------------------------------------------------------------------

def test_device_expf_algorithm_equals_glibc_softmax_range():
    """Every float in [-104, 0] (the softmax argument range, x - max <= 0)
    plus both zeros: the algorithm of moe_expf.h evaluated on the host gives
    glibc's bits."""
    L = host_expf_lib()
    first = C.c_uint32(0)
    neg0 = 0x80000000
    hi = int(np.array([-104.0], np.float32).view(np.uint32)[0])
    bad = L.host_expf_mismatches(neg0, hi - neg0 + 1, 1, oracle.threads(), C.byref(first))
    assert bad == 0, hex(first.value)
    bad = L.host_expf_mismatches(0, 1, 1, 1, C.byref(first))
    assert bad == 0


def test_device_expf_algorithm_equals_glibc_strided_all_floats():
    L = host_expf_lib()
    first = C.c_uint32(0)
    bad = L.host_expf_mismatches(0, 1 << 32, 97, oracle.threads(), C.byref(first))
    assert bad == 0, hex(first.value)
