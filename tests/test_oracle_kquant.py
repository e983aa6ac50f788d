"""The oracle's K-quant path (Q4_K / Q6_K weights, Q8_K activations: the
reference's default -DQ8_DOT build) pinned against the compiled reference's
own outputs (tests/golden/kquant.npz) and against what the formats fix:

  * quantize_row_q8 (quant.c:627-654) bit for bit on seeded and edge blocks
    (zero block, ties of magnitude, x.5 products); the reference test's
    round trip (test/quant_dot.c:37-60: |x - d q| < 0.01, bsums the sums of
    16) and d q reproducing the largest magnitude exactly in sign;
  * dot_q8_quant, dot_f32_quant and dequant_row on the reference test's
    fill patterns (test/quant_dot.c:12-34) and seeded rows bit for bit, with
    the test's own bar between the integer and the fp32 dot (relative
    difference < 0.02, test/quant_dot.c:62-104);
  * the integer dot equal (to fp32 rounding of the per-block steps) to the
    exact float64 sum over the formats' fields d*sc*q - dmin*m times yd*q8,
    written from the block layouts (quant.h:30-57), and the fp32 dot to the
    float64 dot of the dequantized row: a dropped min, a swapped nibble or
    scale index fails these;
  * tensor_mma_transposed_2x2 with Q4_K/Q6_K right operands (T = 1..9, add
    NULL / [N] / [T][N], K = 256 .. 14336) bit for bit;
  * this package's synthetic K-quantizers: dequant(quantize(x)) within the
    formats' step of x (the packing they write is the one the reference's
    get_scale_min_k4 and Q6_K loops read).
"""
import numpy as np
import pytest

import hipmoe
import oracle
from common import bits, golden, kq_case, rel_l2, sha

SEED = 1337


@pytest.fixture(scope="module")
def g():
    return golden("kquant.npz")


def test_q8k_quantize_bitwise_and_roundtrip(g):
    x = g["q8k_x"]
    d, qs, bs = oracle.quantize_q8k(x.reshape(-1))
    assert np.array_equal(bits(d), bits(g["q8k_d"]))
    assert np.array_equal(qs, g["q8k_qs"]) and np.array_equal(bs, g["q8k_bsums"])
    q = qs.reshape(-1, 256).astype(np.int64)
    assert np.array_equal(bs, q.reshape(-1, 16, 16).sum(-1))
    for b in range(x.shape[0]):
        xb = x[b]
        if not np.any(xb):
            assert d[b] == 0 and not np.any(q[b])
            continue
        i = int(np.argmax(np.abs(xb)))            # first index of the largest magnitude
        assert q[b, i] == -127                    # iscale = -127 / x[i]
        assert np.all(np.abs(q[b]) <= 127)
        err = np.max(np.abs(xb.astype(np.float64) - np.float64(d[b]) * q[b]))
        assert err <= 0.5 * abs(float(d[b])) * (1 + 1e-5) + 1e-30, (b, err)
    # test/quant_dot.c:37-60 (its block is the sin ramp, index 16 of the set)
    sinb = x[16]
    assert np.array_equal(sinb, np.sin(np.arange(256, dtype=np.float32) * np.float32(0.1))
                          .astype(np.float32) * np.float32(0.5))
    assert np.max(np.abs(sinb - d[16] * q[16])) < 0.01


def test_q8k_ties_take_the_first(g):
    x = g["q8k_x"]
    d, qs, _ = oracle.quantize_q8k(x.reshape(-1))
    q = qs.reshape(-1, 256)
    # blocks 19/20: +3 at 10 and -3 at 200 (and the reverse): the first sets the sign
    assert q[19][10] == -127 and q[19][200] == 127 and d[19] < 0
    assert q[20][10] == -127 and q[20][200] == 127 and d[20] > 0


def _fields_q4k(blk):
    """(d, dmin, sc[8], m[8], q[256]) of a Q4_K block from its byte layout."""
    d = float(blk[0:2].view(np.float16)[0])
    dmin = float(blk[2:4].view(np.float16)[0])
    s = blk[4:16].astype(np.int64)
    sc = np.zeros(8, np.int64)
    m = np.zeros(8, np.int64)
    for j in range(8):
        if j < 4:
            sc[j], m[j] = s[j] & 63, s[j + 4] & 63
        else:
            sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
            m[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    qs = blk[16:144].astype(np.int64).reshape(4, 32)
    q = np.concatenate([np.concatenate([qs[j] & 15, qs[j] >> 4]) for j in range(4)])
    return d, dmin, sc, m, q


def _fields_q6k(blk):
    """(d, sc[16], q[256] in -32..31) of a Q6_K block from its byte layout."""
    ql = blk[0:128].astype(np.int64)
    qh = blk[128:192].astype(np.int64)
    sc = blk[192:208].view(np.int8).astype(np.int64)
    d = float(blk[208:210].view(np.float16)[0])
    q = np.zeros(256, np.int64)
    for e in range(256):
        c, r = divmod(e, 128)
        gq, l = divmod(r, 32)
        lo = ql[c * 64 + (gq & 1) * 32 + l]
        lo = lo & 15 if gq < 2 else lo >> 4
        q[e] = (lo | (((qh[c * 32 + l] >> (2 * gq)) & 3) << 4)) - 32
    return d, sc, q


def exact_weights(row, wt, n):
    """float64 values of a K-quant row: d*sc*q - dmin*m / d*sc*q, exactly."""
    out = []
    if wt == hipmoe.Q4_K:
        for b in range(n // 256):
            d, dmin, sc, m, q = _fields_q4k(row[b * 144:(b + 1) * 144])
            out.append(d * np.repeat(sc, 32) * q - dmin * np.repeat(m, 32))
    else:
        for b in range(n // 256):
            d, sc, q = _fields_q6k(row[b * 210:(b + 1) * 210])
            out.append(d * np.repeat(sc, 16) * q)
    return np.concatenate(out).astype(np.float64)


def check_row(x, row, wt, n, want_q8=None, want_f32=None, want_deq=None):
    got_q8 = oracle.dot_q8k(x, row, wt)
    got_f32 = oracle.dot(x, row, wt)
    deq = oracle.dequant(row, wt, n)
    if want_q8 is not None:
        assert bits(got_q8) == bits(np.float32(want_q8))
        assert bits(got_f32) == bits(np.float32(want_f32))
    if want_deq is not None:
        assert np.array_equal(bits(deq), bits(want_deq))
    # the formats' own values, in float64
    w = exact_weights(row, wt, n)
    assert np.max(np.abs(deq - w)) <= 4 * 2.0 ** -24 * np.max(np.abs(w)) + 1e-30
    d, qs, _ = oracle.quantize_q8k(x)
    xq = np.repeat(d.astype(np.float64), 256) * qs
    exact = float(np.dot(w, xq))
    scale = float(np.dot(np.abs(w), np.abs(xq)))
    assert abs(float(got_q8) - exact) <= 2.0 ** -20 * scale * (n // 256 + 2), (got_q8, exact)
    exact_f = float(np.dot(deq.astype(np.float64), x.astype(np.float64)))
    scale_f = float(np.dot(np.abs(deq), np.abs(x)))
    assert abs(float(got_f32) - exact_f) <= 2.0 ** -22 * scale_f * 8, (got_f32, exact_f)
    return got_q8, got_f32


@pytest.mark.parametrize("name,wt", [("q4k", hipmoe.Q4_K), ("q6k", hipmoe.Q6_K)])
@pytest.mark.parametrize("nb", [1, 16])
def test_reference_fill_patterns(g, name, wt, nb):
    k = f"fill_{name}_{nb}"
    x, row = g[f"{k}_x"], g[f"{k}_w"]
    q8, f32 = check_row(x, row, wt, 256 * nb, g[f"{k}_dot_q8"], g[f"{k}_dot_f32"],
                        g[f"{k}_deq"])
    # test/quant_dot.c:62-104: the integer dot within 2% of the fp32 one
    assert abs(float(q8) - float(f32)) / (abs(float(f32)) + 1e-9) < 0.02


@pytest.mark.parametrize("name,wt", [("q4k", hipmoe.Q4_K), ("q6k", hipmoe.Q6_K)])
@pytest.mark.parametrize("n", [256, 768, 2048, 4096, 14336])
def test_seeded_rows(g, name, wt, n):
    k = f"rows_{name}_{n}"
    qm = hipmoe.synth_quant_matrix(SEED, 0x7f00 + n + wt, 0.02, wt, 3, n)
    x = hipmoe.synth_normal(SEED, 0x7f80 + n + wt, 3 * n).reshape(3, n)
    assert sha(qm) == str(g[f"{k}_sha_w"]) and sha(x) == str(g[f"{k}_sha_x"])
    rb = hipmoe.row_bytes(wt, n)
    for r in range(3):
        check_row(np.ascontiguousarray(x[r]), qm[r * rb:(r + 1) * rb], wt, n,
                  g[f"{k}_dot_q8"][r], g[f"{k}_dot_f32"][r],
                  g[f"{k}_deq0"] if r == 0 else None)


KQ_NAMES = ["q4k_t1", "q4k_t5_rows", "q4k_t2_bcast_14336", "q4k_t1_256", "q6k_t1",
            "q6k_t3_bcast", "q6k_t9_rows_768", "q6k_t1_14336"]


@pytest.mark.parametrize("name", KQ_NAMES)
def test_qmat_kquant_bitwise(name):
    wt, T, N, K, q, x, a, want = kq_case(name)
    got = oracle.qmat_mul(x, q, wt, N, K, a)
    assert np.array_equal(bits(got), bits(want)), rel_l2(got, want)


@pytest.mark.parametrize("wt", [hipmoe.Q4_K, hipmoe.Q6_K])
def test_synth_kquantizer_roundtrip(wt):
    n = 4096
    x = hipmoe.synth_normal(SEED, 0x7e10 + wt, 4 * n, 0.0, 0.02).reshape(4, n)
    q = hipmoe.synth_quant_matrix(SEED, 0x7e10 + wt, 0.02, wt, 4, n)
    rb = hipmoe.row_bytes(wt, n)
    for r in range(4):
        deq = oracle.dequant(q[r * rb:(r + 1) * rb], wt, n)
        # Q4_K: 15 steps over each 32-value range (6-bit scale and min on
        # top); Q6_K: steps of |v|/32 for the sub-block's largest |v|, whose
        # opposite-signed values clamp at +31 (up to one step off)
        amax = np.max(np.abs(x[r]))
        tol = 0.6 * amax / 7.0 if wt == hipmoe.Q4_K else 1.1 * amax / 32.0
        assert np.max(np.abs(deq - x[r])) <= tol
        assert rel_l2(deq, x[r]) < (0.1 if wt == hipmoe.Q4_K else 0.03)


# ---- MoE layers on K-quant experts (tests/golden/kquant_moe.npz) -----------

def kq_layer(name):
    """(wtype, E, EI, NE, K, renorm, T), the layer and the tokens of K-quant
    layer case `name`, after checking they are the fixture's bytes."""
    import importlib.util
    import os
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                    "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    wt, E, EI, NE, K, renorm, T = mg.KQ_LAYERS[name]
    lw = hipmoe.synth_layer(SEED, 0, wt, E, EI, NE, 0.02, None)
    x = hipmoe.synth_input(SEED, 0, T, E)
    g = golden("kquant_moe.npz")
    assert sha(lw["gate"]) == str(g[f"{name}_sha_gate"])
    assert sha(lw["down"]) == str(g[f"{name}_sha_down"]) and sha(x) == str(g[f"{name}_sha_x"])
    return (wt, E, EI, NE, K, renorm, T), lw, x, g[f"{name}_out"]


@pytest.mark.parametrize("name", ["olmoe_q4k_q6k", "olmoe_q6k", "ragged_q4k_q6k",
                                  "ragged_q6k_q4k",
                                  pytest.param("mixtral_q4k_q6k", marks=pytest.mark.slow)])
def test_oracle_kq_layer_vs_reference(name):
    """The oracle's moe_ffn on K-quant experts (the Q8_K gate/up dots, the
    fp32 down dot) equals the reference's own moe_ffn bit for bit."""
    (wt, E, EI, NE, K, renorm, T), lw, x, want = kq_layer(name)
    got = oracle.moe_ffn(x, lw, K, bool(renorm), None)[0]
    assert np.array_equal(bits(got), bits(want)), rel_l2(got, want)


@pytest.mark.parametrize("name,wt", [("q4k_q6k", hipmoe.Q4_K | hipmoe.Q6_K << 8),
                                     ("q6k_q4k", hipmoe.Q6_K | hipmoe.Q4_K << 8)])
def test_oracle_kq_fused_ffn_vs_reference(name, wt):
    E, EI = 2048, 1024
    gt, dt = hipmoe.wtypes(wt)
    gq = hipmoe.synth_quant_matrix(SEED, 0x9011, 0.02, gt, EI, E)
    uq = hipmoe.synth_quant_matrix(SEED, 0x9012, 0.02, gt, EI, E)
    dq = hipmoe.synth_quant_matrix(SEED, 0x9013, 0.02, dt, E, EI)
    x = hipmoe.synth_normal(SEED, 0x9014, E)
    g = golden("kquant_moe.npz")
    assert sha(np.concatenate([gq, uq, dq, x.view(np.uint8)])) == str(g[f"ffn_{name}_sha"])
    got = oracle.fused_ffn(x, gq, uq, dq, wt, E, EI)
    assert np.array_equal(bits(got), bits(g[f"ffn_{name}_out"]))
    # and against the formats' own values in float64 (a dropped min or a
    # swapped scale moves it far more than the rounding bound)
    d8, q8, _ = oracle.quantize_q8k(x)
    xq = np.repeat(d8.astype(np.float64), 256) * q8
    rb_in, rb_mid = hipmoe.row_bytes(gt, E), hipmoe.row_bytes(dt, EI)
    gv = np.array([exact_weights(gq[j * rb_in:(j + 1) * rb_in], gt, E) @ xq for j in range(EI)])
    uv = np.array([exact_weights(uq[j * rb_in:(j + 1) * rb_in], gt, E) @ xq for j in range(EI)])
    hv = gv / (1 + np.exp(-gv)) * uv
    yv = np.array([exact_weights(dq[i * rb_mid:(i + 1) * rb_mid], dt, EI) @ hv for i in range(E)])
    assert rel_l2(got, yv) < 1e-5
