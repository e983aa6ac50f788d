"""GPU parity of the K-quant dense product (Q4_K / Q6_K matrices through
Q8_K activations: hip_moe_qmat_* and hip_moe_quantize_q8k_dev, kquant.hip)
through the C ABI.  The bar is bit-exact everywhere: the per-super-block
sums are exact integers and the fp32 steps (scale products, the sequential
fma over super-blocks, the final add) are the reference's own.

  * quantize_row_q8 of the fixture's seeded and edge blocks equals the
    compiled reference's (tests/golden/kquant.npz) bit for bit, and the
    oracle's on a large seeded input (Mixtral's d_ff, 4 tokens);
  * the product equals the compiled reference's output on every fixture case
    (K = 256 .. 14336, T = 1..9, add NULL / [N] / [T][N], odd Q6_K blocks at
    2-byte offsets);
  * full sizes: the Mixtral lm_head as Q6_K (32000 x 4096) and a Q4_K
    attention projection (4096 x 4096), T = 1, against the oracle; T = 12 at
    K = 4096 (more tokens than one LDS pass holds: two passes);
  * a HIP graph of the product replays bit-identically.
"""
import sys

import numpy as np
import pytest

import hipmoe
import oracle
from common import bits, golden, kq_case, rel_l2

pytestmark = pytest.mark.gpu
SEED = 1337
KQ_NAMES = ["q4k_t1", "q4k_t5_rows", "q4k_t2_bcast_14336", "q4k_t1_256", "q6k_t1",
            "q6k_t3_bcast", "q6k_t9_rows_768", "q6k_t1_14336"]


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


def test_gpu_q8k_quantize_vs_reference():
    g = golden("kquant.npz")
    x = g["q8k_x"]
    say(f"quantize_q8k: {x.shape[0]} fixture blocks")
    d, qs, bs = hipmoe.quantize_q8k_dev(x.reshape(1, -1))
    assert np.array_equal(bits(d.ravel()), bits(g["q8k_d"]))
    assert np.array_equal(qs.ravel(), g["q8k_qs"])
    assert np.array_equal(bs.reshape(-1, 16), g["q8k_bsums"])
    x2 = hipmoe.synth_normal(SEED, 0x7e20, 4 * 14336, 0.0, 1.0).reshape(4, 14336)
    say("quantize_q8k: 4 x 14336 seeded")
    d, qs, bs = hipmoe.quantize_q8k_dev(x2)
    od, oq, ob = oracle.quantize_q8k(x2.ravel())
    assert np.array_equal(bits(d.ravel()), bits(od))
    assert np.array_equal(qs.ravel(), oq) and np.array_equal(bs.reshape(-1, 16), ob)


@pytest.mark.parametrize("name", KQ_NAMES)
def test_gpu_kquant_qmat_vs_reference_golden(name):
    wt, T, N, K, q, x, a, want = kq_case(name)
    say(f"kquant qmat {name}: wt={wt} T={T} N={N} K={K}")
    W = hipmoe.QMat(q, wt, N, K)
    try:
        got = W.mul(x, a)
    finally:
        W.free()
    same = np.array_equal(bits(got), bits(want))
    say(f"kquant qmat {name}: bitwise {same}, rel L2 {rel_l2(got, want):.3e}")
    assert same


@pytest.mark.parametrize("wt,N,K,T", [(hipmoe.Q6_K, 32000, 4096, 1),
                                      (hipmoe.Q4_K, 4096, 4096, 1),
                                      (hipmoe.Q4_K, 1000, 4096, 12),
                                      (hipmoe.Q6_K, 4096, 14336, 1)])
def test_gpu_kquant_qmat_full_size(wt, N, K, T):
    say(f"kquant qmat full size wt={wt} N={N} K={K} T={T}")
    q = hipmoe.synth_quant_matrix(SEED, 0x7e30 + wt, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7e31 + T, T * K).reshape(T, K)
    W = hipmoe.QMat(q, wt, N, K)
    try:
        got = W.mul(x)
    finally:
        W.free()
    want = oracle.qmat_mul(x, q, wt, N, K)
    nbad = int(np.sum(bits(got) != bits(want)))
    say(f"kquant qmat full size: {nbad} of {want.size} outputs differ")
    assert nbad == 0


def test_gpu_kquant_qmat_graph_replays():
    say("HIP graph of K-quant products (Q6_K 2000 x 2048 T=1, Q4_K 2000 x 2048 T=3)")
    H = hipmoe.hip()
    N, K = 2000, 2048
    q6 = hipmoe.synth_quant_matrix(SEED, 0x7e40, 0.02, hipmoe.Q6_K, N, K)
    q4 = hipmoe.synth_quant_matrix(SEED, 0x7e41, 0.02, hipmoe.Q4_K, N, K)
    x1 = hipmoe.synth_normal(SEED, 0x7e42, K).reshape(1, K)
    x3 = hipmoe.synth_normal(SEED, 0x7e43, 3 * K).reshape(3, K)
    W6, W4 = hipmoe.QMat(q6, hipmoe.Q6_K, N, K), hipmoe.QMat(q4, hipmoe.Q4_K, N, K)
    e1, e3 = W6.mul(x1), W4.mul(x3)
    s = H.stream()
    d_x1, d_x3 = H.upload(x1), H.upload(x3)
    d_o1, d_o3 = H.malloc(N * 4), H.malloc(3 * N * 4)
    try:
        H.begin_capture(s)
        W6.mul_dev(d_x1, 1, d_o1, None, 0, s)
        W4.mul_dev(d_x3, 3, d_o3, None, 0, s)
        ge = H.end_capture(s)
        for rep in range(3):
            H.check(H.h.hipMemsetAsync(d_o1, 0, N * 4, s), "memset")
            H.check(H.h.hipMemsetAsync(d_o3, 0, 3 * N * 4, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            assert np.array_equal(bits(H.download(d_o1, (1, N), np.float32)), bits(e1)), rep
            assert np.array_equal(bits(H.download(d_o3, (3, N), np.float32)), bits(e3)), rep
            W4.mul(x3[:2])
        assert np.array_equal(bits(e1), bits(oracle.qmat_mul(x1, q6, hipmoe.Q6_K, N, K)))
        assert np.array_equal(bits(e3), bits(oracle.qmat_mul(x3, q4, hipmoe.Q4_K, N, K)))
    finally:
        for p in (d_x1, d_x3, d_o1, d_o3):
            H.free(p)
        W6.free()
        W4.free()


# ---- MoE layers on K-quant experts -----------------------------------------

def _kq_layer(name):
    sys.path.insert(0, __import__("os").path.dirname(__import__("os").path.abspath(__file__)))
    from test_oracle_kquant import kq_layer
    return kq_layer(name)


@pytest.mark.parametrize("name", ["olmoe_q4k_q6k", "olmoe_q6k", "mixtral_q4k_q6k",
                                  "ragged_q4k_q6k", "ragged_q6k_q4k"])
def test_gpu_kq_layer_vs_reference_golden(name):
    """hip_moe_upload_typed / hip_moe_ffn on K-quant experts: outputs equal the
    compiled reference's moe_ffn bit for bit, ids and weights the oracle's."""
    (wt, E, EI, NE, K, renorm, T), lw, x, want = _kq_layer(name)
    say(f"kq layer {name}: wtype={wt:#x} T={T} E={E} EI={EI} NE={NE} K={K}")
    M = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    try:
        M.set_path(hipmoe.PATH_GEMV)
        out, ids, w = M.ffn(x)
    finally:
        M.free()
    _, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), None)
    assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
    same = np.array_equal(bits(out), bits(want))
    say(f"kq layer {name}: bitwise {same}, rel L2 {rel_l2(out, want):.3e}")
    assert same


@pytest.mark.parametrize("T", [1, 13, 64])
def test_gpu_kq_layer_token_counts_vs_oracle(T):
    (wt, E, EI, NE, K, renorm, _), lw, _, _ = _kq_layer("olmoe_q4k_q6k")
    x = hipmoe.synth_input(SEED, 4000 + T, T, E)
    say(f"kq layer olmoe_q4k_q6k at T={T} against the oracle")
    M = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    try:
        out, ids, w = M.ffn(x)
    finally:
        M.free()
    oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), None)
    assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
    nbad = int(np.sum(bits(out) != bits(oout)))
    say(f"kq layer T={T}: {nbad} of {out.size} outputs differ")
    assert nbad == 0


@pytest.mark.parametrize("name,Ts", [("olmoe_q4k_q6k", (1,)), ("olmoe_q6k", (1,)),
                                     ("mixtral_q4k_q6k", (1, 2, 4))])
def test_gpu_kq_decode_path_vs_oracle(name, Ts):
    """The decode-sized K-quant layer (routing and gate/up in one launch;
    then, with d_ff up to 1024, down and combine in one launch without
    partials, else the per-pair down and the combine): outputs equal the
    oracle's moe_ffn (bit for bit the reference's, by the golden tests
    above) and the five-launch path's, ids and weights the oracle's, over
    successive calls (the routing epoch advances); past the routing slots
    (T * K > 64) the layer takes the per-pair products."""
    (wt, E, EI, NE, K, renorm, _), lw, _, _ = _kq_layer(name)
    M = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    try:
        for T in Ts:
            M.set_path(hipmoe.PATH_AUTO)
            assert M.path_for(T) == hipmoe.PATH_DECODE, (name, T)
            for rep in range(3):
                x = hipmoe.synth_input(SEED, 0x9300 + 16 * T + rep, T, E)
                M.set_path(hipmoe.PATH_AUTO)
                out, ids, w = M.ffn(x)
                M.set_path(hipmoe.PATH_GEMV)
                out_g, ids_g, w_g = M.ffn(x)
                oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), None)
                assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
                nbad = int(np.sum(bits(out) != bits(oout)))
                say(f"kq decode {name} T={T} call {rep}: {nbad} of {out.size} outputs differ")
                assert nbad == 0
                assert np.array_equal(bits(out), bits(out_g))
        M.set_path(hipmoe.PATH_AUTO)
        big = 64 // K + 1
        assert M.path_for(big) == hipmoe.PATH_GEMV, (name, big)
    finally:
        M.free()


KQ_DEC_SHAPES = {
    # name: (types, E, EI, NE, K, renorm, token counts)
    "mixtral_like_2048": (hipmoe.Q4_K | hipmoe.Q6_K << 8, 2048, 1024, 8, 2, 1, (1, 2, 4)),
    "top1_1024_half_chunk": (hipmoe.Q6_K | hipmoe.Q4_K << 8, 1024, 512, 16, 1, 0, (1, 8)),
    "e4096_ragged_chunk": (hipmoe.Q4_K, 4096, 768, 8, 2, 1, (1, 4)),
}


@pytest.mark.parametrize("name", sorted(KQ_DEC_SHAPES))
def test_gpu_kq_decode_down_combine_shapes_vs_oracle(name):
    """The one-launch down and combine at every pair bound it has an
    instance for (P = 1, 2, 4, 8), with d_ff of 4, 3 and 2 super-blocks
    (a staged chunk partly filled), renormalised (Mixtral) and plain
    (OLMoE) slot weights, both type mixes; the first launch's units at
    d_model 1024, 2048 and 4096 (64, 32, 16 rows a unit)."""
    wt, E, EI, NE, K, renorm, Ts = KQ_DEC_SHAPES[name]
    lw = hipmoe.synth_layer(SEED, 7, wt, E, EI, NE, 0.02, None)
    M = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    try:
        for T in Ts:
            assert M.path_for(T) == hipmoe.PATH_DECODE, (name, T)
            x = hipmoe.synth_input(SEED, 0x9400 + T, T, E)
            out, ids, w = M.ffn(x)
            oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), None)
            assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
            nbad = int(np.sum(bits(out) != bits(oout)))
            say(f"kq decode {name} T={T}: {nbad} of {out.size} outputs differ")
            assert nbad == 0
    finally:
        M.free()


@pytest.mark.parametrize("wt", [hipmoe.Q4_K | hipmoe.Q6_K << 8, hipmoe.Q6_K | hipmoe.Q4_K << 8,
                                hipmoe.Q4_K])
def test_gpu_kq_expert_ffn_vs_oracle(wt):
    E, EI, NE = 2048, 1024, 4
    lw = hipmoe.synth_layer(SEED, 3, wt, E, EI, NE, 0.02, None)
    x = hipmoe.synth_normal(SEED, 0x9020, E)
    say(f"kq expert ffn wtype={wt:#x}")
    M = hipmoe.MoeLayer.from_synth(lw, 2, False)
    try:
        for e in (0, 3):
            got = M.expert_ffn(e, x)
            want = oracle.fused_ffn(x, lw["gate"][e], lw["up"][e], lw["down"][e], wt, E, EI)
            assert np.array_equal(bits(got), bits(want)), (e, rel_l2(got, want))
        with pytest.raises(hipmoe.HipMoeError, match="does not apply"):
            M.set_path(hipmoe.PATH_GROUPED)
            M.ffn(x.reshape(1, E))
    finally:
        M.free()
