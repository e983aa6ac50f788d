"""GPU parity: the HIP path (through the C ABI) against the oracle and the
reference's golden vectors.

Bars:
  * expert ids, routing weights, router logits, softmax probabilities:
    bit-exact (the reference's AVX2 build, tests/golden/);
  * layer outputs: relative L2 <= 1e-3 against the reference CPU path
    (REL_L2_TOL); the fp32 paths (decode, GEMV) land near 1e-6, so their
    tests also assert a tighter 2e-5 to catch regressions early; the grouped
    path (f16 MFMA operands) lands near 5e-4 and is held to 1e-3;
  * the device expf: bit-exact with the host's glibc expf on every float in
    [-104, 0] and on a stride over all floats.
"""
import sys

import numpy as np
import pytest

import hipmoe
import oracle
from common import (CONFIGS, REL_L2_TOL, SEED, bits, golden, layer, qmat_case, qmat_cases,
                    rel_l2, router_inputs, sha)

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    n = hipmoe.hip().device_count()
    assert n >= 1, "no HIP device visible: GPU tests need an MI355X"


_layers = {}


def gpu_layer(cfg):
    if cfg not in _layers:
        _layers.clear()
        wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
        say(f"upload {cfg}")
        _layers[cfg] = hipmoe.MoeLayer.from_synth(layer(cfg), K, bool(renorm))
    return _layers[cfg]


# --------------------------------------------------------------------------
# expf
# --------------------------------------------------------------------------

def _expf_chunk(b0, n, step=1):
    u = (np.arange(n, dtype=np.uint64) * step + b0).astype(np.uint32)
    x = u.view(np.float32)
    g = hipmoe.expf_dev(x)
    if step == 1:
        ref = oracle.expf_bits(b0, n)
    else:
        ref = oracle.expf(x)
    same = (bits(g) == bits(ref)) | (np.isnan(g) & np.isnan(ref))
    return int((~same).sum()), (int(u[~same][0]) if (~same).any() else None)


def test_gpu_expf_softmax_range_exhaustive():
    say("expf exhaustive over [-104, 0]")
    lo = 0x80000000
    hi = int(np.array([-104.0], np.float32).view(np.uint32)[0])
    chunk = 1 << 25
    b = lo
    while b <= hi:
        n = min(chunk, hi - b + 1)
        bad, first = _expf_chunk(b, n)
        assert bad == 0, f"{bad} mismatches from {first:#x}"
        b += n
    bad, _ = _expf_chunk(0, 1)
    assert bad == 0


def test_gpu_expf_all_floats_strided():
    say("expf strided over all floats")
    bad, first = _expf_chunk(0, (1 << 32) // 61 + 1, 61)
    assert bad == 0, f"{bad} mismatches from {first:#x}"


# --------------------------------------------------------------------------
# routing
# --------------------------------------------------------------------------

@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_gpu_routing_bits_vs_reference(cfg):
    say(f"routing {cfg}")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    g = golden(f"route_{cfg}.npz")
    T = int(g["T"])
    wr, bias, x = router_inputs(cfg, T, int(g["input_call"]))
    assert sha(wr) == str(g["sha_router"]) and sha(x) == str(g["sha_x"])
    lay = gpu_layer(cfg)
    assert np.array_equal(bits(lay.router), bits(wr))
    lg, pr, ids, w = lay.route(x, bias)
    keep = g["logits"].shape[0]
    assert np.array_equal(bits(lg[:keep]), bits(g["logits"]))
    assert np.array_equal(bits(pr[:keep]), bits(g["probs"]))
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(bits(w), bits(g["w"]))


def _oracle_route(x, wr, bias, K, renorm):
    lg = oracle.router(x, wr, bias)
    ids = np.empty((x.shape[0], K), np.uint32)
    w = np.empty((x.shape[0], K), np.float32)
    for t in range(x.shape[0]):
        i, ww = oracle.top_k(oracle.softmax(lg[t]), K)
        if renorm:
            s = np.float32(0)
            for v in ww:
                s = np.float32(s + v)
            ww = (ww / s).astype(np.float32)
        ids[t], w[t] = i, ww
    return ids, w


@pytest.mark.parametrize("case", ["equal_logits", "expert0_dominant", "expert0_second",
                                  "huge_spread"])
def test_gpu_routing_edge_cases(case):
    say(f"routing edge case {case}")
    lay = gpu_layer("olmoe_q8")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS["olmoe_q8"]
    x = hipmoe.synth_input(SEED, 9, 16, E)
    bias = np.zeros(NE, np.float32)
    if case == "equal_logits":
        x = np.zeros_like(x)
    elif case == "expert0_dominant":
        bias[0] = 50.0
    elif case == "expert0_second":
        bias[0] = 30.0
        bias[17] = 31.0
    elif case == "huge_spread":
        bias[:] = np.linspace(-200, 0, NE, dtype=np.float32)
    lg, pr, ids, w = lay.route(x, bias)
    oids, ow = _oracle_route(x, lay.router, bias, K, False)
    assert np.array_equal(ids, oids)
    assert np.array_equal(bits(w), bits(ow))
    if case == "equal_logits":
        assert (ids == 0).all()


@pytest.mark.parametrize("NE,T", [(64, 77), (64, 133), (24, 150)])
def test_gpu_router_many_token_tiles_ragged(NE, T):
    """The many-token router tiles (16 experts x 8 tokens, from 36 tiles on)
    at a token count that leaves the last token tile partial and an expert
    count that leaves the last expert tile half empty: every logit equal,
    bit for bit, to the oracle's router (matmul.c:91-105, vector_avx2.h:126-132,
    pinned to the reference by the route goldens)."""
    say(f"router tiles NE={NE} T={T}")
    E = 2048
    if NE == 64:
        lay = gpu_layer("olmoe_q8")
        K = CONFIGS["olmoe_q8"][4]
    else:
        K = 4
        lay = hipmoe.MoeLayer.from_synth(
            hipmoe.synth_layer(SEED, 3, hipmoe.Q8_0, E, 256, NE, 0.02, None), K, False)
    assert ((T + 7) // 8) * ((NE + 15) // 16) >= 36  # the many-token tiles
    x = hipmoe.synth_input(SEED, 40 + T, T, E)
    bias = np.random.default_rng(T).standard_normal(NE).astype(np.float32)
    try:
        lg, pr, ids, w = lay.route(x, bias)
        assert np.array_equal(bits(lg), bits(oracle.router(x, lay.router, bias)))
        oids, ow = _oracle_route(x, lay.router, bias, K, False)
        assert np.array_equal(ids, oids)
        assert np.array_equal(bits(w), bits(ow))
    finally:
        if NE != 64:
            lay.free()


# --------------------------------------------------------------------------
# one expert, one token (fused_ffn_silu)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("wtype,name", [(hipmoe.Q8_0, "q8_0"), (hipmoe.Q4_0, "q4_0")])
def test_gpu_expert_ffn_vs_reference(wtype, name):
    say(f"expert ffn {name}")
    g = golden(f"ffn_{name}.npz")
    E, EI = 2048, 1024
    gm = hipmoe.synth_quant_matrix(SEED, 0x9001, 0.02, wtype, EI, E)
    um = hipmoe.synth_quant_matrix(SEED, 0x9002, 0.02, wtype, EI, E)
    dm = hipmoe.synth_quant_matrix(SEED, 0x9003, 0.02, wtype, E, EI)
    x = hipmoe.synth_normal(SEED, 0x9004, E)
    assert sha(gm) == str(g["sha_gate"]) and sha(dm) == str(g["sha_down"])
    lay = hipmoe.MoeLayer(np.zeros((1, E), np.float32), gm.reshape(1, -1), um.reshape(1, -1),
                          dm.reshape(1, -1), wtype, E, EI, 1, 1, False)
    out = lay.expert_ffn(0, x)
    lay.free()
    err = rel_l2(out, g["out"])
    say(f"expert ffn {name}: rel L2 {err:.3e}")
    assert err <= REL_L2_TOL and err <= TIGHT


# --------------------------------------------------------------------------
# whole layers
# --------------------------------------------------------------------------

@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_gpu_moe_layer_vs_reference_golden(cfg):
    say(f"moe layer golden {cfg}")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    g = golden(f"moe_{cfg}.npz")
    T = int(g["T"])
    lay = gpu_layer(cfg)
    x = hipmoe.synth_input(SEED, 0, T, E)
    assert sha(x) == str(g["sha_x"])
    out, ids, w = lay.ffn(x, layer(cfg)["bias"])
    err = rel_l2(out, g["out"])
    say(f"moe layer golden {cfg}: rel L2 {err:.3e}")
    assert err <= REL_L2_TOL and err <= TIGHT
    lay.set_path(hipmoe.PATH_GROUPED)
    try:
        gout, gids, gw = lay.ffn(x, layer(cfg)["bias"])
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    gerr = rel_l2(gout, g["out"])
    say(f"moe layer golden {cfg} [grouped]: rel L2 {gerr:.3e}")
    assert np.array_equal(gids, ids) and np.array_equal(bits(gw), bits(w))
    assert gerr <= REL_L2_TOL


PATH_NAMES = {hipmoe.PATH_DECODE: "decode", hipmoe.PATH_GEMV: "gemv",
              hipmoe.PATH_GROUPED: "grouped"}


def _check_layer_vs_oracle(cfg, T, call, per_token=True, path=hipmoe.PATH_AUTO,
                           expect_path=None):
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lay = gpu_layer(cfg)
    lw = layer(cfg)
    x = hipmoe.synth_input(SEED, call, T, E)
    lay.set_path(path)
    try:
        taken = lay.path_for(T)
        if expect_path is not None:
            assert taken == expect_path
        out, ids, w = lay.ffn(x, lw["bias"])
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), lw["bias"])
    assert np.array_equal(ids, oids)
    assert np.array_equal(bits(w), bits(ow))
    err = rel_l2(out, oout)
    worst = max(rel_l2(out[t], oout[t]) for t in range(T)) if per_token else err
    say(f"{cfg} T={T} [{PATH_NAMES[taken]}]: rel L2 {err:.3e}, worst token {worst:.3e}")
    assert err <= REL_L2_TOL and worst <= REL_L2_TOL
    if taken != hipmoe.PATH_GROUPED:
        assert err <= TIGHT
    return out


def test_gpu_olmoe_q8_decode_tokens():
    say("olmoe_q8 decode T=1 x 24 calls")
    for call in range(24):
        _check_layer_vs_oracle("olmoe_q8", 1, 100 + call)


def test_gpu_olmoe_q8_batch():
    say("olmoe_q8 T=64")
    _check_layer_vs_oracle("olmoe_q8", 64, 200)


def test_gpu_olmoe_q4_skew_prefill_512():
    say("olmoe_q4_skew prefill T=512")
    _check_layer_vs_oracle("olmoe_q4_skew", 512, 300, expect_path=hipmoe.PATH_GROUPED)


def test_gpu_mixtral_q4_decode_and_64():
    say("mixtral_q4 T=1")
    _check_layer_vs_oracle("mixtral_q4", 1, 400)
    say("mixtral_q4 T=64")
    _check_layer_vs_oracle("mixtral_q4", 64, 401, expect_path=hipmoe.PATH_GROUPED)


# --------------------------------------------------------------------------
# the grouped path (sort by expert + f16 MFMA GEMMs)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("cfg,T", [("olmoe_q8", 1), ("olmoe_q8", 3), ("olmoe_q8", 130),
                                   ("olmoe_q4_skew", 40), ("mixtral_q4", 5)])
def test_gpu_grouped_forced_small_and_ragged(cfg, T):
    """Heavy padding (1..few rows per expert tile), ragged tile tails,
    duplicated expert-0 slots (top_k quirk) all go through the sort."""
    say(f"grouped path forced: {cfg} T={T}")
    _check_layer_vs_oracle(cfg, T, 700 + T, path=hipmoe.PATH_GROUPED,
                           expect_path=hipmoe.PATH_GROUPED)


def test_gpu_grouped_tile_size_switch():
    """The m-tile shrinks from 64 to 32 rows below 32 pairs per expert, and
    the smaller call then needs more tiles: T=256 (2048 pairs, 64-row tiles)
    sizes a fresh layer's scratch, then T=255 (2040 pairs, 32-row tiles,
    up to 64 + 64 = 128 tiles) must fit it."""
    say("grouped path: T=256 then T=255 on a fresh layer (tile size switch)")
    cfg = "olmoe_q4_skew"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lay = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    try:
        for T, call in ((256, 750), (255, 751)):
            x = hipmoe.synth_input(SEED, call, T, E)
            assert lay.path_for(T) == hipmoe.PATH_GROUPED
            out, ids, w = lay.ffn(x, lw["bias"])
            oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, bool(renorm), lw["bias"])
            assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
            err = rel_l2(out, oout)
            say(f"{cfg} T={T}: rel L2 {err:.3e}")
            assert err <= REL_L2_TOL
    finally:
        lay.free()


def test_gpu_grouped_q8_prefill_512():
    say("olmoe_q8 prefill T=512 (grouped, Q8_0)")
    _check_layer_vs_oracle("olmoe_q8", 512, 710, expect_path=hipmoe.PATH_GROUPED)


def test_gpu_grouped_full_tiles():
    """Every token picks the same experts, so each expert's row count (128)
    is an exact multiple of the m-tile (32 rows here: 8 experts of 64
    average 16 pairs; no padding rows)."""
    say("grouped path, identical tokens: full tiles")
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lay = gpu_layer(cfg)
    lw = layer(cfg)
    x = np.repeat(hipmoe.synth_input(SEED, 720, 1, E), 128, axis=0)
    lay.set_path(hipmoe.PATH_GROUPED)
    try:
        out, ids, w = lay.ffn(x)
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    o1, i1, w1, _, _ = oracle.moe_ffn(x[:1], lw, K, False, None)
    assert (ids == i1[0]).all() and (bits(w) == bits(w1[0])).all()
    for t in (0, 63, 64, 127):
        assert rel_l2(out[t], o1[0]) <= REL_L2_TOL
    assert np.array_equal(bits(out), bits(np.repeat(out[:1], 128, axis=0)))


def test_gpu_grouped_deterministic_and_permutation():
    say("grouped path: determinism + token permutation (olmoe_q4_skew, T=256)")
    lay = gpu_layer("olmoe_q4_skew")
    lw = layer("olmoe_q4_skew")
    x = hipmoe.synth_input(SEED, 730, 256, 2048)
    assert lay.path_for(256) == hipmoe.PATH_GROUPED
    a, ia, wa = lay.ffn(x, lw["bias"])
    b, ib, wb = lay.ffn(x, lw["bias"])
    assert np.array_equal(bits(a), bits(b))
    perm = np.random.default_rng(5).permutation(256)
    c, ic, wc = lay.ffn(x[perm], lw["bias"])
    assert np.array_equal(ic, ia[perm])
    # a row's MFMA sums do not depend on the rows sharing its tile
    assert np.array_equal(bits(c), bits(a[perm]))


def test_gpu_grouped_vs_gemv_paths():
    say("grouped vs GEMV path (mixtral_q4, T=16)")
    lay = gpu_layer("mixtral_q4")
    x = hipmoe.synth_input(SEED, 740, 16, 4096)
    lay.set_path(hipmoe.PATH_GEMV)
    try:
        g, ig, wg = lay.ffn(x)
        lay.set_path(hipmoe.PATH_GROUPED)
        m, im, wm = lay.ffn(x)
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    assert np.array_equal(ig, im) and np.array_equal(bits(wg), bits(wm))
    assert rel_l2(m, g) <= REL_L2_TOL


def test_gpu_mixtral_T16_vs_oracle():
    """The MoE layer of sixteen sequences decoding together (one token each):
    Mixtral Q4_0 at T=16 on the path the layer picks (grouped) against the
    oracle's moe_ffn, ids and weights bit-exact."""
    say("mixtral_q4 T=16 vs oracle")
    _check_layer_vs_oracle("mixtral_q4", 16, 741, expect_path=hipmoe.PATH_GROUPED)


# --------------------------------------------------------------------------
# size-independent properties
# --------------------------------------------------------------------------

def test_gpu_deterministic_and_token_permutation():
    say("determinism + token permutation (olmoe_q8, T=96)")
    lay = gpu_layer("olmoe_q8")
    x = hipmoe.synth_input(SEED, 500, 96, 2048)
    a, ia, wa = lay.ffn(x)
    b, ib, wb = lay.ffn(x)
    assert np.array_equal(bits(a), bits(b)) and np.array_equal(ia, ib)
    perm = np.random.default_rng(3).permutation(96)
    c, ic, wc = lay.ffn(x[perm])
    assert np.array_equal(ic, ia[perm]) and np.array_equal(bits(wc), bits(wa[perm]))
    assert rel_l2(c, a[perm]) <= TIGHT


def test_gpu_decode_equals_batched():
    say("T=1 calls vs one T=16 call on the GEMV and grouped paths (olmoe_q8)")
    lay = gpu_layer("olmoe_q8")
    x = hipmoe.synth_input(SEED, 501, 16, 2048)
    try:
        lay.set_path(hipmoe.PATH_GEMV)
        gemv, ig, wg = lay.ffn(x)
        lay.set_path(hipmoe.PATH_AUTO)
        assert lay.path_for(16) == hipmoe.PATH_GROUPED
        grouped, ib, wb = lay.ffn(x)
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    assert np.array_equal(ig, ib) and np.array_equal(bits(wg), bits(wb))
    for t in range(16):
        o, i, w = lay.ffn(x[t:t + 1])
        assert np.array_equal(i[0], ib[t]) and np.array_equal(bits(w[0]), bits(wb[t]))
        assert rel_l2(o[0], gemv[t]) <= TIGHT
        assert rel_l2(o[0], grouped[t]) <= REL_L2_TOL


def test_gpu_dev_entry_matches_host_entry():
    say("hip_moe_ffn_dev vs hip_moe_ffn (olmoe_q8, T=8)")
    H = hipmoe.hip()
    lay = gpu_layer("olmoe_q8")
    x = hipmoe.synth_input(SEED, 502, 8, 2048)
    ref, ids, w = lay.ffn(x)
    d_x = H.upload(x)
    d_o = H.malloc(x.nbytes)
    d_i = H.malloc(8 * 8 * 4)
    d_w = H.malloc(8 * 8 * 4)
    try:
        lay.ffn_dev(d_x, d_o, 8, None, d_i, d_w)
        H.sync()
        out = H.download(d_o, x.shape, np.float32)
        assert np.array_equal(bits(out), bits(ref))
        assert np.array_equal(H.download(d_i, (8, 8), np.uint32), ids)
    finally:
        for p in (d_x, d_o, d_i, d_w):
            H.free(p)


# --------------------------------------------------------------------------
# the persistent decode kernel (T*K <= 64): boundary, reuse, graph replays
# --------------------------------------------------------------------------

def test_gpu_fused_boundary_T8():
    say("olmoe_q8 T=8 (T*K = 64, largest persistent launch)")
    _check_layer_vs_oracle("olmoe_q8", 8, 600, path=hipmoe.PATH_DECODE,
                           expect_path=hipmoe.PATH_DECODE)


def test_gpu_auto_path_boundaries():
    """AUTO takes the decode launch while 4*T*k <= 3*NE, the grouped path
    above it."""
    for cfg, t_dec in (("olmoe_q8", 6), ("mixtral_q4", 3)):
        lay = gpu_layer(cfg)
        assert lay.path_for(t_dec) == hipmoe.PATH_DECODE, cfg
        assert lay.path_for(t_dec + 1) == hipmoe.PATH_GROUPED, cfg


def test_gpu_fused_many_calls_reset_counters():
    say("olmoe_q8: 64 consecutive T=1 calls, each checked")
    lay = gpu_layer("olmoe_q8")
    lw = layer("olmoe_q8")
    xs = hipmoe.synth_input(SEED, 601, 64, 2048)
    oout, oids, ow, _, _ = oracle.moe_ffn(xs, lw, 8, False, None)
    for t in range(64):
        out, ids, w = lay.ffn(xs[t:t + 1])
        assert np.array_equal(ids[0], oids[t]) and np.array_equal(bits(w[0]), bits(ow[t]))
        assert rel_l2(out[0], oout[t]) <= TIGHT


def test_gpu_fresh_layer_after_freed_layer():
    """A layer allocated where a freed layer's scratch lived must not take that
    layer's epoch-tagged partials for its own (its epoch restarts at 1)."""
    say("fresh layer after a freed one: first decode calls")
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    xs = hipmoe.synth_input(SEED, 610, 6, E)
    oout, oids, ow, _, _ = oracle.moe_ffn(xs, lw, K, False, None)
    for rnd in range(3):
        lay = hipmoe.MoeLayer.from_synth(lw, K, False)
        for t in range(6):
            out, ids, w = lay.ffn(xs[t:t + 1])
            assert np.array_equal(ids[0], oids[t])
            assert rel_l2(out[0], oout[t]) <= TIGHT, (rnd, t)
        lay.free()


def test_gpu_default_stream_orders_layers():
    """Calls without a stream on different layers share one stream per
    device: decode launches of several layers, enqueued back to back without
    waiting, must not overlap (a persistent grid needs every CU) and must
    each give the eager result."""
    say("4 layers x 6 rounds of T=1 decode calls on the default stream")
    H = hipmoe.hip()
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lays = [gpu_layer(cfg)] + [hipmoe.MoeLayer.from_synth(lw, K, False) for _ in range(3)]
    xs = hipmoe.synth_input(SEED, 612, 6, E)
    eager = [lays[0].ffn(xs[r:r + 1])[0][0] for r in range(6)]
    d_x = H.upload(xs)
    d_o = H.malloc(6 * 4 * E * 4)
    try:
        for r in range(6):
            for i, lay in enumerate(lays):
                lay.ffn_dev(d_x + r * E * 4, d_o + (r * 4 + i) * E * 4, 1)
        H.sync()
        got = H.download(d_o, (6, 4, E), np.float32)
        for r in range(6):
            for i in range(4):
                assert np.array_equal(bits(got[r, i]), bits(eager[r])), (r, i)
        for lay in lays:  # a synchronous call reports any expired wait
            lay.ffn(xs[:1])
    finally:
        H.free(d_x)
        H.free(d_o)
        for lay in lays[1:]:
            lay.free()


def test_gpu_graph_replays_match_eager():
    say("HIP graph of 4 decode calls, replayed 5 times")
    H = hipmoe.hip()
    lay = gpu_layer("olmoe_q8")
    xs = hipmoe.synth_input(SEED, 602, 4, 2048)
    eager = np.stack([lay.ffn(xs[i:i + 1])[0][0] for i in range(4)])
    s = H.stream()
    d_x = H.upload(xs)
    d_o = H.malloc(4 * 2048 * 4)
    try:
        for i in range(4):  # eager warm-up on the capture stream
            lay.ffn_dev(d_x + i * 8192, d_o + i * 8192, 1, None, None, None, s)
        H.stream_sync(s)
        H.begin_capture(s)
        for i in range(4):
            lay.ffn_dev(d_x + i * 8192, d_o + i * 8192, 1, None, None, None, s)
        ge = H.end_capture(s)
        for rep in range(5):
            H.check(H.h.hipMemsetAsync(d_o, 0, 4 * 2048 * 4, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            got = H.download(d_o, (4, 2048), np.float32)
            assert np.array_equal(bits(got), bits(eager)), f"replay {rep}"
            lay.ffn(xs[:1])  # eager work between replays
    finally:
        H.free(d_x)
        H.free(d_o)


def test_gpu_graph_replays_grouped():
    """The grouped path (router, top-k, sort, GEMMs, combine) in a HIP graph:
    every replay equals the eager call, with eager calls of other sizes on
    the same scratch between the replays."""
    say("HIP graph of grouped calls (mixtral_q4 T=64 and T=16), replayed 3 times")
    H = hipmoe.hip()
    lay = gpu_layer("mixtral_q4")
    E = 4096
    xa = hipmoe.synth_input(SEED, 606, 64, E)
    xb = hipmoe.synth_input(SEED, 607, 16, E)
    assert lay.path_for(64) == hipmoe.PATH_GROUPED and lay.path_for(16) == hipmoe.PATH_GROUPED
    ea, eb = lay.ffn(xa)[0], lay.ffn(xb)[0]
    s = H.stream()
    d_a, d_b = H.upload(xa), H.upload(xb)
    d_oa, d_ob = H.malloc(xa.nbytes), H.malloc(xb.nbytes)
    try:
        lay.ffn_dev(d_a, d_oa, 64, None, None, None, s)  # eager warm-up on the stream
        lay.ffn_dev(d_b, d_ob, 16, None, None, None, s)
        H.stream_sync(s)
        H.begin_capture(s)
        lay.ffn_dev(d_a, d_oa, 64, None, None, None, s)
        lay.ffn_dev(d_b, d_ob, 16, None, None, None, s)
        ge = H.end_capture(s)
        for rep in range(3):
            H.check(H.h.hipMemsetAsync(d_oa, 0, xa.nbytes, s), "memset")
            H.check(H.h.hipMemsetAsync(d_ob, 0, xb.nbytes, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            assert np.array_equal(bits(H.download(d_oa, xa.shape, np.float32)), bits(ea)), rep
            assert np.array_equal(bits(H.download(d_ob, xb.shape, np.float32)), bits(eb)), rep
            lay.ffn(xb[:9])  # eager grouped work of another size between replays
    finally:
        for p in (d_a, d_b, d_oa, d_ob):
            H.free(p)


def test_gpu_mixtral_fused_T2_and_T32():
    say("mixtral_q4 T=2 (persistent path), T=4 and T=32 forced onto it")
    _check_layer_vs_oracle("mixtral_q4", 2, 603, expect_path=hipmoe.PATH_DECODE)
    _check_layer_vs_oracle("mixtral_q4", 4, 605, path=hipmoe.PATH_DECODE,
                           expect_path=hipmoe.PATH_DECODE)
    _check_layer_vs_oracle("mixtral_q4", 32, 604, path=hipmoe.PATH_DECODE,
                           expect_path=hipmoe.PATH_DECODE)


# --------------------------------------------------------------------------
# dense quantized products (tensor_mma_transposed_2x2 on Q8_0/Q4_0)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("i,name", list(enumerate(qmat_cases()[0])))
def test_gpu_qmat_vs_reference_golden(i, name):
    """hip_moe_qmat_mul against the compiled reference's product (fixture):
    fp32 dots in another order, held to the fp32 bar TIGHT."""
    wt, T, N, K, q, x, a, want = qmat_case(i, name)
    say(f"qmat {name}: T={T} N={N} K={K}")
    W = hipmoe.QMat(q, wt, N, K)
    got = W.mul(x, a)
    W.free()
    err = rel_l2(got, want)
    say(f"qmat {name}: rel L2 {err:.3e}")
    assert err <= TIGHT


@pytest.mark.parametrize("wt,N,K", [(hipmoe.Q8_0, 50304, 2048), (hipmoe.Q4_0, 32000, 4096)])
def test_gpu_qmat_lm_head_full_size(wt, N, K):
    """The lm_head shapes (OLMoE Q8_0 50304 x 2048, Mixtral Q4_0 32000 x
    4096), one token: every logit within the fp32 bar of the oracle, and the
    same greedy token where the top two logits are apart."""
    say(f"qmat lm_head wt={wt} N={N} K={K}")
    q = hipmoe.synth_quant_matrix(SEED, 0x7700 + wt, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7701 + wt, K).reshape(1, K)
    W = hipmoe.QMat(q, wt, N, K)
    assert W.bytes() == N * hipmoe.row_bytes(wt, K)
    got = W.mul(x)
    W.free()
    want = oracle.qmat_mul(x, q, wt, N, K)
    err = rel_l2(got, want)
    say(f"qmat lm_head: rel L2 {err:.3e}")
    assert err <= TIGHT
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    top2 = np.sort(want[0])[-2:]
    if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
        assert int(np.argmax(got)) == int(np.argmax(want))


@pytest.mark.parametrize("wt", [hipmoe.Q8_0, hipmoe.Q4_0])
def test_gpu_qmat_matrix_cores_vs_oracle(wt):
    """Several tokens take the matrix-core product (tokens split into two
    f16 parts under a per-block power of two, unscaled quants, the block
    scale applied in fp32): every K it takes (256 .. 4096), token counts
    that fill one tile, pad one (T = 3) and span three (T = 33), ragged N,
    held to the fp32 bar TIGHT against the oracle; T = 65 goes past the
    split buffer of the device entry point (the per-token product) and
    through the host entry point (which grows it)."""
    H = hipmoe.hip()
    for K in (256, 512, 1024, 2048, 4096):
        N = 16 * (K // 256) + 7
        q = hipmoe.synth_quant_matrix(SEED, 0x7c00 + K + wt, 0.02, wt, N, K)
        W = hipmoe.QMat(q, wt, N, K)
        try:
            for T in (3, 16, 33):
                x = hipmoe.synth_normal(SEED, 0x7d00 + K + T + wt, T * K).reshape(T, K)
                a = hipmoe.synth_normal(SEED, 0x7e00 + K + T, N) if T == 16 else None
                got = W.mul(x, a)
                err = rel_l2(got, oracle.qmat_mul(x, q, wt, N, K, a))
                say(f"qmm wt={wt} K={K} N={N} T={T}: rel L2 {err:.3e}")
                assert err <= TIGHT
            if K == 2048:
                T = 65
                x = hipmoe.synth_normal(SEED, 0x7f00 + wt, T * K).reshape(T, K)
                want = oracle.qmat_mul(x, q, wt, N, K)
                d_x, d_o = H.upload(x), H.malloc(T * N * 4)
                try:
                    W.mul_dev(d_x, T, d_o, None, 0, None)
                    H.sync()
                    assert rel_l2(H.download(d_o, (T, N), np.float32), want) <= TIGHT
                finally:
                    H.free(d_x)
                    H.free(d_o)
                assert rel_l2(W.mul(x), want) <= TIGHT
        finally:
            W.free()


def test_gpu_qmat_dev_token_groups_on_stream():
    """Device-pointer entry point on a caller's stream, T = 8 at K = 4096
    (the matrix-core product), N = 257 (a partial last workgroup), add
    [T][N], then add [N] on the same buffers."""
    H = hipmoe.hip()
    wt, N, K, T = hipmoe.Q4_0, 257, 4096, 8
    q = hipmoe.synth_quant_matrix(SEED, 0x7800, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7801, T * K).reshape(T, K)
    a_rows = hipmoe.synth_normal(SEED, 0x7802, T * N)
    a_bc = hipmoe.synth_normal(SEED, 0x7803, N)
    W = hipmoe.QMat(q, wt, N, K)
    s = H.stream()
    d_x, d_ar, d_ab = H.upload(x), H.upload(a_rows), H.upload(a_bc)
    d_o = H.malloc(T * N * 4)
    try:
        for d_a, a in ((d_ar, a_rows), (d_ab, a_bc)):
            say(f"qmat dev: add of {a.size}")
            W.mul_dev(d_x, T, d_o, d_a, a.size, s)
            H.stream_sync(s)
            got = H.download(d_o, (T, N), np.float32)
            err = rel_l2(got, oracle.qmat_mul(x, q, wt, N, K, a))
            say(f"qmat dev: rel L2 {err:.3e}")
            assert err <= TIGHT
        with pytest.raises(hipmoe.HipMoeError, match="16-byte aligned"):
            W.mul_dev(d_x + 4, 1, d_o, None, 0, s)
        with pytest.raises(hipmoe.HipMoeError, match="add holds"):
            W.mul_dev(d_x, T, d_o, d_ab, N + 1, s)
    finally:
        for p in (d_x, d_ar, d_ab, d_o):
            H.free(p)
        W.free()


def test_gpu_qmat_graph_replays():
    """The dense product in a HIP graph (T = 1 and T = 6 with add [T][N]: two
    LDS token groups at K = 2048): every replay equals the eager call, with
    eager calls of another size between the replays."""
    say("HIP graph of dense products (Q8_0 1000 x 2048, T=1 and T=6), replayed 3 times")
    H = hipmoe.hip()
    wt, N, K = hipmoe.Q8_0, 1000, 2048
    q = hipmoe.synth_quant_matrix(SEED, 0x7900, 0.02, wt, N, K)
    x1 = hipmoe.synth_normal(SEED, 0x7901, K).reshape(1, K)
    x6 = hipmoe.synth_normal(SEED, 0x7902, 6 * K).reshape(6, K)
    a6 = hipmoe.synth_normal(SEED, 0x7903, 6 * N)
    W = hipmoe.QMat(q, wt, N, K)
    e1, e6 = W.mul(x1), W.mul(x6, a6)
    s = H.stream()
    d_x1, d_x6, d_a6 = H.upload(x1), H.upload(x6), H.upload(a6)
    d_o1, d_o6 = H.malloc(N * 4), H.malloc(6 * N * 4)
    try:
        H.begin_capture(s)
        W.mul_dev(d_x1, 1, d_o1, None, 0, s)
        W.mul_dev(d_x6, 6, d_o6, d_a6, 6 * N, s)
        ge = H.end_capture(s)
        for rep in range(3):
            H.check(H.h.hipMemsetAsync(d_o1, 0, N * 4, s), "memset")
            H.check(H.h.hipMemsetAsync(d_o6, 0, 6 * N * 4, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            assert np.array_equal(bits(H.download(d_o1, (1, N), np.float32)), bits(e1)), rep
            assert np.array_equal(bits(H.download(d_o6, (6, N), np.float32)), bits(e6)), rep
            W.mul(x6[:3])  # eager work of another size between replays
        assert rel_l2(e6, oracle.qmat_mul(x6, q, wt, N, K, a6)) <= TIGHT
    finally:
        for p in (d_x1, d_x6, d_a6, d_o1, d_o6):
            H.free(p)
        W.free()


@pytest.mark.parametrize("wt,c", [(hipmoe.Q8_0, 128.0), (hipmoe.Q4_0, 8.0)])
def test_gpu_qmat_mean_shifted_activations(wt, c):
    """The product's dots take sum((q + c) x) - c * sum(x) per block (c = 128
    for Q8_0, 8 for Q4_0), so their rounding grows with c * sum|x| rather
    than with |sum q x|.  Activations with a mean far above their spread
    (N(4, 0.25)) make that cancellation largest.  Bar: every output within
    the first-order bound 2^-24 * (32 * (127 + c) + 31 * c + 64 * 255) *
    B_j, with B_j = sum over blocks of |d_b| * sum over the block of |x_i|;
    and the whole output within 1e-5 relative L2 of the oracle."""
    N, K, T = 512, 2048, 2
    q = hipmoe.synth_quant_matrix(SEED, 0x7a00 + wt, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7a10 + wt, T * K, 4.0, 0.25).reshape(T, K)
    W = hipmoe.QMat(q, wt, N, K)
    got = W.mul(x)
    W.free()
    want = oracle.qmat_mul(x, q, wt, N, K)
    # the exact product: d * q is exact in fp32 (|q| <= 127, fp16 d)
    Wd = np.stack([oracle.dequant(q[j * hipmoe.row_bytes(wt, K):
                                        (j + 1) * hipmoe.row_bytes(wt, K)], wt, K)
                   for j in range(N)]).astype(np.float64)
    exact = x.astype(np.float64) @ Wd.T
    bb = 34 if wt == hipmoe.Q8_0 else 18
    d = np.abs(q.reshape(N, K // 32, bb)[:, :, :2].copy().view(np.float16)[..., 0]
               .astype(np.float64))                                    # [N][K/32]
    xs = np.abs(x.astype(np.float64)).reshape(T, K // 32, 32).sum(axis=2)  # [T][K/32]
    B = xs @ d.T                                                         # [T][N]
    bound = 2.0 ** -24 * (32 * (127 + c) + 31 * c + 64 * 255) * B
    dev = np.abs(got.astype(np.float64) - exact)
    err = rel_l2(got, want)
    say(f"qmat mean-shifted wt={wt}: rel L2 {err:.3e}, worst |err|/bound "
        f"{float(np.max(dev / bound)):.3e}")
    assert (dev <= bound).all()
    assert err <= 1e-5
