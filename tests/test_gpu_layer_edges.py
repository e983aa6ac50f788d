"""GPU tests of the whole layer at its edges, through the C ABI:

  * the routing edge cases (equal logits, expert 0 dominant or second, a
    huge logit spread) on every path that routes on its own: the decode
    kernel's in-kernel routing (router rows, replica polls, softmax and the
    wave-split ranks of one token, and the per-wave routing of several
    tokens), the grouped path and the GEMV path, each against the oracle
    (ids and weight bits exact, outputs to the path's bar);
  * the GEMV path as a whole layer against the oracle;
  * the decode kernel's bounded waits: an expired wait is sticky (later
    calls write NaN instead of reading stale tagged data) until
    hip_moe_status reports it and resets the layer;
  * scratch growth refused under stream capture, hip_moe_reserve first.
"""
import sys

import numpy as np
import pytest

import hipmoe
import oracle
from common import CONFIGS, REL_L2_TOL, SEED, bits, layer, rel_l2

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


_layers = {}


def gpu_layer(cfg):
    if cfg not in _layers:
        _layers.clear()
        wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
        say(f"upload {cfg}")
        _layers[cfg] = hipmoe.MoeLayer.from_synth(layer(cfg), K, bool(renorm))
    return _layers[cfg]


EDGE_CASES = ["equal_logits", "expert0_dominant", "expert0_second", "huge_spread"]


def edge_inputs(case, T, E, NE):
    x = hipmoe.synth_input(SEED, 9, T, E)
    bias = np.zeros(NE, np.float32)
    if case == "equal_logits":
        x = np.zeros_like(x)  # every logit 0: top_k fills all slots with expert 0
    elif case == "expert0_dominant":
        bias[0] = 50.0
    elif case == "expert0_second":
        bias[0] = 30.0
        bias[min(17, NE - 1)] = 31.0
    elif case == "huge_spread":
        bias[:] = np.linspace(-200, 0, NE, dtype=np.float32)  # most probabilities 0
    return x, bias


NAMES = {hipmoe.PATH_DECODE: "decode", hipmoe.PATH_GEMV: "gemv",
         hipmoe.PATH_GROUPED: "grouped"}


def check_vs_oracle(cfg, x, bias, path):
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lay = gpu_layer(cfg)
    T = x.shape[0]
    lay.set_path(path)
    try:
        assert lay.path_for(T) == path
        out, ids, w = lay.ffn(x, bias)
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
    oout, oids, ow, _, _ = oracle.moe_ffn(x, layer(cfg), K, bool(renorm), bias)
    assert np.array_equal(ids, oids)
    assert np.array_equal(bits(w), bits(ow))
    err = rel_l2(out, oout)
    say(f"{cfg} T={T} [{NAMES[path]}]: rel L2 {err:.3e}")
    assert np.isfinite(out).all()
    assert err <= (REL_L2_TOL if path == hipmoe.PATH_GROUPED else TIGHT)
    return ids


@pytest.mark.parametrize("case", EDGE_CASES)
@pytest.mark.parametrize("path,T", [(hipmoe.PATH_DECODE, 1), (hipmoe.PATH_DECODE, 8),
                                    (hipmoe.PATH_GROUPED, 8), (hipmoe.PATH_GEMV, 3)])
def test_gpu_routing_edge_cases_in_layer(case, path, T):
    say(f"routing edge case {case} through the layer: path {NAMES[path]}, T={T}")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS["olmoe_q8"]
    x, bias = edge_inputs(case, T, E, NE)
    ids = check_vs_oracle("olmoe_q8", x, bias, path)
    if case == "equal_logits":
        assert (ids == 0).all()
    if case == "expert0_dominant":
        assert (ids[:, -1] == 0).all()


@pytest.mark.parametrize("case", ["expert0_second", "huge_spread"])
def test_gpu_routing_edge_cases_mixtral_decode(case):
    """Mixtral's renormalised weights (llama.c:422-427) through the decode
    kernel's routing at T=2."""
    say(f"routing edge case {case}: mixtral_q4 decode T=2")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS["mixtral_q4"]
    x, bias = edge_inputs(case, 2, E, NE)
    check_vs_oracle("mixtral_q4", x, bias, hipmoe.PATH_DECODE)


@pytest.mark.parametrize("cfg,T", [("olmoe_q8", 5), ("mixtral_q4", 2)])
def test_gpu_gemv_path_whole_layer_vs_oracle(cfg, T):
    say(f"GEMV path whole layer: {cfg} T={T}")
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    x = hipmoe.synth_input(SEED, 810 + T, T, E)
    check_vs_oracle(cfg, x, layer(cfg)["bias"], hipmoe.PATH_GEMV)


def test_gpu_decode_wait_error_is_sticky_until_status():
    """A wait bound of one poll makes the decode kernel's waits run out (the
    router logits need microseconds); every wait still ends.  The error
    stays set: the next device call, at the default bound, writes NaN
    instead of using the tagged data the failed launch left.  hip_moe_status
    reports it and resets the layer, after which calls are correct again."""
    say("decode kernel: forced wait expiry, sticky error, status + reset")
    H = hipmoe.hip()
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lay = hipmoe.MoeLayer.from_synth(lw, K, False)
    x = hipmoe.synth_input(SEED, 820, 2, E)
    oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, False, None)
    d_x = H.upload(x)
    d_o = H.malloc(x.nbytes)
    d_i = H.malloc(2 * K * 4)
    d_w = H.malloc(2 * K * 4)
    try:
        assert lay.status() == 0
        lay.ffn_dev(d_x, d_o, 1, None, d_i, d_w)
        H.sync()
        assert rel_l2(H.download(d_o, (1, E), np.float32), oout[:1]) <= TIGHT
        lay.set_wait_limit(1)
        for _ in range(3):
            lay.ffn_dev(d_x, d_o, 1, None, d_i, d_w)
        H.sync()
        lay.set_wait_limit(0)
        lay.ffn_dev(d_x + E * 4, d_o, 1, None, d_i, d_w)  # another token, default bound
        H.sync()
        poisoned = H.download(d_o, (1, E), np.float32)
        assert np.isnan(poisoned).all(), "a call after an expired wait must not compute"
        assert (H.download(d_i, (1, K), np.uint32) == 0).all()
        code = lay.status()
        say(f"status after forced expiry: {code} ({hipmoe.last_error()})")
        assert code in (1, 2, 3)
        assert lay.status() == 0  # reported once, then reset
        for t in (0, 1):
            lay.ffn_dev(d_x + t * E * 4, d_o, 1, None, d_i, d_w)
            H.sync()
            assert rel_l2(H.download(d_o, (1, E), np.float32), oout[t:t + 1]) <= TIGHT
            assert np.array_equal(H.download(d_i, (1, K), np.uint32), oids[t:t + 1])
        # the synchronous entry point reports and resets by itself
        lay.set_wait_limit(1)
        with pytest.raises(hipmoe.HipMoeError, match="timed out"):
            for _ in range(3):
                lay.ffn(x[:1])
        lay.set_wait_limit(0)
        out, ids, w = lay.ffn(x[1:])
        assert rel_l2(out, oout[1:]) <= TIGHT and np.array_equal(ids, oids[1:])
    finally:
        for p in (d_x, d_o, d_i, d_w):
            H.free(p)
        lay.free()


def test_gpu_scratch_growth_refused_under_capture():
    """A call that would grow the scratch while its stream is captured
    returns 0 and enqueues nothing; after hip_moe_reserve the same size
    captures, and the replays equal the eager calls."""
    say("scratch growth under capture: refused; reserve, then capture T=8")
    H = hipmoe.hip()
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lay = hipmoe.MoeLayer.from_synth(lw, K, False)
    x = hipmoe.synth_input(SEED, 830, 8, E)
    s = H.stream()
    d_x = H.upload(x)
    d_o = H.malloc(x.nbytes)
    try:
        lay.reserve(2)
        eager = lay.ffn(x[:2])[0]
        H.begin_capture(s)
        with pytest.raises(hipmoe.HipMoeError, match="hip_moe_reserve"):
            lay.ffn_dev(d_x, d_o, 8, None, None, None, s)
        lay.ffn_dev(d_x, d_o, 2, None, None, None, s)  # fits: captured
        ge = H.end_capture(s)
        for rep in range(3):
            H.check(H.h.hipMemsetAsync(d_o, 0, x.nbytes, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            got = H.download(d_o, (2, E), np.float32)
            assert np.array_equal(bits(got), bits(eager)), rep
        lay.reserve(8)
        e8 = lay.ffn(x)[0]
        H.begin_capture(s)
        lay.ffn_dev(d_x, d_o, 8, None, None, None, s)
        ge8 = H.end_capture(s)
        for rep in range(2):
            H.graph_launch(ge8, s)
            H.stream_sync(s)
            assert np.array_equal(bits(H.download(d_o, (8, E), np.float32)), bits(e8)), rep
            lay.ffn(x[:3])
    finally:
        H.free(d_x)
        H.free(d_o)
        lay.free()


# --------------------------------------------------------------------------
# the grouped path with the tokens crowded onto one or two experts
# --------------------------------------------------------------------------

_skew_layer = {}


def skew_layer():
    """A reduced Mixtral-shaped layer (d_model 2048, d_ff 1024, 8 experts,
    top-2 with renorm, Q4_0): 32-row tiles at these token counts."""
    if "lw" not in _skew_layer:
        _skew_layer["lw"] = hipmoe.synth_layer(SEED, 5, hipmoe.Q4_0, 2048, 1024, 8, 0.02, None)
    return _skew_layer["lw"]


@pytest.mark.parametrize("T", [52, 100])
@pytest.mark.parametrize("case", ["two_experts", "near_identical_tokens"])
def test_gpu_grouped_path_crowded_experts_vs_oracle(case, T):
    """Every token on the same two experts (a router bias), or tokens that
    differ only slightly (as a model's hidden states can): experts of
    T pairs span several 32-row tiles, others have none."""
    lw = skew_layer()
    E, NE, K = 2048, 8, 2
    x = hipmoe.synth_input(SEED, 830 + T, T, E)
    bias = None
    if case == "two_experts":
        bias = np.zeros(NE, np.float32)
        bias[3], bias[5] = 50.0, 40.0
    else:
        x = (x[:1] + 0.02 * x).astype(np.float32)
    say(f"grouped path, crowded experts: {case} T={T}")
    lay = hipmoe.MoeLayer.from_synth(lw, K, True)
    try:
        lay.set_path(hipmoe.PATH_GROUPED)
        assert lay.path_for(T) == hipmoe.PATH_GROUPED
        out, ids, w = lay.ffn(x, bias)
    finally:
        lay.free()
    oout, oids, ow, _, _ = oracle.moe_ffn(x, lw, K, True, bias)
    counts = np.bincount(oids.reshape(-1).astype(np.int64), minlength=NE)
    err = rel_l2(out, oout)
    say(f"  pairs per expert {counts.tolist()}: rel L2 {err:.3e}")
    assert np.array_equal(ids, oids) and np.array_equal(bits(w), bits(ow))
    assert err <= REL_L2_TOL
