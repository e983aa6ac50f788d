"""hip_moe_ffn_dev_noalloc (the decode path on the GPU's static scratch)
against hip_moe_ffn_dev, through the C ABI: bit-identical outputs, ids and
weights (the same kernel and arithmetic), on two calls in a row, the second
with fewer tokens, for both layer shapes; the allocation-free call runs first
on a fresh layer, whose own scratch does not exist yet.  Also: a graph
captured from it with no reserve step replays the eager result, a call past
the decode path is refused, and the outputs stay within the fp32 bar of the
oracle."""
import sys

import numpy as np
import pytest

import hipmoe
import oracle
from common import CONFIGS, SEED, bits, layer, rel_l2

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


@pytest.mark.parametrize("cfg,T1,T2", [("olmoe_q8", 8, 1), ("mixtral_q4", 3, 1)])
def test_gpu_noalloc_matches_dev_entry(cfg, T1, T2):
    say(f"noalloc vs ffn_dev: {cfg} T={T1} then T={T2}")
    H = hipmoe.hip()
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lay = hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    x = hipmoe.synth_input(SEED, 900, T1, E)
    d_x = H.upload(x)
    bufs = [H.malloc(T1 * E * 4), H.malloc(T1 * E * 4)]
    idw = [H.malloc(T1 * K * 4) for _ in range(4)]
    try:
        lay.set_path(hipmoe.PATH_DECODE)
        for T in (T1, T2):
            assert lay.path_for(T) == hipmoe.PATH_DECODE
            lay.ffn_dev_noalloc(d_x, bufs[0], T, None, idw[0], idw[1])
            H.sync()
            lay.ffn_dev(d_x, bufs[1], T, None, idw[2], idw[3])
            H.sync()
            a = H.download(bufs[0], (T, E), np.float32)
            b = H.download(bufs[1], (T, E), np.float32)
            ia, ib = (H.download(idw[i], (T, K), np.uint32) for i in (0, 2))
            wa, wb = (H.download(idw[i], (T, K), np.float32) for i in (1, 3))
            assert np.array_equal(bits(a), bits(b)), f"T={T}"
            assert np.array_equal(ia, ib) and np.array_equal(bits(wa), bits(wb))
            oout, oids, ow, _, _ = oracle.moe_ffn(x[:T], lw, K, bool(renorm), None)
            assert np.array_equal(ia, oids) and np.array_equal(bits(wa), bits(ow))
            err = rel_l2(a, oout)
            say(f"{cfg} T={T}: noalloc == ffn_dev bitwise, rel L2 vs oracle {err:.3e}")
            assert err <= TIGHT
        assert lay.status() == 0
    finally:
        lay.set_path(hipmoe.PATH_AUTO)
        for p in [d_x] + bufs + idw:
            H.free(p)
        lay.free()


def test_gpu_noalloc_graph_without_reserve_and_refusals():
    say("noalloc: graph capture on a fresh layer, replays; refusals")
    H = hipmoe.hip()
    cfg = "olmoe_q8"
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS[cfg]
    lw = layer(cfg)
    lay = hipmoe.MoeLayer.from_synth(lw, K, False)
    xs = hipmoe.synth_input(SEED, 910, 4, E)
    s = H.stream()
    d_x = H.upload(xs)
    d_o = H.malloc(xs.nbytes)
    try:
        H.begin_capture(s)
        for i in range(4):  # ids/weights left NULL: they go to the static array too
            lay.ffn_dev_noalloc(d_x + i * E * 4, d_o + i * E * 4, 1, None, None, None, s)
        ge = H.end_capture(s)
        oout, oids, ow, _, _ = oracle.moe_ffn(xs, lw, K, False, None)
        first = None
        for rep in range(3):
            H.check(H.h.hipMemsetAsync(d_o, 0, xs.nbytes, s), "memset")
            H.graph_launch(ge, s)
            H.stream_sync(s)
            got = H.download(d_o, (4, E), np.float32)
            if first is None:
                first = got
                assert rel_l2(got, oout) <= TIGHT
            assert np.array_equal(bits(got), bits(first)), rep
            lay.ffn(xs[:2])  # eager work of another size between replays
        with pytest.raises(hipmoe.HipMoeError, match="decode path"):
            lay.ffn_dev_noalloc(d_x, d_o, 9, None, None, None, s)  # T*K = 72 > 64
        lay.set_path(hipmoe.PATH_GROUPED)
        with pytest.raises(hipmoe.HipMoeError, match="decode path"):
            lay.ffn_dev_noalloc(d_x, d_o, 1, None, None, None, s)
        lay.set_path(hipmoe.PATH_AUTO)
        assert lay.status(s) == 0
    finally:
        H.free(d_x)
        H.free(d_o)
        lay.free()
