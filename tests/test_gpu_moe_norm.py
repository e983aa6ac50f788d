"""The one-token MoE launch that normalises its own input (moe_ffn_dev_norm:
the whole-model step's pre-MoE rms_norm, olmoe.c:486-488, inside the layer's
decode launch) against hip_moe_ffn_dev on the row it wrote out: the ids,
weights and outputs are bit for bit the same (every workgroup computes the
same row; the kernel after the norm is the plain one), and the row is
rms_norm(h) * w within 1e-6 of its float64 value.  Q8_0 (OLMoE shape) and
Q4_0 (Mixtral shape) take k_moe_decode, the K-quant layer the K-quant decode
launches."""
import ctypes as C
import sys

import numpy as np
import pytest

import hipmoe
from common import CONFIGS, SEED, bits, layer

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


def norm_lib():
    L = hipmoe.lib()
    vp = C.c_void_p
    L.moe_ffn_dev_norm.restype = C.c_int
    L.moe_ffn_dev_norm.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp]
    L.moe_norm_decode_ok.restype = C.c_int
    L.moe_norm_decode_ok.argtypes = [vp]
    return L


def layer_case(cfg):
    if cfg == "kq":
        sys.path.insert(0, __import__("os").path.dirname(__import__("os").path.abspath(__file__)))
        from test_oracle_kquant import kq_layer
        (wt, E, EI, NE, K, renorm, _), lw, _, _ = kq_layer("olmoe_q4k_q6k")
        return E, K, hipmoe.MoeLayer.from_synth(lw, K, bool(renorm))
    wt, E, EI, NE, K, renorm, _ = CONFIGS[cfg]
    return E, K, hipmoe.MoeLayer.from_synth(layer(cfg), K, bool(renorm))


@pytest.mark.parametrize("cfg", ["olmoe_q8", "mixtral_q4", "kq"])
def test_gpu_moe_norm_matches_dev_entry(cfg):
    say(f"MoE launch normalising its input vs ffn_dev on that row: {cfg}")
    H, L = hipmoe.hip(), norm_lib()
    E, K, lay = layer_case(cfg)
    rng = np.random.default_rng(SEED + 77)
    bufs = []
    try:
        assert L.moe_norm_decode_ok(lay.h) == 1
        for call in range(2):  # a second call: the next launch epoch
            h = (rng.standard_normal(E) * (3.0 + call) + 0.25).astype(np.float32)
            w = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
            d_h, d_w = H.upload(h), H.upload(w)
            d_x, d_o1, d_o2 = (H.malloc(E * 4) for _ in range(3))
            idw = [H.malloc(K * 4) for _ in range(4)]
            bufs += [d_h, d_w, d_x, d_o1, d_o2] + idw
            assert L.moe_ffn_dev_norm(lay.h, d_h, d_w, d_x, d_o1, idw[0], idw[1], None) == 1, \
                hipmoe.last_error()
            H.sync()
            x = H.download(d_x, (E,), np.float32)
            h64, w64 = h.astype(np.float64), w.astype(np.float64)
            ref = h64 / np.sqrt(np.mean(h64 * h64) + 1e-5) * w64
            err = float(np.max(np.abs(x - ref)) / np.max(np.abs(ref)))
            assert err < 1e-6, f"call {call}: normalised row off by {err:.3e}"
            lay.ffn_dev(d_x, d_o2, 1, None, idw[2], idw[3])
            H.sync()
            a, b = (H.download(d, (E,), np.float32) for d in (d_o1, d_o2))
            ia, ib = (H.download(idw[i], (K,), np.uint32) for i in (0, 2))
            wa, wb = (H.download(idw[i], (K,), np.float32) for i in (1, 3))
            assert np.array_equal(ia, ib) and np.array_equal(bits(wa), bits(wb)), f"call {call}"
            assert np.array_equal(bits(a), bits(b)), f"call {call}"
            say(f"{cfg} call {call}: row within {err:.2e} of float64 rms_norm, "
                f"outputs equal ffn_dev bitwise")
    finally:
        for d in bufs:
            H.free(d)
        lay.free()
