"""The drop-in itself: INTEGRATION.md's lines for OLMoE (the upload loop of
olmoe_load, the early return of moe_ffn, the free loop of olmoe_close)
compiled around the reference's own models/olmoe/olmoe.c and linked against
libhip_moe.so (tests/native/dropin_olmoe.c, built by oracle/ref/build_ref.sh
from the reference tree; skipped where that tree was not there to build it).

  * no GPU: hip_moe_upload returns NULL and the reference's CPU body runs,
    giving the golden layer output bit for bit (tests/golden/moe_olmoe_q8.npz);
  * with a GPU: the layer runs on it, within the output bar of the golden.

The reference's thread pool starts with its library and spins until the
process ends, so the library is loaded in a child process.
"""
import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB = os.path.join(REPO, "oracle", "_ref", "libdropin_olmoe.so")


def child():
    sys.path[:0] = [os.path.join(REPO, "llm.c_amd"), HERE]
    import hipmoe
    from common import CONFIGS, SEED, golden, layer, rel_l2, sha
    L = C.CDLL(LIB)
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    L.dropin_olmoe_moe_ffn.argtypes = [vp, vp, sz, vp, vp, vp, vp, i32, sz, sz, sz, sz,
                                       C.POINTER(C.c_int)]
    L.dropin_olmoe_moe_ffn.restype = i32
    wt, E, EI, NE, K, renorm, bias_std = CONFIGS["olmoe_q8"]
    g = golden("moe_olmoe_q8.npz")
    T = int(g["T"])
    lw = layer("olmoe_q8")
    x = hipmoe.synth_input(SEED, 0, T, E)
    assert sha(x) == str(g["sha_x"]) and sha(lw["gate"]) == str(g["sha_gate"])
    out = np.empty((T, E), np.float32)
    up = C.c_int(-1)
    on_gpu = L.dropin_olmoe_moe_ffn(x.ctypes.data, out.ctypes.data, T,
                                    lw["router"].ctypes.data, lw["gate"].ctypes.data,
                                    lw["up"].ctypes.data, lw["down"].ctypes.data, wt, E, EI,
                                    NE, K, C.byref(up))
    bitwise = bool(np.array_equal(out.view(np.uint32), g["out"].view(np.uint32)))
    print(json.dumps({"on_gpu": on_gpu, "uploaded": up.value, "bitwise": bitwise,
                      "rel_l2": rel_l2(out, g["out"]),
                      "error": hipmoe.last_error()}), flush=True)


def run_child():
    if not os.path.exists(LIB):
        pytest.skip("oracle/_ref/libdropin_olmoe.so not built (no reference tree here)")
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "child"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_dropin_without_gpu_runs_reference_cpu_body():
    import hipmoe
    if hipmoe.hip().device_count() > 0:
        pytest.skip("a GPU is visible: the GPU variant covers this host")
    res = run_child()
    assert res["uploaded"] == 0 and "no HIP device" in res["error"]
    assert res["on_gpu"] == 0
    assert res["bitwise"], res


@pytest.mark.gpu
def test_gpu_dropin_runs_layer_on_gpu():
    res = run_child()
    assert res["uploaded"] == 1 and res["on_gpu"] == 1, res
    assert res["rel_l2"] <= 2e-5, res


if __name__ == "__main__" and sys.argv[1:] == ["child"]:
    child()
