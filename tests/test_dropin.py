"""The drop-in itself: INTEGRATION.md's lines for OLMoE (the upload loop of
olmoe_load, the early return of moe_ffn, the free loop of olmoe_close)
compiled around the reference's own models/olmoe/olmoe.c and linked against
libhip_moe.so (tests/native/dropin_olmoe.c, built by oracle/ref/build_ref.sh
from the reference tree; skipped where that tree was not there to build it).

  * no GPU: hip_moe_upload_typed returns NULL and the reference's CPU body
    runs, giving the golden layer output bit for bit (a Q8_0 layer,
    tests/golden/moe_olmoe_q8.npz, and a Q4_K gate/up + Q6_K down layer,
    tests/golden/kquant_moe.npz);
  * with a GPU: the layer runs on it, within the output bar of the golden
    (Q8_0) or bit for bit (the K-quant layer).

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


def child(case):
    sys.path[:0] = [os.path.join(REPO, "llm.c_amd"), HERE]
    import hipmoe
    from common import CONFIGS, SEED, golden, layer, rel_l2, sha
    L = C.CDLL(LIB)
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    L.dropin_olmoe_moe_ffn.argtypes = [vp, vp, sz, vp, vp, vp, vp, i32, sz, sz, sz, sz,
                                       C.POINTER(C.c_int)]
    L.dropin_olmoe_moe_ffn.restype = i32
    if case == "olmoe_q8":
        wt, E, EI, NE, K, renorm, bias_std = CONFIGS["olmoe_q8"]
        g = golden("moe_olmoe_q8.npz")
        T, expect = int(g["T"]), g["out"]
        lw = layer("olmoe_q8")
        x = hipmoe.synth_input(SEED, 0, T, E)
        assert sha(x) == str(g["sha_x"]) and sha(lw["gate"]) == str(g["sha_gate"])
    else:
        # the K-quant layer of kquant_moe.npz: Q4_K gate/up, Q6_K down; the
        # library's type numbers are the reference's TENSOR_* values
        wt, E, EI, NE, K, renorm, T = (hipmoe.Q4_K | hipmoe.Q6_K << 8, 2048, 1024, 64, 8, 0, 4)
        g = golden("kquant_moe.npz")
        expect = g[f"{case}_out"]
        lw = hipmoe.synth_layer(SEED, 0, wt, E, EI, NE, 0.02, None)
        x = hipmoe.synth_input(SEED, 0, T, E)
        assert sha(x) == str(g[f"{case}_sha_x"]) and sha(lw["gate"]) == str(g[f"{case}_sha_gate"])
        assert sha(lw["down"]) == str(g[f"{case}_sha_down"])
    out = np.empty((T, E), np.float32)
    up = C.c_int(-1)
    on_gpu = L.dropin_olmoe_moe_ffn(x.ctypes.data, out.ctypes.data, T,
                                    lw["router"].ctypes.data, lw["gate"].ctypes.data,
                                    lw["up"].ctypes.data, lw["down"].ctypes.data, wt, E, EI,
                                    NE, K, C.byref(up))
    bitwise = bool(np.array_equal(out.view(np.uint32), expect.view(np.uint32)))
    print(json.dumps({"on_gpu": on_gpu, "uploaded": up.value, "bitwise": bitwise,
                      "rel_l2": rel_l2(out, expect),
                      "error": hipmoe.last_error()}), flush=True)


CASES = ["olmoe_q8", "olmoe_q4k_q6k"]


def run_child(case):
    if not os.path.exists(LIB):
        pytest.skip("oracle/_ref/libdropin_olmoe.so not built (no reference tree here)")
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "child", case],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("case", CASES)
def test_dropin_without_gpu_runs_reference_cpu_body(case):
    import hipmoe
    if hipmoe.hip().device_count() > 0:
        pytest.skip("a GPU is visible: the GPU variant covers this host")
    res = run_child(case)
    assert res["uploaded"] == 0 and "no HIP device" in res["error"]
    assert res["on_gpu"] == 0
    assert res["bitwise"], res


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
def test_gpu_dropin_runs_layer_on_gpu(case):
    res = run_child(case)
    assert res["uploaded"] == 1 and res["on_gpu"] == 1, res
    if case == "olmoe_q8":
        assert res["rel_l2"] <= 2e-5, res
    else:
        assert res["bitwise"], res   # the K-quant layer equals the reference bit for bit


if __name__ == "__main__" and sys.argv[1:2] == ["child"]:
    child(sys.argv[2])
