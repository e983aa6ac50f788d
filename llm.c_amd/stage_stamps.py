"""Where a one-token MoE layer call's time goes: the decode kernel's stage
stamps (libhip_moe_stamps.so, built by `make -C llm.c_amd stamps`), per
workgroup, for the last of `calls` back-to-back calls that rotate over
`copies` uploads of the layer and 8 tokens, as min / median / max over the
workgroups of the time since the first workgroup started.

    python llm.c_amd/stage_stamps.py [olmoe_q8|mixtral_q4] [calls] [copies]
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import hipmoe  # noqa: E402

SHAPES = {  # wtype, d_model, d_ff, experts, top-k, renorm
    "olmoe_q8": (hipmoe.Q8_0, 2048, 1024, 64, 8, False),
    "mixtral_q4": (hipmoe.Q4_0, 4096, 14336, 8, 2, True),
}
STAGES = ["start", "routed", "last gate/up done", "partials stored", "combined"]
WGS, NST = 1024, len(STAGES)


def main():
    shape = sys.argv[1] if len(sys.argv) > 1 else "olmoe_q8"
    calls = int(sys.argv[2]) if len(sys.argv) > 2 else 64
    copies = int(sys.argv[3]) if len(sys.argv) > 3 else 4
    hipmoe.LIB_PATH = os.path.join(HERE, "libhip_moe_stamps.so")
    wt, E, EI, NE, K, renorm = SHAPES[shape]
    lw = hipmoe.synth_layer(1337, 0, wt, E, EI, NE, 0.02, None)
    layers = [hipmoe.MoeLayer.from_synth(lw, K, renorm) for _ in range(copies)]
    H = hipmoe.hip()
    xs = [H.upload(hipmoe.synth_input(1337, 100 + i, 1, E)) for i in range(8)]
    d_out = H.malloc(E * 4)
    s = H.stream()
    for i in range(calls):
        layers[i % copies].ffn_dev(xs[i % 8], d_out, 1, None, None, None, s)
    H.stream_sync(s)
    st = np.zeros(WGS * NST, np.uint64)
    L = hipmoe.lib()
    L.moe_stage_stamps.argtypes = [C.c_void_p]
    H.check(L.moe_stage_stamps(st.ctypes.data), "moe_stage_stamps")
    t = st.reshape(WGS, NST).astype(np.int64)
    t = t[t[:, 0] > 0]
    t0 = t[:, 0].min()
    print(f"{shape}: last of {calls} calls over {copies} layer copies, {t.shape[0]} workgroups "
          "(us since the first workgroup's start: min / median / max)")
    for k, name in enumerate(STAGES):
        v = (t[:, k][t[:, k] > 0] - t0) / 100.0
        if v.size:
            print(f"  {name:20s} {v.min():7.2f} {np.median(v):7.2f} {v.max():7.2f}")
    for x in xs:
        H.free(x)
    H.free(d_out)
    for lay in layers:
        lay.free()


if __name__ == "__main__":
    main()
