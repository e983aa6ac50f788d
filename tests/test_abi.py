"""C-ABI checks that need no GPU: the library loads, exports every entry
point its headers declare, and refuses what it cannot do with the
reference's "return 0 / NULL, caller falls back" convention (nn.h:33-39)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import hipmoe
from common import REPO


def declared_functions(header: str):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", text)
    return sorted({n for n in names if n.startswith(("hip_moe_", "moe_", "hip_lm_"))})


@pytest.mark.parametrize("header", ["hip_moe.h", "moe_synth.h", "hip_lm.h"])
def test_library_exports_every_declared_symbol(header):
    L = hipmoe.lib()
    names = declared_functions(header)
    assert len(names) >= 5
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def _tiny_layer(wtype=hipmoe.Q8_0, E=256, EI=256, NE=4):
    rb_in, rb_mid = hipmoe.row_bytes(wtype, E), hipmoe.row_bytes(wtype, EI)
    router = np.zeros((NE, E), np.float32)
    gate = np.zeros((NE, EI * rb_in), np.uint8)
    down = np.zeros((NE, E * rb_mid), np.uint8)
    return router, gate, gate.copy(), down


def _upload(router, gate, up, down, wtype, E, EI, NE, topk, renorm=0):
    L = hipmoe.lib()
    return L.hip_moe_upload(router.ctypes.data, hipmoe.expert_ptrs(gate),
                            hipmoe.expert_ptrs(up), hipmoe.expert_ptrs(down), wtype, E, EI,
                            NE, topk, renorm)


@pytest.mark.parametrize("wtype,E,EI,NE,topk,msg", [
    (4, 256, 256, 4, 2, "unsupported weight type"),
    (0, 256, 256, 4, 2, "unsupported weight type"),
    (3, 16384, 256, 4, 2, "not supported for K-quant experts"),
    (1, 250, 256, 4, 2, "multiples of 256"),
    (1, 256, 300, 4, 2, "multiples of 256"),
    (1, 768, 256, 4, 2, "not supported"),
    (1, 256, 256, 4, 5, "out of range"),
    (1, 256, 256, 300, 2, "out of range"),
])
def test_upload_rejects_unsupported(wtype, E, EI, NE, topk, msg):
    router, gate, up, down = _tiny_layer(1 if wtype not in (1, 2) else wtype, 256, 256, 4)
    h = _upload(router, gate, up, down, wtype, E, EI, NE, topk)
    assert not h
    assert msg in hipmoe.last_error()


@pytest.mark.parametrize("gt,dt,msg", [
    (1, 3, "unsupported weight types"),   # Q8_0 gate/up with a K-quant down
    (3, 1, "unsupported weight types"),
    (1, 2, "unsupported weight types"),   # Q8_0 / Q4_0 take one type
    (3, 5, "no HIP device"),              # a Q4_K_M mix passes the checks
])
def test_upload_typed_checks_the_mix(gt, dt, msg):
    if msg == "no HIP device" and hipmoe.hip().device_count() > 0:
        pytest.skip("a GPU is visible: the GPU tests upload this mix")
    L = hipmoe.lib()
    router, gate, up, down = _tiny_layer(hipmoe.Q8_0, 256, 256, 4)
    h = L.hip_moe_upload_typed(router.ctypes.data, hipmoe.expert_ptrs(gate),
                               hipmoe.expert_ptrs(up), hipmoe.expert_ptrs(down), gt, dt, 256,
                               256, 4, 2, 0)
    assert not h
    assert msg in hipmoe.last_error()


def test_calls_on_null_layer_return_zero():
    L = hipmoe.lib()
    x = np.zeros(256, np.float32)
    assert L.hip_moe_ffn(None, x.ctypes.data, x.ctypes.data, 1, None, None, None) == 0
    assert L.hip_moe_ffn_dev(None, 1, 1, 1, None, None, None, None) == 0
    assert L.hip_moe_route_dev(None, 1, 1, None, None, None, 1, 1, None) == 0
    assert L.hip_moe_expert_ffn_dev(None, 0, 1, 1, None) == 0
    L.hip_moe_free(None)
    assert L.hip_moe_weight_bytes(None) == 0
    assert L.hip_moe_reserve(None, 1) == 0
    assert L.hip_moe_status(None, None) == -1
    assert L.hip_moe_set_wait_limit(None, 1) == 0


def test_upload_without_device_returns_null():
    if hipmoe.hip().device_count() > 0:
        pytest.skip("a GPU is visible")
    router, gate, up, down = _tiny_layer()
    assert not _upload(router, gate, up, down, 1, 256, 256, 4, 2)
    assert "no HIP device" in hipmoe.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(hipmoe, "_lib", None)
    monkeypatch.setattr(hipmoe, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(hipmoe.HipMoeError):
        hipmoe.lib()


def test_oracle_library_is_separate_from_product():
    """The product library links nothing from oracle/."""
    import subprocess
    out = subprocess.run(["ldd", hipmoe.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out
    syms = subprocess.run(["nm", "-D", hipmoe.LIB_PATH], capture_output=True, text=True).stdout
    assert "orc_" not in syms and "ref_" not in syms


@pytest.mark.parametrize("wtype,N,K,msg", [
    (4, 64, 2048, "unsupported weight type"),
    (0, 64, 2048, "unsupported weight type"),
    (3, 64, 2000, "not supported for K-quants"),
    (5, 64, 65536, "not supported for K-quants"),
    (5, 0, 2048, "not supported for K-quants"),
    (1, 64, 14336, "not supported"),
    (1, 64, 768, "not supported"),
    (2, 64, 128, "not supported"),
    (1, 0, 2048, "not supported"),
])
def test_qmat_upload_rejects_unsupported(wtype, N, K, msg):
    q = np.zeros(max(1, N) * hipmoe.row_bytes(1, max(K, 256)), np.uint8)
    assert not hipmoe.lib().hip_moe_qmat_upload(q.ctypes.data, wtype, N, K)
    assert msg in hipmoe.last_error()


def test_qmat_calls_on_null_return_zero():
    L = hipmoe.lib()
    x = np.zeros(256, np.float32)
    assert L.hip_moe_qmat_mul(None, x.ctypes.data, 1, None, 0, x.ctypes.data) == 0
    assert L.hip_moe_qmat_mul_dev(None, 1, 1, None, 0, 1, None) == 0
    assert L.hip_moe_qmat_bytes(None) == 0
    L.hip_moe_qmat_free(None)
    assert L.hip_moe_quantize_q8k_dev(None, 1, 256, None, None, None, None) == 0
    assert "NULL" in hipmoe.last_error()
    assert L.hip_moe_quantize_q8k_dev(16, 1, 200, 16, 16, 16, None) == 0
    assert "multiple of 256" in hipmoe.last_error()


def test_lm_calls_on_null_return_zero():
    import hiplm
    L = hiplm._bind()
    assert not L.hip_lm_upload(None)
    assert "NULL descriptor" in hipmoe.last_error()
    assert L.hip_lm_decode(None, 0, None, None) == 0
    assert L.hip_lm_generate(None, None, 0, 0, None, None) == 0
    assert L.hip_lm_trace(None, None, None, None) == 0
    assert L.hip_lm_reset(None) == 0
    assert L.hip_lm_weight_bytes(None) == 0
    L.hip_lm_free(None)
    assert not L.hip_lm_batch_new(None, 4)
    assert "NULL model" in hipmoe.last_error()
    assert L.hip_lm_batch_decode(None, None, None, None) == 0
    assert L.hip_lm_batch_generate(None, None, 0, 0, None, None) == 0
    assert L.hip_lm_batch_reset(None) == 0
    L.hip_lm_batch_free(None)


def test_lm_upload_rejects_bad_descriptors():
    import hiplm
    L = hiplm._bind()
    d = hiplm.Desc()
    d.arch = 7
    assert not L.hip_lm_upload(C.byref(d))
    assert "unknown arch" in hipmoe.last_error()
    d.arch, d.wtype = hiplm.ARCH_OLMOE, 1
    d.layers, d.E, d.heads, d.kv_heads, d.vocab, d.context = 2, 1024, 4, 4, 10, 8
    assert not L.hip_lm_upload(C.byref(d))
    assert "heads * 128 == E" in hipmoe.last_error()
    d.heads = d.kv_heads = 8
    assert not L.hip_lm_upload(C.byref(d))
    assert "NULL tensor pointer" in hipmoe.last_error()
