"""ctypes binding of libhip_moe.so (include/hip_moe.h, include/moe_synth.h).

The library is the product: HIP kernels for gfx950 behind a C ABI.  This module
only marshals numpy arrays and device pointers; it never computes a result on
the CPU.  If the library is missing it raises instead of falling back.

Device memory and events come from the HIP runtime (libamdhip64) through
ctypes as well, so nothing here needs torch.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhip_moe.so")

Q8_0 = 1
Q4_0 = 2
Q4_K = 3
Q6_K = 5
# execution paths (include/hip_moe.h)
PATH_AUTO, PATH_DECODE, PATH_GEMV, PATH_GROUPED = 0, 1, 2, 3
QK = 32

_lib = None
_hip = None


class HipMoeError(RuntimeError):
    pass


def row_bytes(wtype: int, n: int) -> int:
    if wtype in (Q4_K, Q6_K):
        return (n // 256) * (144 if wtype == Q4_K else 210)
    return (n // QK) * (34 if wtype == Q8_0 else 18)


def lib():
    """Load libhip_moe.so (built by __graft_entry__.build() / make -C llm.c_amd)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipMoeError(f"{LIB_PATH} is not built; run `make -C llm.c_amd` first")
    L = C.CDLL(LIB_PATH)
    vp, sz, i32, f32p, u32p = C.c_void_p, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p
    L.hip_moe_upload.restype = vp
    L.hip_moe_upload.argtypes = [vp, vp, vp, vp, i32, sz, sz, sz, sz, i32]
    L.hip_moe_upload_typed.restype = vp
    L.hip_moe_upload_typed.argtypes = [vp, vp, vp, vp, i32, i32, sz, sz, sz, sz, i32]
    L.hip_moe_ffn.restype = i32
    L.hip_moe_ffn.argtypes = [vp, f32p, f32p, sz, f32p, u32p, f32p]
    L.hip_moe_ffn_dev.restype = i32
    L.hip_moe_ffn_dev.argtypes = [vp, vp, vp, sz, vp, vp, vp, vp]
    L.hip_moe_ffn_dev_noalloc.restype = i32
    L.hip_moe_ffn_dev_noalloc.argtypes = [vp, vp, vp, sz, vp, vp, vp, vp]
    L.hip_moe_reserve.restype = i32
    L.hip_moe_reserve.argtypes = [vp, sz]
    L.hip_moe_status.restype = i32
    L.hip_moe_status.argtypes = [vp, vp]
    L.hip_moe_set_wait_limit.restype = i32
    L.hip_moe_set_wait_limit.argtypes = [vp, i32]
    L.hip_moe_route_dev.restype = i32
    L.hip_moe_route_dev.argtypes = [vp, vp, sz, vp, vp, vp, vp, vp, vp]
    L.hip_moe_expert_ffn_dev.restype = i32
    L.hip_moe_expert_ffn_dev.argtypes = [vp, sz, vp, vp, vp]
    L.hip_moe_free.restype = None
    L.hip_moe_free.argtypes = [vp]
    L.hip_moe_weight_bytes.restype = sz
    L.hip_moe_weight_bytes.argtypes = [vp]
    L.hip_moe_last_error.restype = C.c_char_p
    L.hip_moe_last_error.argtypes = []
    L.hip_moe_expf_dev.restype = i32
    L.hip_moe_expf_dev.argtypes = [vp, vp, sz, vp]
    L.hip_moe_copy_dev.restype = i32
    L.hip_moe_set_path.restype = i32
    L.hip_moe_set_path.argtypes = [vp, i32]
    L.hip_moe_path_for.restype = i32
    L.hip_moe_path_for.argtypes = [vp, sz]
    L.hip_moe_copy_dev.argtypes = [vp, vp, sz, vp]
    L.hip_moe_qmat_upload.restype = vp
    L.hip_moe_qmat_upload.argtypes = [vp, i32, sz, sz]
    L.hip_moe_qmat_mul.restype = i32
    L.hip_moe_qmat_mul.argtypes = [vp, f32p, sz, f32p, sz, f32p]
    L.hip_moe_qmat_mul_dev.restype = i32
    L.hip_moe_qmat_mul_dev.argtypes = [vp, vp, sz, vp, sz, vp, vp]
    L.hip_moe_qmat_bytes.restype = sz
    L.hip_moe_qmat_bytes.argtypes = [vp]
    L.hip_moe_qmat_free.restype = None
    L.hip_moe_qmat_free.argtypes = [vp]
    L.hip_moe_quantize_q8k_dev.restype = i32
    L.hip_moe_quantize_q8k_dev.argtypes = [vp, sz, sz, vp, vp, vp, vp]
    # synthetic inputs
    L.moe_row_bytes.restype = sz
    L.moe_row_bytes.argtypes = [i32, sz]
    L.moe_synth_normal.restype = None
    L.moe_synth_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_float, vp, sz, i32]
    L.moe_quantize_q8_0.restype = None
    L.moe_quantize_q8_0.argtypes = [vp, vp, sz]
    L.moe_quantize_q4_0.restype = None
    L.moe_quantize_q4_0.argtypes = [vp, vp, sz]
    L.moe_synth_quant_matrix.restype = None
    L.moe_synth_quant_matrix.argtypes = [C.c_uint64, C.c_uint64, C.c_float, i32, sz, sz, vp, i32]
    for n in ("router", "bias"):
        f = getattr(L, f"moe_stream_{n}")
        f.restype, f.argtypes = C.c_uint64, [C.c_uint64]
    for n in ("gate", "up", "down"):
        f = getattr(L, f"moe_stream_{n}")
        f.restype, f.argtypes = C.c_uint64, [C.c_uint64, C.c_uint64]
    L.moe_stream_input.restype, L.moe_stream_input.argtypes = C.c_uint64, [C.c_uint64]
    L.moe_f32_to_f16_rne.restype, L.moe_f32_to_f16_rne.argtypes = C.c_uint16, [C.c_float]
    L.moe_f16_to_f32.restype, L.moe_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
    _lib = L
    return L


def last_error() -> str:
    return lib().hip_moe_last_error().decode(errors="replace")


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI must be C-contiguous"
    return a.ctypes.data


def _threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


# --------------------------------------------------------------------------
# synthetic inputs (moe_synth.h)
# --------------------------------------------------------------------------

def synth_normal(seed: int, stream: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().moe_synth_normal(seed, stream, mean, std, _ptr(out), n, _threads())
    return out


def quantize(x: np.ndarray, wtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(row_bytes(wtype, x.size), np.uint8)
    f = lib().moe_quantize_q8_0 if wtype == Q8_0 else lib().moe_quantize_q4_0
    f(_ptr(x), _ptr(out), x.size)
    return out


def synth_quant_matrix(seed, stream, std, wtype, rows, cols) -> np.ndarray:
    out = np.empty(rows * row_bytes(wtype, cols), np.uint8)
    lib().moe_synth_quant_matrix(seed, stream, std, wtype, rows, cols, _ptr(out), _threads())
    return out


def wtypes(wtype: int):
    """(gate/up type, down type) of a layer's wtype: the gate/up type,
    or'ed with the down type << 8 where that differs (a Q4_K_M file's
    Q4_K gate/up with Q6_K down: Q4_K | Q6_K << 8)."""
    gt = wtype & 0xff
    return gt, (wtype >> 8) or gt


def synth_layer(seed: int, layer: int, wtype: int, E: int, EI: int, NE: int,
                std: float = 0.02, bias_std: float | None = None) -> dict:
    """One MoE layer of the given shape: router fp32 N(0, std) [NE][E],
    optional router bias N(0, bias_std) [NE], stacked expert tensors
    gate/up [NE][EI][E/32 blocks] and down [NE][E][EI/32 blocks] as uint8
    arrays of shape [NE, bytes_per_expert] (GGUF *_exps layout).  wtype may
    carry a down type (wtypes)."""
    L = lib()
    router = synth_normal(seed, L.moe_stream_router(layer), NE * E, 0.0, std).reshape(NE, E)
    bias = None
    if bias_std is not None:
        bias = synth_normal(seed, L.moe_stream_bias(layer), NE, 0.0, bias_std)
    gt, dt = wtypes(wtype)
    gu = EI * row_bytes(gt, E)
    dn = E * row_bytes(dt, EI)
    gate = np.empty((NE, gu), np.uint8)
    up = np.empty((NE, gu), np.uint8)
    down = np.empty((NE, dn), np.uint8)
    nt = _threads()
    for e in range(NE):
        L.moe_synth_quant_matrix(seed, L.moe_stream_gate(layer, e), std, gt, EI, E,
                                 _ptr(gate[e]), nt)
        L.moe_synth_quant_matrix(seed, L.moe_stream_up(layer, e), std, gt, EI, E,
                                 _ptr(up[e]), nt)
        L.moe_synth_quant_matrix(seed, L.moe_stream_down(layer, e), std, dt, E, EI,
                                 _ptr(down[e]), nt)
    return dict(router=router, bias=bias, gate=gate, up=up, down=down, wtype=wtype,
                E=E, EI=EI, NE=NE)


def synth_input(seed: int, call: int, T: int, E: int) -> np.ndarray:
    return synth_normal(seed, lib().moe_stream_input(call), T * E, 0.0, 1.0).reshape(T, E)


def expert_ptrs(stacked: np.ndarray):
    """Per-expert base pointers into a stacked [NE, bytes] array: the views
    tensor_at_q (olmoe.c:20-60) forms."""
    arr = (C.c_void_p * stacked.shape[0])()
    for e in range(stacked.shape[0]):
        arr[e] = stacked[e].ctypes.data
    return arr


# --------------------------------------------------------------------------
# HIP runtime plumbing (device memory, streams, events, graphs)
# --------------------------------------------------------------------------

class Hip:
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        lib()  # libamdhip64 is a dependency of libhip_moe.so
        path = None
        for cand in ("libamdhip64.so",
                     os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so")):
            try:
                self.h = C.CDLL(cand)
                path = cand
                break
            except OSError:
                continue
        if path is None:
            raise HipMoeError("libamdhip64.so not found")
        h = self.h
        vp, sz = C.c_void_p, C.c_size_t
        h.hipMalloc.argtypes = [C.POINTER(vp), sz]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, sz, C.c_int]
        h.hipMemcpyAsync.argtypes = [vp, vp, sz, C.c_int, vp]
        h.hipMemsetAsync.argtypes = [vp, C.c_int, sz, vp]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [C.POINTER(vp)]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipEventCreate.argtypes = [C.POINTER(vp)]
        h.hipEventDestroy.argtypes = [vp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        h.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [C.c_int]
        h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, sz]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]

    def check(self, rc, what):
        if rc != 0:
            raise HipMoeError(f"{what}: {self.h.hipGetErrorString(rc).decode()}")

    def device_count(self) -> int:
        n = C.c_int(0)
        rc = self.h.hipGetDeviceCount(C.byref(n))
        return n.value if rc == 0 else 0

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self.check(self.h.hipMalloc(C.byref(p), max(1, nbytes)), "hipMalloc")
        return p.value

    def free(self, p: int):
        if p:
            self.h.hipFree(C.c_void_p(p))

    def upload(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = self.malloc(a.nbytes)
        self.check(self.h.hipMemcpy(p, _ptr(a), a.nbytes, self.H2D), "hipMemcpy H2D")
        return p

    def copy_in(self, p: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self.check(self.h.hipMemcpy(p, _ptr(a), a.nbytes, self.H2D), "hipMemcpy H2D")

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.check(self.h.hipMemcpy(_ptr(out), p, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def sync(self):
        self.check(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self) -> int:
        s = C.c_void_p()
        self.check(self.h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s: int):
        self.check(self.h.hipStreamSynchronize(s), "hipStreamSynchronize")

    def event(self) -> int:
        e = C.c_void_p()
        self.check(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def record(self, e: int, s: int):
        self.check(self.h.hipEventRecord(e, s), "hipEventRecord")

    def elapsed_ms(self, e0: int, e1: int) -> float:
        self.check(self.h.hipEventSynchronize(e1), "hipEventSynchronize")
        ms = C.c_float()
        self.check(self.h.hipEventElapsedTime(C.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def begin_capture(self, s: int):
        self.check(self.h.hipStreamBeginCapture(s, 0), "hipStreamBeginCapture")

    def end_capture(self, s: int) -> int:
        g = C.c_void_p()
        self.check(self.h.hipStreamEndCapture(s, C.byref(g)), "hipStreamEndCapture")
        ge = C.c_void_p()
        self.check(self.h.hipGraphInstantiate(C.byref(ge), g, None, None, 0),
                   "hipGraphInstantiate")
        self.h.hipGraphDestroy(g)
        return ge.value

    def graph_launch(self, ge: int, s: int):
        self.check(self.h.hipGraphLaunch(ge, s), "hipGraphLaunch")


_hip_singleton = None


def hip() -> Hip:
    global _hip_singleton
    if _hip_singleton is None:
        _hip_singleton = Hip()
    return _hip_singleton


# --------------------------------------------------------------------------
# layer object
# --------------------------------------------------------------------------

class MoeLayer:
    """One uploaded MoE layer (hip_moe_upload)."""

    def __init__(self, router, gate, up, down, wtype, E, EI, NE, topk, renorm):
        L = lib()
        self.router = np.ascontiguousarray(router, np.float32)
        self.E, self.EI, self.NE, self.topk = E, EI, NE, topk
        self.wtype, self.renorm = wtype, renorm
        gp, upp, dp = expert_ptrs(gate), expert_ptrs(up), expert_ptrs(down)
        gt, dt = wtypes(wtype)
        if gt == dt:
            self.h = L.hip_moe_upload(_ptr(self.router), gp, upp, dp, wtype, E, EI, NE, topk,
                                      int(renorm))
        else:
            self.h = L.hip_moe_upload_typed(_ptr(self.router), gp, upp, dp, gt, dt, E, EI, NE,
                                            topk, int(renorm))
        if not self.h:
            raise HipMoeError("hip_moe_upload: " + last_error())

    @classmethod
    def from_synth(cls, layer: dict, topk: int, renorm: bool):
        return cls(layer["router"], layer["gate"], layer["up"], layer["down"], layer["wtype"],
                   layer["E"], layer["EI"], layer["NE"], topk, renorm)

    def ffn(self, x: np.ndarray, bias: np.ndarray | None = None):
        """Host-pointer entry point: returns (out [T][E], ids [T][k], w [T][k])."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.E)
        T = x.shape[0]
        out = np.empty((T, self.E), np.float32)
        ids = np.empty((T, self.topk), np.uint32)
        w = np.empty((T, self.topk), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        rc = lib().hip_moe_ffn(self.h, _ptr(x), _ptr(out), T, None if b is None else _ptr(b),
                               _ptr(ids), _ptr(w))
        if rc != 1:
            raise HipMoeError("hip_moe_ffn: " + last_error())
        return out, ids, w

    def ffn_dev(self, d_x, d_out, T, d_bias=None, d_ids=None, d_w=None, stream=None):
        rc = lib().hip_moe_ffn_dev(self.h, d_x, d_out, T, d_bias, d_ids, d_w, stream)
        if rc != 1:
            raise HipMoeError("hip_moe_ffn_dev: " + last_error())

    def ffn_dev_noalloc(self, d_x, d_out, T, d_bias=None, d_ids=None, d_w=None, stream=None):
        """hip_moe_ffn_dev_noalloc: the decode path on the GPU's static scratch."""
        rc = lib().hip_moe_ffn_dev_noalloc(self.h, d_x, d_out, T, d_bias, d_ids, d_w, stream)
        if rc != 1:
            raise HipMoeError("hip_moe_ffn_dev_noalloc: " + last_error())

    def reserve(self, T: int):
        """Size the scratch for calls of up to T tokens (before a graph capture)."""
        if lib().hip_moe_reserve(self.h, T) != 1:
            raise HipMoeError("hip_moe_reserve: " + last_error())

    def status(self, stream=None) -> int:
        """0, or the code of a decode-kernel wait that ran out (the layer is reset)."""
        return lib().hip_moe_status(self.h, stream)

    def set_wait_limit(self, polls: int):
        if lib().hip_moe_set_wait_limit(self.h, polls) != 1:
            raise HipMoeError("hip_moe_set_wait_limit: " + last_error())

    def route(self, x: np.ndarray, bias: np.ndarray | None = None):
        """Routing stage through hip_moe_route_dev: (logits, probs, ids, w)."""
        H = hip()
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.E)
        T = x.shape[0]
        d_x = H.upload(x)
        d_b = H.upload(np.ascontiguousarray(bias, np.float32)) if bias is not None else 0
        d_lg = H.malloc(T * self.NE * 4)
        d_pr = H.malloc(T * self.NE * 4)
        d_ids = H.malloc(T * self.topk * 4)
        d_w = H.malloc(T * self.topk * 4)
        try:
            rc = lib().hip_moe_route_dev(self.h, d_x, T, d_b or None, d_lg, d_pr, d_ids, d_w,
                                         None)
            if rc != 1:
                raise HipMoeError("hip_moe_route_dev: " + last_error())
            H.sync()
            return (H.download(d_lg, (T, self.NE), np.float32),
                    H.download(d_pr, (T, self.NE), np.float32),
                    H.download(d_ids, (T, self.topk), np.uint32),
                    H.download(d_w, (T, self.topk), np.float32))
        finally:
            for p in (d_x, d_b, d_lg, d_pr, d_ids, d_w):
                H.free(p)

    def expert_ffn(self, expert: int, x: np.ndarray) -> np.ndarray:
        H = hip()
        x = np.ascontiguousarray(x, np.float32).reshape(self.E)
        d_x = H.upload(x)
        d_o = H.malloc(self.E * 4)
        try:
            rc = lib().hip_moe_expert_ffn_dev(self.h, expert, d_x, d_o, None)
            if rc != 1:
                raise HipMoeError("hip_moe_expert_ffn_dev: " + last_error())
            H.sync()
            return H.download(d_o, (self.E,), np.float32)
        finally:
            H.free(d_x)
            H.free(d_o)

    def weight_bytes(self) -> int:
        return lib().hip_moe_weight_bytes(self.h)

    def set_path(self, path: int):
        """Force PATH_DECODE / PATH_GEMV / PATH_GROUPED (PATH_AUTO restores)."""
        if lib().hip_moe_set_path(self.h, path) != 1:
            raise HipMoeError("hip_moe_set_path: " + last_error())

    def path_for(self, T: int) -> int:
        return lib().hip_moe_path_for(self.h, T)

    def free(self):
        if self.h:
            lib().hip_moe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class QMat:
    """One uploaded Q8_0/Q4_0/Q4_K/Q6_K matrix of N rows of K columns
    (hip_moe_qmat_upload)."""

    def __init__(self, q: np.ndarray, wtype: int, N: int, K: int):
        self.q = np.ascontiguousarray(q, np.uint8)
        if self.q.size != N * row_bytes(wtype, K):
            raise ValueError("qmat: block bytes do not match N x K")
        self.wtype, self.N, self.K = wtype, N, K
        self.h = lib().hip_moe_qmat_upload(_ptr(self.q), wtype, N, K)
        if not self.h:
            raise HipMoeError("hip_moe_qmat_upload: " + last_error())

    def mul(self, x: np.ndarray, add: np.ndarray | None = None) -> np.ndarray:
        """Host-pointer entry point: add + x[T][K] . W^T, add None, [N] or [T][N]."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.K)
        T = x.shape[0]
        out = np.empty((T, self.N), np.float32)
        a = None if add is None else np.ascontiguousarray(add, np.float32).ravel()
        rc = lib().hip_moe_qmat_mul(self.h, _ptr(x), T, None if a is None else _ptr(a),
                                    0 if a is None else a.size, _ptr(out))
        if rc != 1:
            raise HipMoeError("hip_moe_qmat_mul: " + last_error())
        return out

    def mul_dev(self, d_x, T, d_out, d_add=None, add_len=0, stream=None):
        rc = lib().hip_moe_qmat_mul_dev(self.h, d_x, T, d_add, add_len, d_out, stream)
        if rc != 1:
            raise HipMoeError("hip_moe_qmat_mul_dev: " + last_error())

    def bytes(self) -> int:
        return lib().hip_moe_qmat_bytes(self.h)

    def free(self):
        if self.h:
            lib().hip_moe_qmat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def quantize_q8k_dev(x: np.ndarray):
    """quantize_row_q8 of each row of x[T][K] on the GPU
    (hip_moe_quantize_q8k_dev): (d[T][K/256], qs[T][K], bsums[T][K/256][16])."""
    H = hip()
    x = np.ascontiguousarray(x, np.float32)
    T, K = x.reshape(-1, x.shape[-1]).shape
    nb = K // 256
    d_x = H.upload(x)
    d_d, d_q, d_b = H.malloc(T * nb * 4), H.malloc(T * K), H.malloc(T * nb * 32)
    try:
        if lib().hip_moe_quantize_q8k_dev(d_x, T, K, d_d, d_q, d_b, None) != 1:
            raise HipMoeError("hip_moe_quantize_q8k_dev: " + last_error())
        H.sync()
        return (H.download(d_d, (T, nb), np.float32), H.download(d_q, (T, K), np.int8),
                H.download(d_b, (T, nb, 16), np.int16))
    finally:
        for q in (d_x, d_d, d_q, d_b):
            H.free(q)


def expf_dev(x: np.ndarray) -> np.ndarray:
    H = hip()
    x = np.ascontiguousarray(x, np.float32)
    d_i = H.upload(x)
    d_o = H.malloc(x.nbytes)
    try:
        if lib().hip_moe_expf_dev(d_i, d_o, x.size, None) != 1:
            raise HipMoeError("hip_moe_expf_dev: " + last_error())
        H.sync()
        return H.download(d_o, x.shape, np.float32)
    finally:
        H.free(d_i)
        H.free(d_o)
