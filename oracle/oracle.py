"""ctypes binding of the CPU oracle (liboracle.so, moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
Q8_0, Q4_0 = 1, 2

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.orc_router.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        L.orc_router.restype = None
        L.orc_softmax_1d.argtypes = [vp, sz]
        L.orc_softmax_1d.restype = None
        L.orc_top_k.argtypes = [vp, sz, vp, vp, sz]
        L.orc_top_k.restype = None
        L.orc_dot_quant.argtypes = [vp, vp, i32, sz]
        L.orc_dot_quant.restype = C.c_float
        L.orc_qmat_mul.argtypes = [vp, sz, vp, i32, sz, sz, vp, sz, vp]
        L.orc_qmat_mul.restype = None
        L.orc_dequant_row.argtypes = [vp, i32, vp, sz]
        L.orc_dequant_row.restype = None
        L.orc_quantize_q8k.argtypes = [vp, sz, vp, vp, vp]
        L.orc_quantize_q8k.restype = None
        L.orc_dot_q8k.argtypes = [vp, vp, vp, vp, i32, sz]
        L.orc_dot_q8k.restype = C.c_float
        L.orc_fused_ffn.argtypes = [vp, vp, vp, vp, i32, sz, sz, vp, vp]
        L.orc_fused_ffn.restype = None
        L.orc_moe_ffn.argtypes = [vp, vp, sz, vp, vp, vp, vp, vp, i32, sz, sz, sz, sz, i32,
                                  vp, vp, vp, vp, i32]
        L.orc_moe_ffn.restype = None
        L.orc_expf_array.argtypes = [vp, vp, sz]
        L.orc_expf_array.restype = None
        L.orc_expf_bits.argtypes = [C.c_uint32, sz, vp, i32]
        L.orc_expf_bits.restype = None
        L.orc_dot_f32.argtypes = [vp, vp, sz]
        L.orc_dot_f32.restype = C.c_float
        L.orc_olmoe_new.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, i32, vp]
        L.orc_olmoe_new.restype = vp
        L.orc_olmoe_decode.argtypes = [vp, i32, i32, vp, vp, vp, vp, i32]
        L.orc_olmoe_decode.restype = i32
        L.orc_olmoe_run.argtypes = [vp, vp, sz, sz, vp, vp, i32]
        L.orc_olmoe_run.restype = None
        L.orc_olmoe_free.argtypes = [vp]
        L.orc_olmoe_free.restype = None
        L.orc_llama_new.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, sz, i32, vp]
        L.orc_llama_new.restype = vp
        L.orc_olmoe_new_typed.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, vp, vp]
        L.orc_olmoe_new_typed.restype = vp
        L.orc_llama_new_typed.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, sz, vp,
                                          vp]
        L.orc_llama_new_typed.restype = vp
        L.orc_llama_decode.argtypes = [vp, i32, i32, vp, vp, vp, vp, i32]
        L.orc_llama_decode.restype = i32
        L.orc_llama_run.argtypes = [vp, vp, sz, sz, vp, vp, i32]
        L.orc_llama_run.restype = None
        L.orc_llama_free.argtypes = [vp]
        L.orc_llama_free.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _ptrs(stacked):
    arr = (C.c_void_p * stacked.shape[0])()
    for e in range(stacked.shape[0]):
        arr[e] = stacked[e].ctypes.data
    return arr


def threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def router(x, wr, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    wr = np.ascontiguousarray(wr, np.float32)
    T, E = x.shape
    NE = wr.shape[0]
    out = np.empty((T, NE), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_router(_p(x), _p(wr), _p(b), T, E, NE, _p(out))
    return out


def softmax(row):
    r = np.array(row, np.float32, copy=True)
    lib().orc_softmax_1d(_p(r), r.size)
    return r


def top_k(row, k):
    r = np.ascontiguousarray(row, np.float32)
    ids = np.empty(k, np.uint32)
    w = np.empty(k, np.float32)
    lib().orc_top_k(_p(r), r.size, _p(ids), _p(w), k)
    return ids, w


def dot(x, qrow, wtype):
    x = np.ascontiguousarray(x, np.float32)
    q = np.ascontiguousarray(qrow, np.uint8)
    return np.float32(lib().orc_dot_quant(_p(x), _p(q), wtype, x.size))


def quantize_q8k(x):
    """Q8_K blocks of x (quantize_row_q8): (d[n/256], qs[n], bsums[n/256,16])."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    nb = x.size // 256
    d = np.empty(nb, np.float32)
    qs = np.empty(x.size, np.int8)
    bs = np.empty((nb, 16), np.int16)
    lib().orc_quantize_q8k(_p(x), x.size, _p(d), _p(qs), _p(bs))
    return d, qs, bs


def dot_q8k(x, qrow, wtype):
    """The -DQ8_DOT product of x with one Q4_K/Q6_K row: x quantized to
    Q8_K, then the integer dot (dot_q8_quant)."""
    d, qs, bs = quantize_q8k(x)
    q = np.ascontiguousarray(qrow, np.uint8)
    return np.float32(lib().orc_dot_q8k(_p(d), _p(qs), _p(bs), _p(q), wtype, qs.size))


def qmat_mul(x, q, wtype, N, K, add=None):
    """out[T][N] = add + x[T][K] . W^T for a Q8_0/Q4_0/Q4_K/Q6_K matrix of N
    rows (moe_oracle.c orc_qmat_mul; K-quants with K % 256 == 0 through Q8_K);
    add None, [N] or [T][N]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    q = np.ascontiguousarray(q, np.uint8)
    T = x.shape[0]
    a = None if add is None else np.ascontiguousarray(add, np.float32).ravel()
    out = np.empty((T, N), np.float32)
    lib().orc_qmat_mul(_p(x), T, _p(q), wtype, N, K, None if a is None else _p(a),
                       0 if a is None else a.size, _p(out))
    return out


def dequant(qrow, wtype, n):
    q = np.ascontiguousarray(qrow, np.uint8)
    out = np.empty(n, np.float32)
    lib().orc_dequant_row(_p(q), wtype, _p(out), n)
    return out


def fused_ffn(x, gate, up, down, wtype, E, EI):
    x = np.ascontiguousarray(x, np.float32)
    h = np.empty(EI, np.float32)
    out = np.empty(E, np.float32)
    lib().orc_fused_ffn(_p(x), _p(gate), _p(up), _p(down), wtype, E, EI, _p(h), _p(out))
    return out


def moe_ffn(x, layer: dict, topk: int, renorm: bool, bias=None, nthreads=None):
    """Whole layer: returns (out, ids, w, logits, probs)."""
    x = np.ascontiguousarray(x, np.float32)
    T, E = x.shape
    NE, EI = layer["NE"], layer["EI"]
    out = np.empty((T, E), np.float32)
    ids = np.empty((T, topk), np.uint32)
    w = np.empty((T, topk), np.float32)
    lg = np.empty((T, NE), np.float32)
    pr = np.empty((T, NE), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_moe_ffn(_p(x), _p(out), T, _p(layer["router"]), _p(b), _ptrs(layer["gate"]),
                      _ptrs(layer["up"]), _ptrs(layer["down"]), layer["wtype"], E, EI, NE,
                      topk, int(renorm), _p(ids), _p(w), _p(lg), _p(pr),
                      nthreads or threads())
    return out, ids, w, lg, pr


def expf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_expf_array(_p(x), _p(out), x.size)
    return out


def expf_bits(bits0: int, n: int, nthreads=None):
    out = np.empty(n, np.float32)
    lib().orc_expf_bits(bits0, n, _p(out), nthreads or threads())
    return out


class OlmoeModel:
    """The decode step of the reference's OLMoE (orc_olmoe_*) or Mixtral
    (orc_llama_*) model: md is a model dict of llm.c_amd/hiplm.py
    (synth_olmoe / synth_mixtral), C the context length, table its pointer
    table (hiplm.ptr_table / ptr_table_llama)."""

    def __init__(self, md: dict, C_ctx: int, table):
        self.md = md
        self.V, self.E, self.L, self.K = md["V"], md["E"], md["layers"], md["K"]
        self.table = table  # keeps the pointer table alive
        L = lib()
        # per-tensor block types (hiplm.q4_k_m_types), as orc_*_new_typed take them
        self.types = None
        if "types" in md:
            t = md["types"]
            self.types = np.asarray([t["embd"], t["output"]] +
                                    [x for lt in t["layers"] for x in lt], np.int32)
        if md["arch"] == "olmoe":
            self._dec, self._run, self._free = L.orc_olmoe_decode, L.orc_olmoe_run, L.orc_olmoe_free
            args = (md["layers"], md["E"], md["H"], md["V"], md["NE"], md["K"], md["EI"], C_ctx,
                    md["theta"])
            self.h = (L.orc_olmoe_new(*args, md["wtype"], table) if self.types is None else
                      L.orc_olmoe_new_typed(*args, _p(self.types), table))
        else:
            self._dec, self._run, self._free = L.orc_llama_decode, L.orc_llama_run, L.orc_llama_free
            args = (md["layers"], md["E"], md["H"], md["KH"], md["V"], md["NE"], md["K"], md["EI"],
                    C_ctx, md["theta"], md["window"])
            self.h = (L.orc_llama_new(*args, md["wtype"], table) if self.types is None else
                      L.orc_llama_new_typed(*args, _p(self.types), table))
        self.pos = 0

    def decode(self, tok: int, trace: bool = False):
        """(greedy pick, logits [V]) and, with trace, (moe_in [L][E], ids [L][K], w [L][K])."""
        lg = np.empty(self.V, np.float32)
        mi = np.empty((self.L, self.E), np.float32) if trace else None
        ids = np.empty((self.L, self.K), np.uint32) if trace else None
        w = np.empty((self.L, self.K), np.float32) if trace else None
        nxt = self._dec(self.h, int(tok), self.pos, _p(lg), _p(mi), _p(ids), _p(w), threads())
        self.pos += 1
        return (nxt, lg, (mi, ids, w)) if trace else (nxt, lg)

    def run(self, prompt, n_gen: int):
        """The prompt token by token then n_gen greedy steps: (tokens [n_gen+1],
        logits [n_gen+1][V])."""
        pr = np.ascontiguousarray(prompt, np.int32)
        lg = np.empty((n_gen + 1, self.V), np.float32)
        toks = np.empty(n_gen + 1, np.int32)
        self._run(self.h, _p(pr), pr.size, n_gen, _p(lg), _p(toks), threads())
        self.pos += pr.size + n_gen
        return toks, lg

    def free(self):
        if self.h:
            self._free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
