"""ctypes binding of the whole-model decode ABI of libhip_moe.so
(include/hip_lm.h) and the seeded synthetic models the tests and the bench
run it on.

Like hipmoe.py it only marshals arrays and pointers; it never computes a
result on the CPU, and it raises if the library is missing.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import hipmoe
from hipmoe import Q4_0, Q8_0, HipMoeError, _ptr, last_error, lib, row_bytes  # noqa: F401

# tensor kinds of moe_stream_tensor (include/moe_synth.h)
T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_O = 0, 1, 2, 3
T_ATTN_NORM, T_Q_NORM, T_K_NORM, T_FFN_NORM = 4, 5, 6, 7
T_TOKEN_EMBD, T_OUTPUT, T_OUTPUT_NORM, T_PROMPT = 8, 9, 10, 11
T_GLOBAL = 0xFFFFFFFF

# per-layer order of the flat pointer table (oracle/moe_oracle.h, oracle/ref/ref_olmoe.c)
LAYER_KEYS = ("attn_norm", "q", "k", "v", "q_norm", "k_norm", "o", "ffn_norm", "router",
              "gate", "up", "down")


def _stream(layer, kind):
    return lib().moe_stream_tensor(layer, kind)


def _norm(seed, layer, kind, n, norm_std):
    if norm_std == 0:
        return np.ones(n, np.float32)
    return hipmoe.synth_normal(seed, _stream(layer, kind), n, 1.0, norm_std)


def q4_k_m_types(layers: int) -> dict:
    """Per-tensor block types as a Q4_K_M GGUF mixes them: Q4_K throughout,
    Q6_K for the output, and for attn_v and the experts' down in the first
    and last eighth of the layers and every third layer between
    (hip_lm_desc's embd_type / output_type / layer_types)."""
    Q4K, Q6K = hipmoe.Q4_K, hipmoe.Q6_K

    def more(l):
        return l < layers // 8 or l >= 7 * layers // 8 or (l - layers // 8) % 3 == 2
    return dict(embd=Q4K, output=Q6K,
                layers=[(Q4K, Q4K, Q6K if more(l) else Q4K, Q4K, Q4K, Q6K if more(l) else Q4K)
                        for l in range(layers)])


def synth_olmoe(seed: int, layers: int, E: int, H: int, V: int, NE: int, K: int, EI: int,
                wtype: int = Q8_0, std: float = 0.02, norm_std: float = 0.0,
                theta: float = 10000.0, types: dict | None = None) -> dict:
    """An OLMoE-shaped model (models/olmoe/olmoe.c:123-183 tensors): every
    matrix N(0, std) quantized to wtype (or to its type in `types`, as
    q4_k_m_types gives them), the router fp32 N(0, std), norm weights fp32
    (1, or N(1, norm_std))."""
    G = T_GLOBAL
    md = dict(arch="olmoe", layers=layers, E=E, H=H, V=V, NE=NE, K=K, EI=EI, wtype=wtype,
              theta=theta)
    et = types["embd"] if types else wtype
    ot = types["output"] if types else wtype
    if types:
        md["types"] = types
    md["token_embd"] = hipmoe.synth_quant_matrix(seed, _stream(G, T_TOKEN_EMBD), std, et, V, E)
    md["output"] = hipmoe.synth_quant_matrix(seed, _stream(G, T_OUTPUT), std, ot, V, E)
    md["output_norm"] = _norm(seed, G, T_OUTPUT_NORM, E, norm_std)
    md["blk"] = []
    for l in range(layers):
        b = {}
        lt = types["layers"][l] if types else (wtype,) * 6
        for i, (key, kind) in enumerate((("q", T_ATTN_Q), ("k", T_ATTN_K), ("v", T_ATTN_V),
                                         ("o", T_ATTN_O))):
            b[key] = hipmoe.synth_quant_matrix(seed, _stream(l, kind), std, lt[i], E, E)
        for key, kind in (("attn_norm", T_ATTN_NORM), ("q_norm", T_Q_NORM),
                          ("k_norm", T_K_NORM), ("ffn_norm", T_FFN_NORM)):
            b[key] = _norm(seed, l, kind, E, norm_std)
        mt = lt[4] | (lt[5] << 8 if lt[5] != lt[4] else 0)
        moe = hipmoe.synth_layer(seed, l, mt, E, EI, NE, std, None)
        b["router"], b["gate"], b["up"], b["down"] = (moe["router"], moe["gate"], moe["up"],
                                                      moe["down"])
        md["blk"].append(b)
    return md


def synth_mixtral(seed: int, layers: int, E: int, H: int, KH: int, V: int, NE: int, K: int,
                  EI: int, wtype: int = Q4_0, std: float = 0.02, norm_std: float = 0.0,
                  theta: float = 1e6, window: int = 0, share_layers: bool = False,
                  types: dict | None = None) -> dict:
    """A Mixtral-shaped model (models/llama/llama.c:80-175 tensors): H query
    heads and KH kv heads of 128, NE experts in separate tensors (kept
    stacked here, one row per expert), every matrix N(0, std) quantized to
    wtype, the router fp32, norms 1 or N(1, norm_std).  share_layers: every
    layer holds layer 0's arrays (the same values, still uploaded once per
    layer) - for benchmarks of models too large to generate layer by layer."""
    G = T_GLOBAL
    HL = 128
    md = dict(arch="mixtral", layers=layers, E=E, H=H, KH=KH, V=V, NE=NE, K=K, EI=EI,
              wtype=wtype, theta=theta, window=window)
    et = types["embd"] if types else wtype
    ot = types["output"] if types else wtype
    if types:
        md["types"] = types
    md["token_embd"] = hipmoe.synth_quant_matrix(seed, _stream(G, T_TOKEN_EMBD), std, et, V, E)
    md["output"] = hipmoe.synth_quant_matrix(seed, _stream(G, T_OUTPUT), std, ot, V, E)
    md["output_norm"] = _norm(seed, G, T_OUTPUT_NORM, E, norm_std)
    md["blk"] = []
    for l in range(layers):
        if share_layers and l > 0:
            md["blk"].append(md["blk"][0])
            continue
        b = {}
        lt = types["layers"][l] if types else (wtype,) * 6
        for i, (key, kind, rows, cols) in enumerate(
                (("q", T_ATTN_Q, H * HL, E), ("k", T_ATTN_K, KH * HL, E),
                 ("v", T_ATTN_V, KH * HL, E), ("o", T_ATTN_O, E, H * HL))):
            b[key] = hipmoe.synth_quant_matrix(seed, _stream(l, kind), std, lt[i], rows, cols)
        for key, kind in (("attn_norm", T_ATTN_NORM), ("ffn_norm", T_FFN_NORM)):
            b[key] = _norm(seed, l, kind, E, norm_std)
        mt = lt[4] | (lt[5] << 8 if lt[5] != lt[4] else 0)
        moe = hipmoe.synth_layer(seed, l, mt, E, EI, NE, std, None)
        b["router"], b["gate"], b["up"], b["down"] = (moe["router"], moe["gate"], moe["up"],
                                                      moe["down"])
        md["blk"].append(b)
    return md


def ptr_table_llama(md: dict):
    """The flat table the llama oracle and harness take: token_embd, output,
    output_norm, then per layer attn_norm, q, k, v, o, ffn_norm, router, the
    NE gate experts, the NE up experts, the NE down experts."""
    arrs = [md["token_embd"], md["output"], md["output_norm"]]
    for b in md["blk"]:
        arrs += [b[k] for k in ("attn_norm", "q", "k", "v", "o", "ffn_norm", "router")]
        for key in ("gate", "up", "down"):
            arrs += [b[key][e] for e in range(md["NE"])]
    tab = (C.c_void_p * len(arrs))()
    for i, a in enumerate(arrs):
        assert a.flags["C_CONTIGUOUS"]
        tab[i] = a.ctypes.data
    return tab


def synth_prompt(seed: int, n: int, V: int) -> np.ndarray:
    """n token ids in [0, V), a pure function of (seed, n, V)."""
    u = hipmoe.synth_normal(seed, _stream(T_GLOBAL, T_PROMPT), n, 0.0, 1.0).astype(np.float64)
    return (np.floor(np.abs(u) * 1e6).astype(np.int64) % V).astype(np.int32)


def ptr_table(md: dict):
    """The flat table 3 + 12 * layers pointers (token_embd, output,
    output_norm, then LAYER_KEYS per layer) the oracle and the reference
    harness take.  The arrays stay owned by md."""
    arrs = [md["token_embd"], md["output"], md["output_norm"]]
    for b in md["blk"]:
        arrs += [b[k] for k in LAYER_KEYS]
    tab = (C.c_void_p * len(arrs))()
    for i, a in enumerate(arrs):
        assert a.flags["C_CONTIGUOUS"]
        tab[i] = a.ctypes.data
    return tab


# --------------------------------------------------------------------------
# the model ABI (include/hip_lm.h)
# --------------------------------------------------------------------------

ARCH_OLMOE, ARCH_MIXTRAL = 1, 2
_vp, _sz = C.c_void_p, C.c_size_t


class Desc(C.Structure):
    """struct hip_lm_desc"""
    _fields_ = [("arch", C.c_int), ("wtype", C.c_int), ("layers", _sz), ("E", _sz),
                ("heads", _sz), ("kv_heads", _sz), ("vocab", _sz), ("context", _sz),
                ("NE", _sz), ("topk", _sz), ("EI", _sz), ("rope_theta", C.c_float),
                ("sliding_window", _sz), ("token_embd", _vp), ("output", _vp),
                ("output_norm", _vp), ("attn_norm", _vp), ("attn_q", _vp), ("attn_k", _vp),
                ("attn_v", _vp), ("attn_o", _vp), ("q_norm", _vp), ("k_norm", _vp),
                ("ffn_norm", _vp), ("gate_inp", _vp), ("gate_e", _vp), ("up_e", _vp),
                ("down_e", _vp), ("embd_type", C.c_int), ("output_type", C.c_int),
                ("layer_types", _vp)]


_lm_bound = False


def _bind():
    global _lm_bound
    if _lm_bound:
        return lib()
    L = lib()
    i32, f32p = C.c_int, C.POINTER(C.c_float)
    L.hip_lm_upload.restype = _vp
    L.hip_lm_upload.argtypes = [C.POINTER(Desc)]
    L.hip_lm_decode.restype = i32
    L.hip_lm_decode.argtypes = [_vp, i32, _vp, C.POINTER(C.c_int)]
    L.hip_lm_generate.restype = i32
    L.hip_lm_generate.argtypes = [_vp, _vp, _sz, _sz, _vp, f32p]
    L.hip_lm_set_moe_path.restype = i32
    L.hip_lm_set_moe_path.argtypes = [_vp, i32]
    L.hip_lm_prefill.restype = i32
    L.hip_lm_prefill.argtypes = [_vp, _vp, _sz, _vp, C.POINTER(C.c_int)]
    L.hip_lm_trace.restype = i32
    L.hip_lm_trace.argtypes = [_vp, _vp, _vp, _vp]
    L.hip_lm_reset.restype = i32
    L.hip_lm_reset.argtypes = [_vp]
    L.hip_lm_weight_bytes.restype = _sz
    L.hip_lm_weight_bytes.argtypes = [_vp]
    L.hip_lm_free.restype = None
    L.hip_lm_free.argtypes = [_vp]
    L.hip_lm_batch_new.restype = _vp
    L.hip_lm_batch_new.argtypes = [_vp, _sz]
    L.hip_lm_batch_decode.restype = i32
    L.hip_lm_batch_decode.argtypes = [_vp, _vp, _vp, _vp]
    L.hip_lm_batch_generate.restype = i32
    L.hip_lm_batch_generate.argtypes = [_vp, _vp, _sz, _sz, _vp, f32p]
    L.hip_lm_batch_reset.restype = i32
    L.hip_lm_batch_reset.argtypes = [_vp]
    L.hip_lm_batch_free.restype = None
    L.hip_lm_batch_free.argtypes = [_vp]
    _lm_bound = True
    return L


def _parr(arrs):
    tab = (C.c_void_p * len(arrs))()
    for i, a in enumerate(arrs):
        assert a.flags["C_CONTIGUOUS"]
        tab[i] = a.ctypes.data
    return tab


class LmModel:
    """One uploaded model (hip_lm_upload) of a synth_olmoe dict."""

    def __init__(self, md: dict, context: int):
        L = _bind()
        self.md = md
        self.V, self.E, self.L, self.K = md["V"], md["E"], md["layers"], md["K"]
        blk, NE = md["blk"], md["NE"]
        self._keep = []

        def per_layer(key):
            t = _parr([b[key] for b in blk])
            self._keep.append(t)
            return C.cast(t, _vp)

        def experts(key):
            t = (C.c_void_p * (len(blk) * NE))()
            for l, b in enumerate(blk):
                for e in range(NE):
                    t[l * NE + e] = b[key][e].ctypes.data
            self._keep.append(t)
            return C.cast(t, _vp)

        d = Desc()
        d.arch = ARCH_OLMOE if md["arch"] == "olmoe" else ARCH_MIXTRAL
        d.wtype = md["wtype"]
        d.layers, d.E, d.heads = md["layers"], md["E"], md["H"]
        d.kv_heads = md.get("KH", md["H"])
        d.vocab, d.context, d.NE, d.topk, d.EI = md["V"], context, NE, md["K"], md["EI"]
        d.rope_theta = md["theta"]
        d.sliding_window = md.get("window", 0)
        d.token_embd, d.output = md["token_embd"].ctypes.data, md["output"].ctypes.data
        d.output_norm = md["output_norm"].ctypes.data
        d.attn_norm, d.attn_q, d.attn_k = per_layer("attn_norm"), per_layer("q"), per_layer("k")
        d.attn_v, d.attn_o, d.ffn_norm = per_layer("v"), per_layer("o"), per_layer("ffn_norm")
        if d.arch == ARCH_OLMOE:
            d.q_norm, d.k_norm = per_layer("q_norm"), per_layer("k_norm")
        d.gate_inp = per_layer("router")
        d.gate_e, d.up_e, d.down_e = experts("gate"), experts("up"), experts("down")
        if "types" in md:
            ty = md["types"]
            d.embd_type, d.output_type = ty["embd"], ty["output"]
            lt = np.ascontiguousarray(np.asarray(ty["layers"], np.int32).reshape(-1))
            self._keep.append(lt)
            d.layer_types = lt.ctypes.data
        self.h = L.hip_lm_upload(C.byref(d))
        if not self.h:
            raise HipMoeError("hip_lm_upload: " + last_error())

    def decode(self, tok: int):
        """One step at the model's position: (greedy pick, logits [V])."""
        lg = np.empty(self.V, np.float32)
        nxt = C.c_int(-1)
        if _bind().hip_lm_decode(self.h, int(tok), lg.ctypes.data, C.byref(nxt)) != 1:
            raise HipMoeError("hip_lm_decode: " + last_error())
        return nxt.value, lg

    def prefill(self, prompt):
        """The prompt as one forward (hip_lm_prefill): (greedy pick, logits
        [V] of its last row)."""
        pr = np.ascontiguousarray(prompt, np.int32)
        lg = np.empty(self.V, np.float32)
        nxt = C.c_int(-1)
        if _bind().hip_lm_prefill(self.h, pr.ctypes.data, pr.size, lg.ctypes.data,
                                  C.byref(nxt)) != 1:
            raise HipMoeError("hip_lm_prefill: " + last_error())
        return nxt.value, lg

    def generate(self, prompt, n_gen: int):
        """(tokens [n_gen + 1], device ms of the n_gen generated steps)."""
        pr = np.ascontiguousarray(prompt, np.int32)
        toks = np.empty(n_gen + 1, np.int32)
        ms = C.c_float(0)
        if _bind().hip_lm_generate(self.h, pr.ctypes.data, pr.size, n_gen, toks.ctypes.data,
                                   C.byref(ms)) != 1:
            raise HipMoeError("hip_lm_generate: " + last_error())
        return toks, ms.value

    def trace(self):
        """The last step's (moe_in [L][E], ids [L][K], w [L][K])."""
        mi = np.empty((self.L, self.E), np.float32)
        ids = np.empty((self.L, self.K), np.uint32)
        w = np.empty((self.L, self.K), np.float32)
        if _bind().hip_lm_trace(self.h, mi.ctypes.data, ids.ctypes.data, w.ctypes.data) != 1:
            raise HipMoeError("hip_lm_trace: " + last_error())
        return mi, ids, w

    def reset(self):
        if _bind().hip_lm_reset(self.h) != 1:
            raise HipMoeError("hip_lm_reset: " + last_error())

    def set_moe_path(self, path: int):
        """Force every layer's MoE path (hipmoe.PATH_*)."""
        if _bind().hip_lm_set_moe_path(self.h, path) != 1:
            raise HipMoeError("hip_lm_set_moe_path: " + last_error())

    def weight_bytes(self) -> int:
        return _bind().hip_lm_weight_bytes(self.h)

    def free(self):
        if self.h:
            _bind().hip_lm_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LmBatch:
    """nseq sequences decoding in lockstep on an LmModel's weights
    (hip_lm_batch_*)."""

    def __init__(self, model: LmModel, nseq: int):
        self.model, self.S, self.V = model, nseq, model.V
        self.h = _bind().hip_lm_batch_new(model.h, nseq)
        if not self.h:
            raise HipMoeError("hip_lm_batch_new: " + last_error())

    def decode(self, toks):
        """One step: (picks [S], logits [S][V])."""
        t = np.ascontiguousarray(toks, np.int32)
        assert t.size == self.S
        lg = np.empty((self.S, self.V), np.float32)
        nxt = np.empty(self.S, np.int32)
        if _bind().hip_lm_batch_decode(self.h, t.ctypes.data, lg.ctypes.data,
                                       nxt.ctypes.data) != 1:
            raise HipMoeError("hip_lm_batch_decode: " + last_error())
        return nxt, lg

    def generate(self, prompts, n_gen: int):
        """prompts [S][n_prompt] -> (tokens [S][n_gen + 1], device ms of the
        n_gen generated steps)."""
        pr = np.ascontiguousarray(prompts, np.int32)
        assert pr.ndim == 2 and pr.shape[0] == self.S
        toks = np.empty((self.S, n_gen + 1), np.int32)
        ms = C.c_float(0)
        if _bind().hip_lm_batch_generate(self.h, pr.ctypes.data, pr.shape[1], n_gen,
                                         toks.ctypes.data, C.byref(ms)) != 1:
            raise HipMoeError("hip_lm_batch_generate: " + last_error())
        return toks, ms.value

    def reset(self):
        if _bind().hip_lm_batch_reset(self.h) != 1:
            raise HipMoeError("hip_lm_batch_reset: " + last_error())

    def free(self):
        if self.h:
            _bind().hip_lm_batch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
