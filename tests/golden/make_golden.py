"""Write golden vectors for the MoE FFN path from the compiled reference.

Run in a container that holds the reference tree (after
`oracle/ref/build_ref.sh`), as a standalone process:

    python tests/golden/make_golden.py

The reference library (oracle/_ref/libref_moe.so) is built from the
reference's own C sources with AVX2 flags; its thread pool starts with the
library and spins until the process exits, which is why this is a separate
script.  Inputs come from the package's seeded generator (llm.c_amd/host/
synth.c); each fixture stores the seed plus SHA-256 digests of the generated
input bytes, so a test regenerates the inputs and first proves they are the
same bytes.  Outputs are the reference's own results:

  quant.npz          quantize_row_q8_0 (quant.c:62-78) and the Q4_0 quantizer
                     of test/quant.c:45-79 on seeded and edge-case blocks
  dot.npz            dot_f32_quant (quant.c:577-614) on seeded rows
  route_<cfg>.npz    router logits, softmax probabilities, top-k ids/weights
                     (matmul.c:451-462, nn.c:221-308, llama.c:422-427)
  ffn_<wt>.npz       fused_ffn_silu for one expert (nn.c:496-539)
  moe_<cfg>.npz      full moe_ffn layer outputs (olmoe.c:343-407,
                     llama.c:393-457; with a router bias through the add
                     argument of tensor_mma_transposed_2x2)
  qmat.npz           tensor_mma_transposed_2x2 with a Q8_0/Q4_0 right operand
                     (matmul.c:13-33,285-312) for T = 1..9, add NULL/[N]/[T][N]
  kquant.npz         the K-quant path of the default -DQ8_DOT build:
                     quantize_row_q8 (quant.c:627-654) on seeded and edge
                     blocks; dot_q8_quant / dot_f32_quant / dequant_row on
                     Q4_K/Q6_K rows (the fill patterns of test/quant_dot.c:
                     12-34 and seeded rows); tensor_mma_transposed_2x2 with
                     a Q4_K/Q6_K right operand (matmul.c:285-312)
  kquant_moe.npz     the reference's moe_ffn (olmoe.c:343-407, llama.c:393-457)
                     on Q4_K/Q6_K experts (gate/up Q4_K with down Q6_K, as a
                     Q4_K_M file mixes them, and all Q6_K), and one expert's
                     fused_ffn_silu (nn.c:496-539) for both mixes
  model_<case>.npz   the whole OLMoE model (olmoe.c:409-580) or Mixtral model
                     (llama.c:458-576): greedy tokens and per-step logits of
                     the reference's olmoe_decode / llama_decode run over the
                     prompt then n_gen steps, and (but for MODEL_DEC_ONLY) of
                     its generate order (one prefill of the prompt, then
                     decode)
  batch_<case>.npz   several seeded prompts, each decoded by the reference
                     alone (BATCH_CASES), for the lockstep batch

`python tests/golden/make_golden.py qmat` writes qmat.npz alone, `... kquant`
kquant.npz alone, `... model` the model fixtures alone.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(HERE, "..", ".."))
sys.path.insert(0, os.path.join(REPO, "llm.c_amd"))
import hipmoe  # noqa: E402

SEED = 1337
REF_LIB = os.path.join(REPO, "oracle", "_ref", "libref_moe.so")

CONFIGS = {
    # name: (wtype, E, EI, NE, topk, renorm, bias_std)
    "olmoe_q8": (hipmoe.Q8_0, 2048, 1024, 64, 8, 0, None),
    "olmoe_q4_skew": (hipmoe.Q4_0, 2048, 1024, 64, 8, 0, 1.0),
    "mixtral_q4": (hipmoe.Q4_0, 4096, 14336, 8, 2, 1, None),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref():
    L = C.CDLL(REF_LIB)
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    L.ref_route.argtypes = [vp, sz, sz, sz, vp, vp, sz, i32, vp, vp, vp, vp]
    L.ref_moe_ffn_composed.argtypes = [vp, vp, sz, vp, vp, vp, vp, vp, i32, sz, sz, sz, sz,
                                       i32]
    L.ref_olmoe_moe_ffn.argtypes = [vp, vp, sz, vp, vp, vp, vp, i32, sz, sz, sz, sz]
    L.ref_llama_moe_ffn.argtypes = [vp, vp, sz, vp, vp, vp, vp, i32, sz, sz, sz, sz]
    L.ref_fused_ffn.argtypes = [vp, vp, vp, vp, i32, sz, sz, vp]
    L.ref_dot.argtypes = [vp, vp, i32, sz]
    L.ref_qmat_mul.argtypes = [vp, sz, vp, i32, sz, sz, vp, sz, vp]
    L.ref_dot.restype = C.c_float
    L.ref_quantize_q8_0.argtypes = [vp, vp, sz]
    L.ref_quantize_q4_0.argtypes = [vp, vp, sz]
    L.ref_quantize_q8k.argtypes = [vp, sz, vp, vp, vp]
    L.ref_quantize_q8k.restype = None
    L.ref_dot_q8k.argtypes = [vp, vp, i32, sz]
    L.ref_dot_q8k.restype = C.c_float
    L.ref_dequant.argtypes = [vp, i32, vp, sz]
    L.ref_dequant.restype = None
    return L


def p(a):
    return None if a is None else a.ctypes.data


def quant_blocks() -> np.ndarray:
    """Seeded blocks plus edge cases, 32 floats each."""
    rng_blocks = [hipmoe.synth_normal(SEED, 0x5151_0000 + i, 32, 0.0, s)
                  for i, s in enumerate([0.02] * 24 + [1.0] * 24 + [1e-3, 50.0, 3e4, 1e-6])]
    edge = []
    edge.append(np.zeros(32, np.float32))                      # amax = 0
    b = np.zeros(32, np.float32); b[5] = -1.0; edge.append(b)  # single negative
    edge.append(np.linspace(-1, 1, 32, dtype=np.float32))      # ramp
    b = np.full(32, 0.5, np.float32); b[0] = 127.0; edge.append(b)  # x*id ties
    b = (np.arange(32, dtype=np.float32) - 16) * 0.25; edge.append(b)
    edge.append(np.full(32, 7e4, np.float32))                   # scale overflows fp16
    edge.append(np.full(32, -3e-8, np.float32))                 # subnormal fp16 scale
    b = np.arange(32, dtype=np.float32) / 7.0; edge.append(b)  # Q4 half-way ties
    return np.stack(rng_blocks + edge).astype(np.float32)


# name: (wtype, T, N, K, add: None | "bcast" ([N]) | "rows" ([T][N]))
QMAT_CASES = {
    "q8_t1": (hipmoe.Q8_0, 1, 203, 2048, None),
    "q8_t5_rows": (hipmoe.Q8_0, 5, 77, 512, "rows"),
    "q8_t9": (hipmoe.Q8_0, 9, 50, 256, None),
    "q4_t1": (hipmoe.Q4_0, 1, 130, 4096, None),
    "q4_t3_bcast": (hipmoe.Q4_0, 3, 64, 4096, "bcast"),
    "q4_t7_rows": (hipmoe.Q4_0, 7, 33, 1024, "rows"),
}


def qmat_inputs(i: int, wt: int, T: int, N: int, K: int, add):
    q = hipmoe.synth_quant_matrix(SEED, 0x7400 + i, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7500 + i, T * K).reshape(T, K)
    a = None
    if add is not None:
        a = hipmoe.synth_normal(SEED, 0x7600 + i, N if add == "bcast" else T * N)
    return q, x, a


# K-quant products: name: (wtype, T, N, K, add) as QMAT_CASES.  K = 768
# (three super-blocks) puts odd Q6_K blocks and rows at 2-byte offsets;
# 14336 is Mixtral's d_ff; 256 one super-block a row.
KQ_CASES = {
    "q4k_t1": (hipmoe.Q4_K, 1, 203, 2048, None),
    "q4k_t5_rows": (hipmoe.Q4_K, 5, 77, 4096, "rows"),
    "q4k_t2_bcast_14336": (hipmoe.Q4_K, 2, 40, 14336, "bcast"),
    "q4k_t1_256": (hipmoe.Q4_K, 1, 300, 256, None),
    "q6k_t1": (hipmoe.Q6_K, 1, 130, 4096, None),
    "q6k_t3_bcast": (hipmoe.Q6_K, 3, 64, 2048, "bcast"),
    "q6k_t9_rows_768": (hipmoe.Q6_K, 9, 33, 768, "rows"),
    "q6k_t1_14336": (hipmoe.Q6_K, 1, 24, 14336, None),
}


def kq_inputs(i: int, wt: int, T: int, N: int, K: int, add):
    q = hipmoe.synth_quant_matrix(SEED, 0x7a00 + i, 0.02, wt, N, K)
    x = hipmoe.synth_normal(SEED, 0x7b00 + i, T * K).reshape(T, K)
    a = None
    if add is not None:
        a = hipmoe.synth_normal(SEED, 0x7c00 + i, N if add == "bcast" else T * N)
    return q, x, a


def fill_q4_K(nb: int) -> np.ndarray:
    """The deterministic Q4_K blocks of test/quant_dot.c:12-22."""
    out = np.zeros((nb, 144), np.uint8)
    for i in range(nb):
        out[i, 0:2] = (0x00, 0x3C)   # d = 1.0 (f16 0x3C00, little-endian)
        out[i, 2:4] = (0x00, 0x38)   # dmin = 0.5
        out[i, 4:16] = [5 + (j * 3) % 40 for j in range(12)]
        out[i, 16:144] = [((i + j) * 7 + 3) & 0xFF for j in range(128)]
    return out.reshape(-1)


def fill_q6_K(nb: int) -> np.ndarray:
    """The deterministic Q6_K blocks of test/quant_dot.c:24-34."""
    out = np.zeros((nb, 210), np.uint8)
    for i in range(nb):
        out[i, 0:128] = [((i + j) * 11 + 7) & 0xFF for j in range(128)]
        out[i, 128:192] = [((i + j) * 5 + 2) & 0xFF for j in range(64)]
        out[i, 192:208] = np.array([((i + j) * 3) % 61 - 30 for j in range(16)],
                                   np.int8).view(np.uint8)
        out[i, 208:210] = (0x00, 0x3C)
    return out.reshape(-1)


def q8k_blocks() -> np.ndarray:
    """Seeded 256-value blocks plus edge cases for quantize_row_q8."""
    blocks = [hipmoe.synth_normal(SEED, 0x7d00 + i, 256, 0.0, s)
              for i, s in enumerate([0.02] * 6 + [1.0] * 6 + [1e-3, 40.0, 3e4, 1e-30])]
    i = np.arange(256, dtype=np.float32)
    blocks.append(np.sin(i * np.float32(0.1)).astype(np.float32) * np.float32(0.5))
    blocks.append(np.zeros(256, np.float32))                  # amax = 0: zero block
    b = np.zeros(256, np.float32); b[77] = -2.5; blocks.append(b)   # one negative spike
    b = hipmoe.synth_normal(SEED, 0x7e00, 256, 0.0, 0.1)
    b[10], b[200] = 3.0, -3.0; blocks.append(b)               # tie: the first wins (+)
    b = hipmoe.synth_normal(SEED, 0x7e01, 256, 0.0, 0.1)
    b[10], b[200] = -3.0, 3.0; blocks.append(b)               # tie: the first wins (-)
    b = np.full(256, 0.25, np.float32); b[3] = -0.5; blocks.append(b)  # +63.5 rounds away
    blocks.append((i - 128) / np.float32(64.0))               # ramp with x.5 products
    return np.stack(blocks).astype(np.float32)


def kquant_goldens(R):
    fx = {}
    # quantize_row_q8
    xb = q8k_blocks()
    flat = np.ascontiguousarray(xb.reshape(-1))
    nb = xb.shape[0]
    d = np.empty(nb, np.float32)
    qs = np.empty(flat.size, np.int8)
    bs = np.empty((nb, 16), np.int16)
    R.ref_quantize_q8k(p(flat), flat.size, p(d), p(qs), p(bs))
    fx.update(q8k_x=xb, q8k_d=d, q8k_qs=qs, q8k_bsums=bs)
    # the reference test's rows (test/quant_dot.c:62-153): dots and dequant
    for wt, name, fill in ((hipmoe.Q4_K, "q4k", fill_q4_K), (hipmoe.Q6_K, "q6k", fill_q6_K)):
        for nbk in (1, 16):
            n = 256 * nbk
            row = fill(nbk)
            x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.037))
                 * np.float32(0.1)).astype(np.float32)
            deq = np.empty(n, np.float32)
            R.ref_dequant(p(row), wt, p(deq), n)
            fx[f"fill_{name}_{nbk}_w"] = row
            fx[f"fill_{name}_{nbk}_x"] = x
            fx[f"fill_{name}_{nbk}_dot_q8"] = np.float32(R.ref_dot_q8k(p(x), p(row), wt, n))
            fx[f"fill_{name}_{nbk}_dot_f32"] = np.float32(R.ref_dot(p(x), p(row), wt, n))
            fx[f"fill_{name}_{nbk}_deq"] = deq
        # seeded rows: every K the products use
        for n in (256, 768, 2048, 4096, 14336):
            rows = 3
            qm = hipmoe.synth_quant_matrix(SEED, 0x7f00 + n + wt, 0.02, wt, rows, n)
            x = hipmoe.synth_normal(SEED, 0x7f80 + n + wt, rows * n).reshape(rows, n)
            rb = hipmoe.row_bytes(wt, n)
            q8 = np.empty(rows, np.float32)
            f32 = np.empty(rows, np.float32)
            deq = np.empty((rows, n), np.float32)
            for r in range(rows):
                xr = np.ascontiguousarray(x[r])
                wr = np.ascontiguousarray(qm[r * rb:(r + 1) * rb])
                q8[r] = R.ref_dot_q8k(p(xr), p(wr), wt, n)
                f32[r] = R.ref_dot(p(xr), p(wr), wt, n)
                R.ref_dequant(p(wr), wt, p(deq[r]), n)
            fx[f"rows_{name}_{n}_sha_w"] = sha(qm)
            fx[f"rows_{name}_{n}_sha_x"] = sha(x)
            fx[f"rows_{name}_{n}_dot_q8"] = q8
            fx[f"rows_{name}_{n}_dot_f32"] = f32
            fx[f"rows_{name}_{n}_deq0"] = deq[0]
    # the product
    for i, (name, (wt, T, N, K, add)) in enumerate(KQ_CASES.items()):
        q, x, a = kq_inputs(i, wt, T, N, K, add)
        out = np.empty((T, N), np.float32)
        R.ref_qmat_mul(p(x), T, p(q), wt, N, K, p(a), 0 if a is None else a.size, p(out))
        fx[f"{name}_sha_w"] = sha(q)
        fx[f"{name}_sha_x"] = sha(x)
        fx[f"{name}_sha_add"] = sha(a) if a is not None else ""
        fx[f"{name}_out"] = out
        print(f"kquant {name}: T={T} N={N} K={K} add={add} |out|={np.linalg.norm(out):.4f}")
    np.savez(os.path.join(HERE, "kquant.npz"), seed=SEED, **fx)


# K-quant MoE layers (the gate/up type | the down type << 8, as a Q4_K_M
# file mixes them): name: (wtype, E, EI, NE, topk, renorm, T)
KQ_LAYERS = {
    "olmoe_q4k_q6k": (hipmoe.Q4_K | hipmoe.Q6_K << 8, 2048, 1024, 64, 8, 0, 4),
    "olmoe_q6k": (hipmoe.Q6_K, 2048, 1024, 64, 8, 0, 2),
    "mixtral_q4k_q6k": (hipmoe.Q4_K | hipmoe.Q6_K << 8, 4096, 14336, 8, 2, 1, 2),
    # d_model of 5 super-blocks (128 % 5 != 0: the gate/up kernel's rows per
    # workgroup do not divide its 128 lanes) and d_ff of 6 (the down
    # kernel's last chunk of super-blocks is partial), both type mixes
    "ragged_q4k_q6k": (hipmoe.Q4_K | hipmoe.Q6_K << 8, 1280, 1536, 16, 4, 0, 3),
    "ragged_q6k_q4k": (hipmoe.Q6_K | hipmoe.Q4_K << 8, 1280, 1536, 16, 4, 1, 2),
}


def kq_layer_goldens(R):
    """The reference's own static moe_ffn (olmoe.c:343-407 / llama.c:393-457)
    on K-quant expert tensors, and one expert's fused_ffn_silu for both
    mixes."""
    fx = {}
    for name, (wt, E, EI, NE, K, renorm, T) in KQ_LAYERS.items():
        lw = hipmoe.synth_layer(SEED, 0, wt, E, EI, NE, 0.02, None)
        x = hipmoe.synth_input(SEED, 0, T, E)
        gp, up_, dp = (hipmoe.expert_ptrs(lw[k]) for k in ("gate", "up", "down"))
        out = np.empty((T, E), np.float32)
        if renorm:
            R.ref_llama_moe_ffn(p(x), p(out), T, p(lw["router"]), gp, up_, dp, wt, E, EI, NE, K)
        else:
            R.ref_olmoe_moe_ffn(p(x), p(out), T, p(lw["router"]), p(lw["gate"]), p(lw["up"]),
                                p(lw["down"]), wt, E, EI, NE, K)
        fx[f"{name}_sha_gate"] = sha(lw["gate"])
        fx[f"{name}_sha_down"] = sha(lw["down"])
        fx[f"{name}_sha_x"] = sha(x)
        fx[f"{name}_out"] = out
        print(f"kq layer {name}: T={T} |out|={np.linalg.norm(out):.4f}")
        del lw
    for name, wt in (("q4k_q6k", hipmoe.Q4_K | hipmoe.Q6_K << 8),
                     ("q6k_q4k", hipmoe.Q6_K | hipmoe.Q4_K << 8)):
        E, EI = 2048, 1024
        gt, dt = hipmoe.wtypes(wt)
        g = hipmoe.synth_quant_matrix(SEED, 0x9011, 0.02, gt, EI, E)
        u = hipmoe.synth_quant_matrix(SEED, 0x9012, 0.02, gt, EI, E)
        d = hipmoe.synth_quant_matrix(SEED, 0x9013, 0.02, dt, E, EI)
        x = hipmoe.synth_normal(SEED, 0x9014, E)
        out = np.empty(E, np.float32)
        R.ref_fused_ffn(p(x), p(g), p(u), p(d), wt, E, EI, p(out))
        fx[f"ffn_{name}_sha"] = sha(np.concatenate([g, u, d, x.view(np.uint8)]))
        fx[f"ffn_{name}_out"] = out
    np.savez(os.path.join(HERE, "kquant_moe.npz"), seed=SEED, **fx)


def qmat_goldens(R):
    fx = {}
    for i, (name, (wt, T, N, K, add)) in enumerate(QMAT_CASES.items()):
        q, x, a = qmat_inputs(i, wt, T, N, K, add)
        out = np.empty((T, N), np.float32)
        R.ref_qmat_mul(p(x), T, p(q), wt, N, K, p(a), 0 if a is None else a.size, p(out))
        fx[f"{name}_sha_w"] = sha(q)
        fx[f"{name}_sha_x"] = sha(x)
        fx[f"{name}_sha_add"] = sha(a) if a is not None else ""
        fx[f"{name}_out"] = out
        print(f"qmat {name}: T={T} N={N} K={K} add={add} |out|={np.linalg.norm(out):.4f}")
    np.savez(os.path.join(HERE, "qmat.npz"), seed=SEED, **fx)


# name: (layers, E, H, V, NE, K, EI, C, wtype, norm_std, n_prompt, n_gen, logit stride)
# (Mixtral cases add kv heads and the sliding window in MIXTRAL_EXTRA.)
# The small cases run past their context (48 positions, C = 32: one
# kvcache_rotate; Mixtral's with a sliding window of 20, the rows it keeps)
# with non-unit norms; olmoe_full is the OLMoE-1B-7B shape with unit norms;
# mixtral_2l two layers of the Mixtral-8x7B shape (32 query / 8 kv heads,
# d_ff 14336, vocab 32000).  Logits are kept at every `stride`-th id plus
# each step's top 32.
MODEL_CASES = {
    "olmoe_small": (2, 1024, 8, 512, 64, 8, 512, 32, hipmoe.Q8_0, 0.1, 8, 40, 1),
    "olmoe_full": (16, 2048, 16, 50304, 64, 8, 1024, 2048, hipmoe.Q8_0, 0.0, 4, 4, 16),
    "mixtral_small": (2, 2048, 16, 512, 8, 2, 1024, 32, hipmoe.Q4_0, 0.1, 8, 40, 1),
    "mixtral_2l": (2, 4096, 32, 32000, 8, 2, 14336, 64, hipmoe.Q4_0, 0.0, 4, 4, 16),
    # caches longer than one 64-row attention block (nn.c:542,570-641 in
    # Mixtral's flash_attention; OLMoE's masked softmax over AT rows,
    # olmoe.c:286-320): 308 positions in a 256-row context, so up to four
    # blocks, one kvcache_rotate at 256 (OLMoE keeps 128, the Mixtral one its
    # sliding window of 200, which straddles block boundaries as it moves)
    "olmoe_long": (2, 1024, 8, 512, 64, 8, 512, 256, hipmoe.Q8_0, 0.1, 8, 300, 4),
    "mixtral_long": (2, 2048, 16, 512, 8, 2, 1024, 256, hipmoe.Q4_0, 0.1, 8, 300, 4),
    # the full OLMoE-1B-7B shape over 300 positions (five blocks), and two
    # layers of the Mixtral-8x7B shape after a 1024-token prompt (seventeen
    # blocks): the benchmarked lengths
    "olmoe_full_long": (16, 2048, 16, 50304, 64, 8, 1024, 2048, hipmoe.Q8_0, 0.0, 4, 296, 64),
    "mixtral_2l_long": (2, 4096, 32, 32000, 8, 2, 14336, 4096, hipmoe.Q4_0, 0.0, 1024, 32, 64),
    # long prompts in the reference's generate order (one prefill of the
    # prompt, olmoe.c:504-508, llama.c:560-564): OLMoE's masked softmax over
    # a 200-row prompt, and Mixtral's flash_attention over 240 rows with its
    # window of 200 masking inside the prefill
    "olmoe_prompt": (2, 1024, 8, 512, 64, 8, 512, 256, hipmoe.Q8_0, 0.1, 200, 8, 4),
    "mixtral_window_prompt": (2, 2048, 16, 512, 8, 2, 1024, 256, hipmoe.Q4_0, 0.1, 240, 8, 4),
    # K-quant models, the tensors' types mixed as a Q4_K_M GGUF mixes them
    # (hiplm.q4_k_m_types: Q4_K, Q6_K output, Q6_K attn_v and experts' down
    # in layer 1 of 2, in 8 of 16): past the context (one kvcache_rotate),
    # and the full OLMoE-1B-7B shape.  One-id prompts, so that the logits of
    # every position are written (a Q8_K rounding flip can come at any)
    "olmoe_q4km": (2, 1024, 8, 512, 64, 8, 512, 32, hipmoe.Q4_K, 0.1, 1, 47, 1),
    "mixtral_q4km": (2, 2048, 16, 512, 8, 2, 1024, 32, hipmoe.Q4_K, 0.1, 1, 47, 1),
    "olmoe_full_q4km": (16, 2048, 16, 50304, 64, 8, 1024, 2048, hipmoe.Q4_K, 0.0, 1, 11, 16),
}
# cases whose tensors carry per-tensor block types (hiplm.q4_k_m_types)
MODEL_TYPED = ("olmoe_q4km", "mixtral_q4km", "olmoe_full_q4km")
# Mixtral cases: (kv heads, sliding window, rope theta).  The window stays
# at least C - 64: with a longer cache, once the first 64-row block lies
# wholly outside the window the reference's flash_attention computes
# expf(-inf - -inf) for it (nn.c:603-608) and every later logit is NaN
# (C = 256, window 100: from position 163 on).
MIXTRAL_EXTRA = {
    "mixtral_small": (4, 20, 1e6),
    "mixtral_2l": (8, 0, 1e6),
    "mixtral_long": (4, 200, 1e6),
    "mixtral_2l_long": (8, 0, 1e6),
    "mixtral_window_prompt": (4, 200, 1e6),
    "mixtral_q4km": (4, 20, 1e6),
}
# cases written in decode order only (one olmoe_decode / llama_decode per
# prompt id); the others also in generate order (one prefill of the prompt)
MODEL_DEC_ONLY = ("olmoe_full_long", "mixtral_2l_long") + MODEL_TYPED
MODEL_TOPN = 32

# Several sequences at once, for the lockstep batch (hip_lm_batch_*): nseq
# prompts of n_prompt ids (sequence s: synth_prompt(SEED + 101 + s)), each
# decoded by the reference alone, then n_gen greedy steps; the reference's
# logits are written for the sequences in `check` (every sequence is
# independent of the others).  Sizes put the attention grid (kv heads x
# blocks x sequences) past three workgroups per CU of a 256-CU device with
# four blocks per kv head.
BATCH_CASES = {
    "olmoe_long": dict(nseq=26, n_prompt=200, n_gen=6, check=(0, 13, 25)),
    "mixtral_long": dict(nseq=52, n_prompt=200, n_gen=4, check=(0, 26, 51)),
}


def batch_prompts(name: str, V: int) -> np.ndarray:
    import hiplm
    bc = BATCH_CASES[name]
    return np.stack([hiplm.synth_prompt(SEED + 101 + s, bc["n_prompt"], V)
                     for s in range(bc["nseq"])])


def model_case(name: str):
    """(model dict, prompt, case tuple) of a MODEL_CASES entry, regenerated
    from the seed."""
    import hiplm
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = MODEL_CASES[name]
    types = hiplm.q4_k_m_types(L) if name in MODEL_TYPED else None
    if name in MIXTRAL_EXTRA:
        KH, window, theta = MIXTRAL_EXTRA[name]
        md = hiplm.synth_mixtral(SEED, L, E, H, KH, V, NE, K, EI, wt, 0.02, nstd, theta, window,
                                 types=types)
    else:
        md = hiplm.synth_olmoe(SEED, L, E, H, V, NE, K, EI, wt, 0.02, nstd, types=types)
    prompt = hiplm.synth_prompt(SEED, n_prompt, V)
    return md, prompt, MODEL_CASES[name]


def model_table(md: dict):
    import hiplm
    return hiplm.ptr_table(md) if md["arch"] == "olmoe" else hiplm.ptr_table_llama(md)


def model_digest(md: dict) -> str:
    h = hashlib.sha256()
    for k in ("token_embd", "output", "output_norm"):
        h.update(md[k].tobytes())
    for b in md["blk"]:
        for k in ("attn_norm", "q", "k", "v", "q_norm", "k_norm", "o", "ffn_norm", "router",
                  "gate", "up", "down"):
            if k in b:
                h.update(np.ascontiguousarray(b[k]).tobytes())
    return h.hexdigest()


def model_goldens(R, names):
    import hiplm
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    R.ref_olmoe_model_new.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, i32, vp]
    R.ref_olmoe_model_new.restype = vp
    R.ref_olmoe_model_run.argtypes = [vp, vp, sz, i32, sz, vp, vp]
    R.ref_olmoe_model_free.argtypes = [vp]
    R.ref_llama_model_new.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, sz, i32, vp]
    R.ref_llama_model_new.restype = vp
    R.ref_llama_model_run.argtypes = [vp, vp, sz, i32, sz, vp, vp]
    R.ref_llama_model_free.argtypes = [vp]
    R.ref_olmoe_model_new_typed.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, vp, vp]
    R.ref_olmoe_model_new_typed.restype = vp
    R.ref_llama_model_new_typed.argtypes = [sz, sz, sz, sz, sz, sz, sz, sz, sz, C.c_float, sz,
                                            vp, vp]
    R.ref_llama_model_new_typed.restype = vp
    for name in names:
        md, prompt, case = model_case(name)
        L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
        tab = model_table(md)
        fx = dict(seed=SEED, prompt=prompt, sha_model=model_digest(md), stride=stride)
        modes = (("dec", 0),) if name in MODEL_DEC_ONLY else (("dec", 0), ("pre", 1))
        ty = np.asarray([wt] * (2 + 6 * L), np.int32)
        if "types" in md:
            t = md["types"]
            ty = np.asarray([t["embd"], t["output"]] + [x for lt in t["layers"] for x in lt],
                            np.int32)
        for mode, prefill in modes:
            if md["arch"] == "olmoe":
                h = R.ref_olmoe_model_new_typed(L, E, H, V, NE, K, EI, Cx, md["theta"], p(ty),
                                                tab)
                run, free = R.ref_olmoe_model_run, R.ref_olmoe_model_free
            else:
                h = R.ref_llama_model_new_typed(L, E, H, md["KH"], V, NE, K, EI, Cx,
                                                md["theta"], md["window"], p(ty), tab)
                run, free = R.ref_llama_model_run, R.ref_llama_model_free
            lg = np.empty((n_gen + 1, V), np.float32)
            toks = np.empty(n_gen + 1, np.int32)
            run(h, p(prompt), n_prompt, prefill, n_gen, p(lg), p(toks))
            free(h)
            top = np.argsort(-lg, axis=1, kind="stable")[:, :MODEL_TOPN].astype(np.int32)
            fx[f"{mode}_tokens"] = toks
            fx[f"{mode}_logits"] = np.ascontiguousarray(lg[:, ::stride])
            fx[f"{mode}_top_ids"] = top
            fx[f"{mode}_top_logits"] = np.take_along_axis(lg, top, axis=1)
            assert np.isfinite(lg).all(), f"{name} [{mode}]: non-finite reference logits"
            print(f"model {name} [{mode}]: tokens {toks.tolist()}", flush=True)
        np.savez_compressed(os.path.join(HERE, f"model_{name}.npz"), **fx)
        if name in BATCH_CASES:
            batch_goldens(R, name, md, case, tab)
        del md


def batch_goldens(R, name, md, case, tab):
    """batch_<name>.npz: the reference's decode of each checked sequence of
    BATCH_CASES[name] alone (logits at every stride-th id, each step's top
    MODEL_TOPN, greedy tokens)."""
    L, E, H, V, NE, K, EI, Cx, wt, nstd, _, _, stride = case
    bc = BATCH_CASES[name]
    prompts = batch_prompts(name, V)
    fx = dict(seed=SEED, sha_model=model_digest(md), sha_prompts=sha(prompts), stride=stride,
              check=np.asarray(bc["check"], np.int32), nseq=bc["nseq"],
              n_prompt=bc["n_prompt"], n_gen=bc["n_gen"])
    for s in bc["check"]:
        if md["arch"] == "olmoe":
            h = R.ref_olmoe_model_new(L, E, H, V, NE, K, EI, Cx, md["theta"], wt, tab)
            run, free = R.ref_olmoe_model_run, R.ref_olmoe_model_free
        else:
            h = R.ref_llama_model_new(L, E, H, md["KH"], V, NE, K, EI, Cx, md["theta"],
                                      md["window"], wt, tab)
            run, free = R.ref_llama_model_run, R.ref_llama_model_free
        n_gen = bc["n_gen"]
        lg = np.empty((n_gen + 1, V), np.float32)
        toks = np.empty(n_gen + 1, np.int32)
        run(h, p(prompts[s]), bc["n_prompt"], 0, n_gen, p(lg), p(toks))
        free(h)
        assert np.isfinite(lg).all()
        top = np.argsort(-lg, axis=1, kind="stable")[:, :MODEL_TOPN].astype(np.int32)
        fx[f"s{s}_tokens"] = toks
        fx[f"s{s}_logits"] = np.ascontiguousarray(lg[:, ::stride])
        fx[f"s{s}_top_ids"] = top
        fx[f"s{s}_top_logits"] = np.take_along_axis(lg, top, axis=1)
        print(f"batch {name} sequence {s}: tokens {toks.tolist()}", flush=True)
    np.savez_compressed(os.path.join(HERE, f"batch_{name}.npz"), **fx)


def main():
    if not os.path.exists(REF_LIB):
        sys.exit(f"{REF_LIB} missing: run oracle/ref/build_ref.sh first")
    R = ref()
    if sys.argv[1:2] == ["model"]:
        model_goldens(R, sys.argv[2:] or list(MODEL_CASES))
        return
    if sys.argv[1:] == ["kquant"]:
        kquant_goldens(R)
        kq_layer_goldens(R)
        return
    qmat_goldens(R)
    if sys.argv[1:] == ["qmat"]:
        return
    kquant_goldens(R)
    kq_layer_goldens(R)

    # ---- quantizers -----------------------------------------------------
    blocks = quant_blocks()
    flat = np.ascontiguousarray(blocks.reshape(-1))
    q8 = np.empty(blocks.shape[0] * 34, np.uint8)
    q4 = np.empty(blocks.shape[0] * 18, np.uint8)
    R.ref_quantize_q8_0(p(flat), p(q8), flat.size)
    R.ref_quantize_q4_0(p(flat), p(q4), flat.size)
    np.savez(os.path.join(HERE, "quant.npz"), x=blocks, q8_0=q8, q4_0=q4)

    # ---- dots -------------------------------------------------------------
    dots = {}
    for wt, name in ((hipmoe.Q8_0, "q8_0"), (hipmoe.Q4_0, "q4_0")):
        for n in (256, 1024, 2048, 4096, 14336):
            rows = 4
            qm = hipmoe.synth_quant_matrix(SEED, 0x7000 + n + wt, 0.02, wt, rows, n)
            x = hipmoe.synth_normal(SEED, 0x7100 + n + wt, rows * n).reshape(rows, n)
            rb = hipmoe.row_bytes(wt, n)
            out = np.array([R.ref_dot(p(np.ascontiguousarray(x[r])),
                                      p(np.ascontiguousarray(qm[r * rb:(r + 1) * rb])), wt, n)
                            for r in range(rows)], np.float32)
            dots[f"{name}_{n}_sha_w"] = sha(qm)
            dots[f"{name}_{n}_sha_x"] = sha(x)
            dots[f"{name}_{n}_dot"] = out
    np.savez(os.path.join(HERE, "dot.npz"), seed=SEED, **dots)

    # ---- routing ----------------------------------------------------------
    for cfg, (wt, E, EI, NE, K, renorm, bias_std) in CONFIGS.items():
        T = 2048
        wr = hipmoe.synth_normal(SEED, hipmoe.lib().moe_stream_router(0), NE * E, 0.0,
                                 0.02).reshape(NE, E)
        bias = None
        if bias_std is not None:
            bias = hipmoe.synth_normal(SEED, hipmoe.lib().moe_stream_bias(0), NE, 0.0, bias_std)
        x = hipmoe.synth_normal(SEED, hipmoe.lib().moe_stream_input(777), T * E).reshape(T, E)
        lg = np.empty((T, NE), np.float32)
        pr = np.empty((T, NE), np.float32)
        ids = np.empty((T, K), np.uint32)
        w = np.empty((T, K), np.float32)
        R.ref_route(p(x), T, E, NE, p(wr), p(bias), K, renorm, p(lg), p(pr), p(ids), p(w))
        keep = 256
        np.savez(os.path.join(HERE, f"route_{cfg}.npz"), seed=SEED, input_call=777, T=T,
                 sha_x=sha(x), sha_router=sha(wr), sha_bias=sha(bias) if bias is not None else "",
                 logits=lg[:keep], probs=pr[:keep], ids=ids, w=w)
        dup = int(np.sum(ids[:, 0] == 0) if K > 1 else 0)
        print(f"route {cfg}: {T} tokens, tokens with expert 0 in slot 0: {dup}")

    # ---- one expert, one token ---------------------------------------------
    for wt, name in ((hipmoe.Q8_0, "q8_0"), (hipmoe.Q4_0, "q4_0")):
        E, EI = 2048, 1024
        g = hipmoe.synth_quant_matrix(SEED, 0x9001, 0.02, wt, EI, E)
        u = hipmoe.synth_quant_matrix(SEED, 0x9002, 0.02, wt, EI, E)
        d = hipmoe.synth_quant_matrix(SEED, 0x9003, 0.02, wt, E, EI)
        x = hipmoe.synth_normal(SEED, 0x9004, E)
        out = np.empty(E, np.float32)
        R.ref_fused_ffn(p(x), p(g), p(u), p(d), wt, E, EI, p(out))
        np.savez(os.path.join(HERE, f"ffn_{name}.npz"), seed=SEED, sha_gate=sha(g),
                 sha_up=sha(u), sha_down=sha(d), sha_x=sha(x), out=out)

    # ---- whole layers -----------------------------------------------------------
    for cfg, (wt, E, EI, NE, K, renorm, bias_std) in CONFIGS.items():
        T = 4 if NE == 64 else 2
        layer = hipmoe.synth_layer(SEED, 0, wt, E, EI, NE, 0.02, bias_std)
        x = hipmoe.synth_input(SEED, 0, T, E)
        gp, up_, dp = (hipmoe.expert_ptrs(layer[k]) for k in ("gate", "up", "down"))
        out_c = np.empty((T, E), np.float32)
        R.ref_moe_ffn_composed(p(x), p(out_c), T, p(layer["router"]), p(layer["bias"]), gp,
                               up_, dp, wt, E, EI, NE, K, renorm)
        if layer["bias"] is None:
            out_s = np.empty((T, E), np.float32)
            if renorm:
                R.ref_llama_moe_ffn(p(x), p(out_s), T, p(layer["router"]), gp, up_, dp, wt, E,
                                    EI, NE, K)
            else:
                R.ref_olmoe_moe_ffn(p(x), p(out_s), T, p(layer["router"]), p(layer["gate"]),
                                    p(layer["up"]), p(layer["down"]), wt, E, EI, NE, K)
            assert np.array_equal(out_s.view(np.uint32), out_c.view(np.uint32)), \
                f"{cfg}: composed loop differs from the reference's static moe_ffn"
            print(f"moe {cfg}: composed loop == static moe_ffn (bitwise)")
        np.savez(os.path.join(HERE, f"moe_{cfg}.npz"), seed=SEED, T=T,
                 sha_router=sha(layer["router"]), sha_gate=sha(layer["gate"]),
                 sha_up=sha(layer["up"]), sha_down=sha(layer["down"]), sha_x=sha(x),
                 sha_bias=sha(layer["bias"]) if layer["bias"] is not None else "", out=out_c)
        print(f"moe {cfg}: T={T} |out|={np.linalg.norm(out_c):.4f}")
        del layer


if __name__ == "__main__":
    main()
