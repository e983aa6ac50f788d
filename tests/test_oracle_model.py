"""Pins the model oracle (oracle/lm_oracle.c: the OLMoE and Mixtral decode
steps around the MoE oracle) against the compiled reference before it is
trusted as the checker of the GPU model: per-step logits and greedy tokens of
the reference's own olmoe_decode / llama_decode (driven by
oracle/ref/ref_olmoe.c and ref_llama.c over seeded weights,
tests/golden/model_*.npz) bit for bit, on reduced models with non-unit norms
that run past their context (kvcache_rotate; Mixtral's keeps its sliding
window, and its flash_attention masks), at the full OLMoE shape and on two
layers of the Mixtral-8x7B shape; with per-tensor block types (Q4_K_M's
mix of Q4_K and Q6_K); and the reference's generate order (one prefill of
the prompt) within fp32 rounding."""
import numpy as np
import pytest

import hiplm
import oracle
from common import bits, model_case, rel_l2


def _run(name):
    md, prompt, case, g = model_case(name)
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    tab = hiplm.ptr_table(md) if md["arch"] == "olmoe" else hiplm.ptr_table_llama(md)
    m = oracle.OlmoeModel(md, Cx, tab)
    try:
        toks, lg = m.run(prompt, n_gen)
    finally:
        m.free()
    return toks, lg, g, stride


def test_model_oracle_matches_reference_decode_bits_small():
    toks, lg, g, stride = _run("olmoe_small")
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))
    # the reference's own generate (prefill of the prompt) lands within fp32 rounding
    assert np.array_equal(toks, g["pre_tokens"])
    for s in range(lg.shape[0]):
        assert rel_l2(lg[s], g["pre_logits"][s]) <= 1e-5


@pytest.mark.slow
def test_model_oracle_matches_reference_decode_bits_full_shape():
    toks, lg, g, stride = _run("olmoe_full")
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))
    top = np.take_along_axis(lg, g["dec_top_ids"].astype(np.int64), axis=1)
    assert np.array_equal(bits(top), bits(g["dec_top_logits"]))
    for s in range(lg.shape[0]):
        assert rel_l2(lg[s, ::stride], g["pre_logits"][s]) <= 1e-5


def test_model_oracle_routing_trace_is_the_layer_oracle():
    """The per-layer routing the model oracle reports is the MoE oracle's
    routing of the reported router input (a trace the GPU test relies on)."""
    md, prompt, case, g = model_case("olmoe_small")
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    tab = hiplm.ptr_table(md)
    m = oracle.OlmoeModel(md, Cx, tab)
    try:
        for t in prompt[:3]:
            nxt, lg, (mi, ids, w) = m.decode(int(t), trace=True)
            for l in range(L):
                b = md["blk"][l]
                lay = dict(router=b["router"], gate=b["gate"], up=b["up"], down=b["down"],
                           wtype=wt, E=E, EI=EI, NE=NE)
                _, oids, ow, _, _ = oracle.moe_ffn(mi[l:l + 1], lay, K, False, None)
                assert np.array_equal(ids[l], oids[0]) and np.array_equal(bits(w[l]), bits(ow[0]))
    finally:
        m.free()


def test_model_oracle_matches_reference_decode_bits_mixtral_small():
    toks, lg, g, stride = _run("mixtral_small")
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))
    assert np.array_equal(toks, g["pre_tokens"])
    for s in range(lg.shape[0]):
        assert rel_l2(lg[s], g["pre_logits"][s]) <= 1e-5


@pytest.mark.slow
def test_model_oracle_matches_reference_decode_bits_mixtral_layer_shape():
    toks, lg, g, stride = _run("mixtral_2l")
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))
    top = np.take_along_axis(lg, g["dec_top_ids"].astype(np.int64), axis=1)
    assert np.array_equal(bits(top), bits(g["dec_top_logits"]))


# --------------------------------------------------------------------------
# caches longer than one 64-row attention block
# --------------------------------------------------------------------------

def _check_long(name):
    toks, lg, g, stride = _run(name)
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))
    top = np.take_along_axis(lg, g["dec_top_ids"].astype(np.int64), axis=1)
    assert np.array_equal(bits(top), bits(g["dec_top_logits"]))
    assert np.array_equal(toks, g["pre_tokens"])
    for s in range(lg.shape[0]):
        assert rel_l2(lg[s, ::stride], g["pre_logits"][s]) <= 1e-5


def test_model_oracle_matches_reference_decode_bits_olmoe_long_cache():
    """308 positions in a 256-row context: OLMoE's masked softmax over up to
    256 cache rows, one kvcache_rotate (keeps 128), RoPE positions restarting
    at the cache size after it (olmoe.c:509-520)."""
    _check_long("olmoe_long")


def test_model_oracle_matches_reference_decode_bits_mixtral_long_cache():
    """The multi-block flash_attention (nn.c:570-641: up to four 64-row
    blocks, rescaled by each block's maximum) with a sliding window of 200
    that straddles block boundaries, grouped-query heads (16 / 4), and one
    kvcache_rotate that keeps the window."""
    _check_long("mixtral_long")


@pytest.mark.parametrize("name", ["olmoe_long", "mixtral_long"])
def test_batch_fixture_prompts_regenerate(name):
    """The lockstep-batch fixtures' prompts and model are the seeded ones."""
    import hashlib
    from common import batch_case
    md, prompts, bc, g = batch_case(name)
    assert hashlib.sha256(np.ascontiguousarray(prompts).tobytes()).hexdigest() == \
        str(g["sha_prompts"])


def test_model_oracle_matches_reference_batch_sequence_long_prompt():
    """One checked sequence of the lockstep-batch fixture (a 200-id prompt,
    then greedy steps) decoded by the model oracle alone equals the
    reference's decode bit for bit."""
    from common import batch_case
    md, prompts, bc, g = batch_case("olmoe_long")
    s = int(g["check"][-1])
    L, E, H, V, NE, K, EI, Cx, wt, nstd, _, _, stride = bc["case"]
    m = oracle.OlmoeModel(md, Cx, hiplm.ptr_table(md))
    try:
        toks, lg = m.run(prompts[s], int(g["n_gen"]))
    finally:
        m.free()
    assert np.array_equal(toks, g[f"s{s}_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g[f"s{s}_logits"]))


@pytest.mark.parametrize("name", ["olmoe_prompt", "mixtral_window_prompt"])
def test_model_oracle_matches_reference_long_prompt(name):
    """A 200-id prompt (OLMoE) and a 240-id prompt under a 200-row sliding
    window (Mixtral): the decode order bit for bit, and the reference's
    generate order (one prefill of the whole prompt, whose flash_attention
    masks rows outside the window, nn.c:597-603) within fp32 rounding."""
    _check_long(name)


@pytest.mark.parametrize("name", ["olmoe_q4km", "mixtral_q4km"])
def test_model_oracle_matches_reference_q4_k_m(name):
    """Per-tensor block types as a Q4_K_M GGUF mixes them (hiplm.q4_k_m_types:
    Q4_K, the output and layer 1's attn_v and experts' down Q6_K): the
    embedding row through dequant_row, every product through Q8_K
    activations (dot_q8_quant, quant.c:627-666), the K-quant experts; every
    position of a one-id prompt and 47 steps, past the context, bit for
    bit."""
    toks, lg, g, stride = _run(name)
    assert np.array_equal(toks, g["dec_tokens"])
    assert np.array_equal(bits(lg[:, ::stride]), bits(g["dec_logits"]))

