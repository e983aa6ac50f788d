"""GPU parity of attention over caches longer than one 64-row chunk, through
the C ABI (include/hip_lm.h), against the compiled reference's own decode
(tests/golden/model_*_long.npz, batch_*_long.npz):

  * k_lm_attn splits the cache rows [lo, size] into chunks of 64 and merges
    the chunks' partials by their maxima.  One sequence's grid (kv heads x
    chunks) is resident at once, so chunk 0 merges, polling the others'
    tagged partials; a lockstep batch whose grid is larger than three
    workgroups per CU merges in the last chunk to count in.  Both forms run
    here with four chunks and more;
  * the reduced OLMoE (masked softmax over AT rows, olmoe.c:286-320) runs
    308 positions in a 256-row cache through one kvcache_rotate; the reduced
    Mixtral (flash_attention's 64-row blocks, nn.c:570-641) has a sliding
    window of 200 rows that crosses chunk boundaries as it moves, with
    grouped-query heads (16 / 4);
  * the full OLMoE-1B-7B shape over 300 positions (five chunks), and two
    layers of the Mixtral-8x7B shape after a 1024-token prompt (seventeen
    chunks, eight kv heads of four query heads): the lengths the benchmarks
    run;
  * a sliding window of at least the context: the steps until the cache is
    full run, the next one is refused (the reference's kvcache_rotate keeps
    every row there and its next step writes past the cache);
  * step graphs captured before a lockstep batch reallocated the shared MoE
    scratch are captured again.
Logits within 2e-5 relative L2 of the reference's on the reduced models
(fp32 in another summation order), 1e-3 where a lockstep batch's MoE layer
takes the grouped path (f16 operands) and at the full shapes; the greedy
pick equal wherever the reference's top two logits are apart; routing
bit-exact at sampled steps.
"""
import ctypes as C

import numpy as np
import pytest

import hiplm
from common import (ROUTE_GAP, SEED, batch_case, generate_upto, model_case, rel_l2,
                    routing_margins)
from test_gpu_model import TIGHT, safe_steps, say, teacher_forced

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    import hipmoe
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


def merge_form(KH, nact, nseq):
    import hipmoe
    f = hipmoe.lib().lm_attn_merge_form
    f.argtypes = [C.c_int, C.c_int, C.c_int]
    f.restype = C.c_int
    return f(KH, nact, nseq)


def test_gpu_model_olmoe_long_cache_vs_reference():
    md, _, case, _ = model_case("olmoe_long")
    assert merge_form(md["H"], 4, 1) == 2
    teacher_forced("olmoe_long", TIGHT, route_steps=(0, 70, 200, 255, 256, 300))


def test_gpu_model_mixtral_long_cache_window_vs_reference():
    md, _, case, _ = model_case("mixtral_long")
    assert merge_form(md["KH"], 4, 1) == 2
    teacher_forced("mixtral_long", TIGHT, route_steps=(0, 130, 210, 256, 300))


@pytest.mark.timeout(900)
def test_gpu_model_full_shape_long_vs_reference():
    teacher_forced("olmoe_full_long", 1e-3, route_steps=(150, 299))


@pytest.mark.timeout(900)
def test_gpu_model_mixtral_layer_shape_long_prompt_vs_reference():
    md, _, case, _ = model_case("mixtral_2l_long")
    assert merge_form(md["KH"], 17, 1) == 2
    teacher_forced("mixtral_2l_long", 1e-3, route_steps=(1023, 1050), fp32_generate=True)


def batch_vs_reference(name, tol):
    """Every sequence of the fixture's batch in lockstep; the checked ones
    teacher-forced on the reference's tokens (the others on seeded ids),
    their logits against the reference's decode of that sequence alone;
    then generate from fresh caches gives the checked sequences' tokens.

    The MoE layer at T = nseq takes the grouped path, whose f16 operands
    move a layer's output by ~5e-4 relative L2; where a later layer's
    routing has two experts within ROUTE_GAP (relative) of each other at
    the top-k boundary, that is enough to pick the other one (the mixtral
    fixture's sequence 0 has experts 7 and 1 at 0.183083 / 0.183081 in layer
    1 at step 3), and the step's logits follow another expert.  Those steps
    are skipped here, as steps whose top two logits tie are for the pick;
    the layer on its own is checked against the oracle at every input."""
    md, prompts, bc, g = batch_case(name)
    L, E, H, V, NE, K, EI, Cx, wt, nstd, _, _, stride = bc["case"]
    S, n_prompt, n_gen = int(g["nseq"]), int(g["n_prompt"]), int(g["n_gen"])
    check = [int(s) for s in g["check"]]
    KH = md.get("KH", H)
    nact = (n_prompt + n_gen + 63) // 64
    assert merge_form(KH, nact, S) == 1, "the grid must be larger than the device holds"
    feed = np.stack([hiplm.synth_prompt(SEED + 9001 + s, n_gen, V) for s in range(S)])
    for s in check:
        feed[s] = g[f"s{s}_tokens"][:-1]
    seqs = np.concatenate([prompts, feed], axis=1)
    say(f"{name}: routing margins of the checked sequences (model oracle)")
    route_ok = {s: routing_margins(md, Cx, seqs[s], n_prompt) > ROUTE_GAP for s in check}
    rows = min(max(1, 2048 // n_prompt), S) * n_prompt
    nskip = sum(int((~v).sum()) for v in route_ok.values())
    assert nskip <= len(check) * (n_gen + 1) // 4, "too few steps without a routing near-tie"
    say(f"{name}: {S} sequences in lockstep, {n_prompt} prompt ids + {n_gen} steps, "
        f"grid {KH} x {nact} x {S} (last chunk to count in merges)")
    M = hiplm.LmModel(md, Cx)
    Bt = hiplm.LmBatch(M, S)
    try:
        worst = 0.0
        for i in range(seqs.shape[1]):
            nxt, lg = Bt.decode(seqs[:, i])
            st = i - (n_prompt - 1)
            if st < 0:
                continue
            for s in check:
                err = rel_l2(lg[s, ::stride], g[f"s{s}_logits"][st])
                top = lg[s, g[f"s{s}_top_ids"][st]]
                err_top = rel_l2(top, g[f"s{s}_top_logits"][st])
                if not route_ok[s][st]:
                    say(f"  sequence {s} step {st}: routing near-tie, rel L2 {err:.3e} "
                        f"(not asserted)")
                    continue
                worst = max(worst, err, err_top)
                assert err <= tol and err_top <= tol, \
                    f"sequence {s} step {st}: rel L2 {err:.3e} / {err_top:.3e}"
                if safe_steps(g[f"s{s}_top_logits"])[st]:
                    assert nxt[s] == g[f"s{s}_tokens"][st], f"sequence {s} step {st}"
        say(f"{name}: teacher-forced, worst logit rel L2 {worst:.3e} "
            f"({nskip} routing near-ties skipped)")
        Bt.reset()
        toks, ms = Bt.generate(prompts, n_gen)
        for s in check:
            # the prompts as prefills (grouped-path MoE layers at these rows)
            upto = generate_upto(md, Cx, prompts[s], g[f"s{s}_tokens"],
                                 g[f"s{s}_top_logits"], rows)
            assert np.array_equal(toks[s, :upto], g[f"s{s}_tokens"][:upto]), \
                (s, toks[s], g[f"s{s}_tokens"])
        say(f"{name}: generate {n_gen} steps x {S} sequences: checked tokens equal the "
            f"reference's, {ms:.2f} ms")
    finally:
        Bt.free()
        M.free()


@pytest.mark.timeout(600)
def test_gpu_batch_olmoe_long_last_to_arrive_merge_vs_reference():
    batch_vs_reference("olmoe_long", 1e-3)


@pytest.mark.timeout(600)
def test_gpu_batch_mixtral_long_last_to_arrive_merge_vs_reference():
    batch_vs_reference("mixtral_long", 1e-3)


def test_gpu_model_window_at_context_refuses_the_step_past_a_full_cache():
    """A sliding window of at least the context: the steps until the cache
    is full run (the window never masks there); the step after is refused,
    for decode and generate alike (generate before any launch)."""
    md, prompt, case, g = model_case("mixtral_small")
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    md = dict(md)
    md["window"] = Cx
    M = hiplm.LmModel(md, Cx)
    try:
        seq = list(prompt) + list(g["dec_tokens"][:-1])
        for i in range(Cx):
            M.decode(int(seq[i]))
        with pytest.raises(hiplm.HipMoeError, match="keep every row"):
            M.decode(int(seq[Cx]))
        M.reset()
        with pytest.raises(hiplm.HipMoeError, match="keep every row"):
            M.generate(prompt, Cx)
        M.reset()
        toks, _ = M.generate(prompt, Cx - len(prompt))
        assert toks.size == Cx - len(prompt) + 1
    finally:
        M.free()


def test_gpu_model_generate_after_a_batch_grew_the_moe_scratch():
    """A lockstep batch reserves the shared MoE layers' scratch for its
    sequences, which reallocates it; the model's step graphs captured by an
    earlier generate name the freed buffers and are captured again, so a
    later generate gives the same tokens as the first (the runs are
    deterministic: the grouped path's rows do not depend on their order)."""
    md, prompt, case, g = model_case("olmoe_small")
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    M = hiplm.LmModel(md, Cx)
    try:
        first, _ = M.generate(prompt, n_gen)
        Bt = hiplm.LmBatch(M, 24)
        try:
            nxt, _ = Bt.decode(np.full(24, int(prompt[0]), np.int32))
        finally:
            Bt.free()
        M.reset()
        toks, _ = M.generate(prompt, n_gen)
        assert np.array_equal(toks, first)
        say("olmoe_small: generate, a 24-sequence batch, generate again: the same tokens")
    finally:
        M.free()
