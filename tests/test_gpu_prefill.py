"""GPU parity of the prompt prefill (hip_lm_prefill, and the prompt of
hip_lm_generate) through the C ABI, against the compiled reference's own
generate order (tests/golden/model_*.npz, "pre": one olmoe_prefill /
llama_prefill of the whole prompt, olmoe.c:504-508, llama.c:560-564, then
one olmoe_decode / llama_decode step per generated token):

  * the prefill's logits (the last prompt row's lm_head), then the decode
    steps after it, teacher-forced on the reference's tokens;
  * with every MoE layer in fp32 (hip_lm_set_moe_path GEMV), so that the
    prefill's own parts are held at 2e-5: the causal attention over a
    prompt of 200 rows (OLMoE's masked softmax) and of 240 rows (Mixtral's
    flash_attention with its sliding window of 200 masking inside the
    prefill), the q/k norms and RoPE of every row, the products on T rows;
    and two layers of the Mixtral-8x7B shape after a 1024-id prompt
    (sixteen query blocks, 8 kv heads of 4 query heads) at 1e-3 against
    the reference's decode of that prompt (the same values up to fp32
    rounding order);
  * with the default paths (the MoE layers on the grouped path at the
    prompt's token count, f16 operands) on 8-id prompts at 1e-3, where no
    prompt row's routing has a near-tie (ROUTE_GAP, as in the lockstep
    batch tests: past a near-tie the f16 layer may pick the other expert),
    the later steps' near-ties skipped as there; the full OLMoE shape's
    4-id prompts, whose MoE layers take the fp32 decode kernel;
  * generate (the prompt as one prefill, then replayed step graphs) gives
    the reference's tokens.
"""
import numpy as np
import pytest

import hiplm
import hipmoe
from common import ROUTE_GAP, generate_upto, model_case, rel_l2, routing_margins
from test_gpu_model import TIGHT, safe_steps, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    assert hipmoe.hip().device_count() >= 1, "no HIP device visible: GPU tests need an MI355X"


def prefill_vs_reference(name, tol, fp32_moe, check_margins=False):
    md, prompt, case, g = model_case(name)
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    key = "pre" if "pre_logits" in g.files else "dec"
    toks_ref = g[f"{key}_tokens"]
    route_ok = np.ones(n_gen + 1, bool)
    if check_margins:
        seq = np.concatenate([prompt, toks_ref[:-1]])
        rg = routing_margins(md, Cx, seq, 1)
        if rg[:n_prompt - 1].min() <= ROUTE_GAP:
            pytest.skip(f"{name}: a prompt row's routing has a near-tie "
                        f"({rg[:n_prompt - 1].min():.2e})")
        route_ok = rg[n_prompt - 1:] > ROUTE_GAP
    say(f"{name}: prefill of {n_prompt} ids, then {n_gen} steps against the reference's "
        f"{'generate' if key == 'pre' else 'decode'} order "
        f"({'fp32 MoE' if fp32_moe else 'default paths'})")
    M = hiplm.LmModel(md, Cx)
    try:
        if fp32_moe:
            M.set_moe_path(hipmoe.PATH_GEMV)
        safe = safe_steps(g[f"{key}_top_logits"])
        worst = 0.0
        nxt, lg = M.prefill(prompt)
        for s in range(n_gen + 1):
            if s > 0:
                nxt, lg = M.decode(int(toks_ref[s - 1]))
            err = rel_l2(lg[::stride], g[f"{key}_logits"][s])
            err_top = rel_l2(lg[g[f"{key}_top_ids"][s]], g[f"{key}_top_logits"][s])
            if not route_ok[s]:
                continue  # a routing near-tie downstream of the f16 prefill
            worst = max(worst, err, err_top)
            assert err <= tol and err_top <= tol, f"step {s}: rel L2 {err:.3e} / {err_top:.3e}"
            if safe[s]:
                assert nxt == int(toks_ref[s]), f"step {s}: pick {nxt}"
        say(f"{name}: prefill + {n_gen} steps, worst logit rel L2 {worst:.3e}")
        M.reset()
        toks, ms = M.generate(prompt, n_gen)
        rows = 1 if fp32_moe else n_prompt
        upto = generate_upto(md, Cx, prompt, toks_ref, g[f"{key}_top_logits"], rows)
        assert np.array_equal(toks[:upto], toks_ref[:upto]), (toks, toks_ref)
        say(f"{name}: generate (prefill + {n_gen} steps): {upto} tokens equal the reference's")
    finally:
        M.free()


@pytest.mark.parametrize("name", ["olmoe_prompt", "mixtral_window_prompt", "olmoe_small",
                                  "mixtral_small"])
def test_gpu_prefill_fp32_moe_vs_reference(name):
    prefill_vs_reference(name, TIGHT, True)


@pytest.mark.timeout(900)
def test_gpu_prefill_mixtral_layer_shape_1024_prompt_vs_reference():
    prefill_vs_reference("mixtral_2l_long", 1e-3, True)


@pytest.mark.parametrize("name", ["olmoe_small", "mixtral_small", "olmoe_long", "mixtral_long"])
def test_gpu_prefill_default_paths_vs_reference(name):
    prefill_vs_reference(name, 1e-3, False, check_margins=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["olmoe_full", "olmoe_full_long"])
def test_gpu_prefill_full_shape_decode_kernel_moe_vs_reference(name):
    """The full OLMoE-1B-7B shape's 4-id prompt: the prefill's MoE layers
    take the one-launch decode kernel (fp32) at these rows."""
    prefill_vs_reference(name, 1e-3, False)


def test_gpu_prefill_refuses_a_prompt_past_the_context():
    """The reference's prefill does not rotate the cache: a prompt longer
    than the free rows is refused (generate then runs it a step per id,
    rotating as the decode steps do)."""
    md, prompt, case, g = model_case("olmoe_small")
    L, E, H, V, NE, K, EI, Cx, wt, nstd, n_prompt, n_gen, stride = case
    M = hiplm.LmModel(md, Cx)
    try:
        long_prompt = np.resize(prompt, Cx + 1)
        with pytest.raises(hiplm.HipMoeError, match="do not fit"):
            M.prefill(long_prompt)
        nxt, _ = M.prefill(prompt)
        with pytest.raises(hiplm.HipMoeError, match="do not fit"):
            M.prefill(np.resize(prompt, Cx - n_prompt + 1))
        toks, _ = M.generate(np.resize(prompt, Cx + 4), 2)
        assert toks.size == 3
    finally:
        M.free()
