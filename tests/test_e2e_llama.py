"""A small Llama (random weights) with attn_implementation="flash_lab" against the same model on
SDPA, after the reference's tests/test_e2e_llama.py:1-123.

The reference runs Llama-3.2-1B-Instruct from the local Hugging Face cache; no checkpoint can be
downloaded here, so the models are built from local configs with seeded random weights and
prompts are random token ids: a 2-layer Llama of the same head layout (head_dim 128, GQA 4) for
the quick checks, and the full Llama-3.1-8B shape with an 8,192-token prompt (config L). The three
checks are the reference's: against an fp32 copy of the same weights, flash_lab's bf16 logits are
at most twice as far off as SDPA's; greedy generation follows SDPA's tokens until SDPA's own top
two logits are within two bf16 steps of each other; and with a static cache the decode step
compiles in one graph (fullgraph, HIP graphs) and still follows SDPA.
"""

import copy
import math

import pytest
import torch

transformers = pytest.importorskip("transformers")

import flash_lab.hf  # noqa: E402

NEW_TOKENS = 32
PROMPT_LENS = [37, 64, 129, 200]

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def small_llama():
    config = transformers.LlamaConfig(
        vocab_size=32000,
        hidden_size=1024,
        intermediate_size=2816,
        num_hidden_layers=2,
        num_attention_heads=8,
        num_key_value_heads=2,
        head_dim=128,
        max_position_embeddings=4096,
        rope_parameters={"rope_type": "default", "rope_theta": 500000.0},
        initializer_range=0.05,
        bos_token_id=1,
        eos_token_id=2,
    )
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = transformers.AutoModelForCausalLM.from_config(
            config, dtype=torch.bfloat16, attn_implementation="sdpa"
        )
    return model.eval()


NAME = flash_lab.hf.NAME


@pytest.fixture(scope="module")
def model():
    global NAME
    NAME = flash_lab.hf.register()  # the name transformers accepts for flash_lab's function
    return small_llama()


@pytest.fixture(scope="module")
def prompts():
    gen = torch.Generator().manual_seed(1)
    return [torch.randint(3, 32000, (1, n), generator=gen).cuda() for n in PROMPT_LENS]


def greedy(model, input_ids, impl, cache=None, new_tokens=None):
    """Greedy tokens and the logits of every step; a static cache also compiles the decode step,
    with fullgraph=True so that any graph break raises."""
    model.set_attn_implementation(impl)
    compile_kwargs = {}
    if cache is not None:
        compile_kwargs = dict(
            past_key_values=cache, compile_config=transformers.CompileConfig(fullgraph=True)
        )
    out = model.generate(
        input_ids,
        attention_mask=torch.ones_like(input_ids),
        max_new_tokens=new_tokens or NEW_TOKENS,
        min_new_tokens=new_tokens or NEW_TOKENS,
        do_sample=False,
        temperature=None,
        top_p=None,
        pad_token_id=model.config.eos_token_id,
        return_dict_in_generate=True,
        output_logits=True,
        **compile_kwargs,
    )
    return out.sequences[0, input_ids.shape[1]:], torch.stack(out.logits)[:, 0]


@pytest.fixture(scope="module")
def sdpa_runs(model, prompts):
    return [greedy(model, p, "sdpa") for p in prompts]


def assert_follows(run, reference) -> int | None:
    """The same tokens as the reference, up to a step where the reference's top two logits were
    within two bf16 steps. Returns that step, or None if all tokens match."""
    tokens, ref_tokens, ref_logits = run[0], reference[0], reference[1]
    differ = (tokens != ref_tokens).nonzero()
    if len(differ) == 0:
        return None
    step = int(differ[0])
    first, second = ref_logits[step].float().topk(2).values.tolist()
    tie = 2 * torch.finfo(torch.bfloat16).eps * 2 ** math.floor(math.log2(abs(first)))
    assert first - second <= tie, f"left the reference at token {step}, margin {first - second}"
    return step


@torch.no_grad()
def test_logit_error_at_most_twice_sdpa(model):
    print("e2e: logits vs fp32", flush=True)
    ids = torch.randint(3, 32000, (2, 300), generator=torch.Generator().manual_seed(0)).cuda()
    reference = copy.deepcopy(model).float()
    reference.set_attn_implementation("sdpa")
    want = reference(ids).logits.double()
    del reference
    errors = {}
    for impl in ("sdpa", NAME):
        model.set_attn_implementation(impl)
        errors[impl] = (model(ids).logits.double() - want).abs().max().item()
    assert errors[NAME] <= 2 * errors["sdpa"], errors


def test_greedy_generation_follows_sdpa(model, prompts, sdpa_runs):
    print("e2e: greedy generation", flush=True)
    for p, reference in zip(prompts, sdpa_runs, strict=True):
        assert_follows(greedy(model, p, NAME), reference)


def test_static_cache_decode_compiles_in_one_graph(model, prompts, sdpa_runs):
    # The decode step runs compiled (HIP graphs) on the static cache buffers. One cache size for
    # all prompts keeps it to a single compilation.
    print("e2e: compiled static-cache decode", flush=True)
    torch._dynamo.reset()
    cache = transformers.StaticCache(config=model.config, max_cache_len=256)
    for p, reference in zip(prompts, sdpa_runs, strict=True):
        cache.reset()
        assert_follows(greedy(model, p, NAME, cache), reference)


# Config L at full size: the Llama-3.1-8B shape (32 layers, hidden
# 4096, 32 query / 8 KV heads of 128, MLP 14336, vocab 128256, RoPE theta 5e5) with random bf16
# weights, B=1 and an 8,192-token random prompt. The reference checks its end-to-end model with
# the same two rules (tests/test_e2e_llama.py:94-135, bench/e2e.py:76-177): logits at the last
# prompt position at most twice as far from an fp32 copy of the weights as SDPA's, and greedy
# tokens from the compiled static-cache decode step that follow SDPA's up to a near-tie.
L_PROMPT = 8192
L_NEW_TOKENS = 256  # the configured generation length


@pytest.mark.timeout(900)
def test_config_l_llama_8b_shape():
    import e2e

    print("e2e L: building the 32-layer model", flush=True)
    name = flash_lab.hf.register()
    model = e2e.build_model(32, seed=0)
    ids = torch.randint(0, 128000, (1, L_PROMPT), generator=torch.Generator().manual_seed(0)).cuda()
    print("e2e L: fp32 reference logits", flush=True)
    want = e2e.reference_logits(model, {L_PROMPT: ids}, L_PROMPT)[L_PROMPT]
    model.set_attn_implementation("sdpa")
    err_sdpa = (e2e.last_logits(model, ids) - want).abs().max().item()
    model.set_attn_implementation(name)
    err = (e2e.last_logits(model, ids, L_PROMPT + L_NEW_TOKENS) - want).abs().max().item()
    print(f"e2e L: logit error {err:.4g} (sdpa {err_sdpa:.4g})", flush=True)
    assert err <= 2 * err_sdpa + 1e-3, (err, err_sdpa)

    print("e2e L: sdpa greedy tokens", flush=True)
    reference = greedy(model, ids, "sdpa", new_tokens=L_NEW_TOKENS)
    print("e2e L: compiled static-cache decode", flush=True)
    torch._dynamo.reset()
    cache = transformers.StaticCache(config=model.config, max_cache_len=L_PROMPT + L_NEW_TOKENS)
    step = assert_follows(greedy(model, ids, name, cache, new_tokens=L_NEW_TOKENS), reference)
    print(f"e2e L: tokens follow sdpa (first difference: {step})", flush=True)
    del model, cache
    torch._dynamo.reset()
    torch.cuda.empty_cache()
