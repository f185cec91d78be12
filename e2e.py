"""End-to-end generation on a Llama-3.1-8B-shaped model (random weights), by attention implementation.

    python e2e.py                                   # config L: 32 layers, prompts 512 and 8192
    python e2e.py --layers 4 --prompt-lens 512 --new-tokens 64 --runs 1

The reference's bench/e2e.py (bench/e2e.py:1-263) times generate() on a downloaded Llama
checkpoint. No checkpoint can be downloaded here, so the model is built from a local LlamaConfig of
Llama-3.1-8B's shape (32 layers, hidden 4096, 32 query / 8 KV heads of 128, MLP 14336, vocab
128256, RoPE theta 5e5) with random bf16 weights, initialised on the GPU. Everything else follows
the reference:

* each implementation generates --new-tokens greedy tokens from the same random prompt with a
  static KV cache, so generate() compiles the decode step (torch.compile, fullgraph, HIP graphs)
  for every implementation alike; untimed warmup runs pay for the compilation;
* a streamer timestamps every step: the first gap is the time to first token (prefill), the rest
  are decode steps;
* before timing, each implementation's logits at the last prompt position (through the static
  cache, as generate() runs it) are checked against an fp32 copy of the same weights with the
  kernel benchmarks' rule, at most twice SDPA's bf16 error plus 1e-3; an implementation that fails
  is recorded as incorrect and not timed. Generated tokens are compared with the first
  implementation's (random weights give near-ties, so a difference is reported, not failed).

"flash_lab" is the gfx950 kernels of this repository through flash_lab.hf (prefill:
attention_mma_pipelined, decode: decode_splitkv); "sdpa" is PyTorch's scaled_dot_product_attention
as transformers calls it. One JSON line at the end carries every result and the GPU clocks sampled
while each implementation ran.
"""

from __future__ import annotations

import argparse
import copy
import gc
import json
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "flash-attention-lab_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

FLOOR_BF16 = 1e-3  # the reference's bench/run.py:35 floor for bf16
IMPLS = ["sdpa", "flash_lab"]


def llama_config(layers: int):
    """Llama-3.1-8B's architecture (its config.json values) as a local LlamaConfig."""
    from transformers import LlamaConfig

    return LlamaConfig(
        vocab_size=128256,
        hidden_size=4096,
        intermediate_size=14336,
        num_hidden_layers=layers,
        num_attention_heads=32,
        num_key_value_heads=8,
        head_dim=128,
        max_position_embeddings=131072,
        rms_norm_eps=1e-5,
        rope_parameters={"rope_type": "default", "rope_theta": 500000.0},
        bos_token_id=128000,
        eos_token_id=128001,
        tie_word_embeddings=False,
    )


def build_model(layers: int, seed: int):
    import torch
    from transformers import AutoModelForCausalLM

    torch.manual_seed(seed)
    with torch.device("cuda"):
        model = AutoModelForCausalLM.from_config(
            llama_config(layers), dtype=torch.bfloat16, attn_implementation="sdpa"
        )
    return model.eval()


class StepClock:
    """generate()'s streamer: called once with the prompt, then once per step's new tokens."""

    def __init__(self, progress_every: int = 0):
        self.times: list[float] = []
        self.progress_every = progress_every

    def put(self, value):
        import torch

        torch.cuda.synchronize()
        self.times.append(time.perf_counter())
        n = len(self.times) - 1
        if self.progress_every and n and n % self.progress_every == 0:
            print(f"  step {n}", file=sys.stderr, flush=True)

    def end(self):
        pass


def generate(model, input_ids, new_tokens: int, eos_id: int, progress_every: int = 0):
    import torch
    from transformers import CompileConfig

    clock = StepClock(progress_every)
    out = model.generate(
        input_ids,
        attention_mask=torch.ones_like(input_ids),
        max_new_tokens=new_tokens,
        min_new_tokens=new_tokens,
        do_sample=False,
        temperature=None,
        top_p=None,
        pad_token_id=eos_id,
        cache_implementation="static",
        compile_config=CompileConfig(fullgraph=True),
        streamer=clock,
    )
    gaps = [(b - a) * 1e3 for a, b in zip(clock.times, clock.times[1:])]
    return out[:, input_ids.shape[1]:], gaps


def last_logits(model, input_ids, cache_len: int | None = None):
    """Logits at the last prompt position, through a static cache of cache_len rows (the path
    generate() takes) or with no cache."""
    import torch
    from transformers import StaticCache

    kwargs = {}
    if cache_len is not None:
        kwargs["past_key_values"] = StaticCache(config=model.config, max_cache_len=cache_len)
        kwargs["cache_position"] = torch.arange(input_ids.shape[1], device=input_ids.device)
    with torch.no_grad():
        return model(input_ids, logits_to_keep=1, **kwargs).logits[:, -1].double()


def reference_logits(model, prompts: dict, max_len: int) -> dict:
    """fp32 logits of the same weights (an fp32 copy, SDPA) for the prompts up to max_len."""
    import torch

    ref = copy.deepcopy(model).float()
    ref.set_attn_implementation("sdpa")
    out = {n: last_logits(ref, ids) for n, ids in prompts.items() if n <= max_len}
    del ref
    gc.collect()
    torch.cuda.empty_cache()
    return out


def first_difference(tokens, reference) -> int | None:
    differ = (tokens != reference).any(dim=0).nonzero()
    return int(differ[0]) if len(differ) else None


def bench_impl(model, impl, prompts, args, eos_id, checks, reference_tokens, clocks) -> list[dict]:
    import torch

    model.set_attn_implementation(args.registered.get(impl, impl))
    torch._dynamo.reset()
    results = []
    for prompt_len, input_ids in prompts.items():
        config = {"prompt_len": prompt_len, "batch": args.batch, "new_tokens": args.new_tokens}
        print(f"{impl} prompt {prompt_len}: check", flush=True)
        if prompt_len in checks:
            want, err_torch, margin = checks[prompt_len]
            got = last_logits(model, input_ids, prompt_len + args.new_tokens)
            check = {
                "max_logit_err_vs_fp32": (got - want).abs().max().item(),
                "max_logit_err_torch_vs_fp32": err_torch,
                "fp32_top2_margin": margin,
            }
            if not check["max_logit_err_vs_fp32"] <= 2 * err_torch + FLOOR_BF16:
                results.append({"config": config, "impl": impl, "status": "incorrect", **check})
                print(f"{impl} prompt {prompt_len}: incorrect {check}", flush=True)
                continue
        else:
            check = {"logit_check": "skipped: prompt longer than --check-max-len"}
        for i in range(args.n_warmup):
            print(f"{impl} prompt {prompt_len}: warmup {i + 1}", flush=True)
            generate(model, input_ids, args.new_tokens, eos_id, progress_every=64)
        start = time.time()
        runs = []
        for i in range(args.runs):
            print(f"{impl} prompt {prompt_len}: run {i + 1}", flush=True)
            runs.append(generate(model, input_ids, args.new_tokens, eos_id))
        gpu = clocks.window(start, time.time())
        tokens = runs[0][0]
        reference = reference_tokens.setdefault(prompt_len, (impl, tokens))
        ttft = [gaps[0] for _, gaps in runs]
        steps = [step for _, gaps in runs for step in gaps[1:]]
        step_ms = statistics.median(steps)
        result = {
            "config": config,
            "impl": impl,
            "status": "ok",
            "ttft_ms": {"median": statistics.median(ttft), "min": min(ttft), "max": max(ttft)},
            "decode_step_ms": {
                "median": step_ms,
                "p10": statistics.quantiles(steps, n=10)[0],
                "p90": statistics.quantiles(steps, n=10)[-1],
            },
            "decode_tokens_per_s": args.batch * 1e3 / step_ms,
            "gpu_during_timing": gpu,
            **check,
            "compared_with": reference[0],
            "first_token_difference": first_difference(tokens, reference[1]),
        }
        results.append(result)
        print(
            f"{impl:<10} prompt {prompt_len:>6}: ttft {result['ttft_ms']['median']:8.1f} ms, "
            f"decode {step_ms:6.2f} ms/step ({result['decode_tokens_per_s']:7.1f} tokens/s)",
            flush=True,
        )
    return results


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--layers", type=int, default=32)
    parser.add_argument("--impls", default=",".join(IMPLS))
    parser.add_argument("--prompt-lens", default="512,8192")
    parser.add_argument("--batch", type=int, default=1)
    parser.add_argument("--new-tokens", type=int, default=256)
    parser.add_argument("--n-warmup", type=int, default=1)
    parser.add_argument("--runs", type=int, default=2)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--check-max-len", type=int, default=8192)
    return parser.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    import torch

    import flash_lab
    import flash_lab.hf
    from flash_lab import ops
    from flash_lab.observe import ClockSampler

    if not torch.cuda.is_available():
        print("e2e.py needs a GPU", file=sys.stderr)
        return 2
    if not ops.HAS_EXTENSION:
        raise RuntimeError(f"the HIP library did not load: {ops.EXTENSION_ERROR}")
    torch.backends.cuda.matmul.allow_tf32 = False
    # transformers 5 will not select a function named "flash_lab" (see flash_lab.hf.register).
    args.registered = {"flash_lab": flash_lab.hf.register()}

    print(f"building a {args.layers}-layer Llama-3.1-8B-shaped model (random bf16 weights)", flush=True)
    model = build_model(args.layers, args.seed)
    vocab_ids = min(model.config.vocab_size, 128000)  # below Llama 3's special tokens
    gen = torch.Generator().manual_seed(args.seed)
    prompts = {
        int(n): torch.randint(0, vocab_ids, (args.batch, int(n)), generator=gen).cuda()
        for n in args.prompt_lens.split(",")
    }
    eos_id = model.config.eos_token_id

    print("fp32 reference logits", flush=True)
    reference = reference_logits(model, prompts, args.check_max_len)
    checks = {}
    for n, ids in prompts.items():
        if n not in reference:
            continue
        model.set_attn_implementation("sdpa")
        err_torch = (last_logits(model, ids) - reference[n]).abs().max().item()
        top2 = reference[n].topk(2, dim=-1).values
        checks[n] = (reference[n], err_torch, (top2[:, 0] - top2[:, 1]).min().item())

    results = []
    reference_tokens: dict = {}
    with ClockSampler() as clocks:
        for impl in args.impls.split(","):
            results += bench_impl(
                model, impl, prompts, args, eos_id, checks, reference_tokens, clocks
            )
            torch.cuda.empty_cache()

    out = {
        "suite": "e2e_llama",
        "model": f"Llama-3.1-8B-shaped, {args.layers} layers, random bf16 weights (seed {args.seed})",
        "data": "synthetic: uniform random prompt ids, random weights (no checkpoint offline)",
        "dtype": "bf16",
        "cache": "static",
        "n_warmup": args.n_warmup,
        "runs": args.runs,
        "device": torch.cuda.get_device_name(0),
        "results": results,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
