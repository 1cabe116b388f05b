"""Batched verification and greedy speculative decoding on an MI355X
(the checks of tests/speculative_check.py, which also run on the mock HIP
runtime in tests/test_speculative.py), through this repository's compute API
on the gfx950 kernels:

- nya_compute_plan_verify over chunks of 5 (the vocabulary product on the
  small-N kernels), 20 and 33 tokens (the prefill GEMM) gives the logits of
  one plan_token per token within the engine's logit bound
  (backend/tests/test_inference.c:214-219) and its greedy choices; earlier
  positions run again follow the new tokens;
- nya_compute_generate_greedy emits the target's serial greedy decode with
  drafts that disagree, agree, or agree at some positions only (proposals
  both accepted and rejected), and without a draft;
- nya_compute_generate_sampled emits the tokens of the engine's speculative
  sampling loop restated (oracle/speculative.py, pinned to the engine in
  tests/test_sampling_oracle.py) fed by plans making the same calls, with
  drafts of other weights, the target's own, and none; the first token
  follows the target's distribution over 400 seeds and top-p below the
  leading probability keeps only the leading token
  (backend/tests/test_generation.c:345-387);
- the device greedy choice skips suppressed tokens."""
import pytest

from fyodor_amd import Q4_K, Q6_K, Q8_0
from fyodor_amd import model as fm
from speculative_check import (first_token_follows_target, generation_equals_target_decode,
                               sampled_generation_matches_oracle, suppressed_tokens_are_skipped, verify_matches_steps)

pytestmark = pytest.mark.gpu

PROMPT = [5, 17, 200, 3, 42]


@pytest.fixture(autouse=True)
def rocm_env(monkeypatch):
    from fyodor_amd import KERNEL_LIBRARY
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(KERNEL_LIBRARY))
    for v in ("NYA_ROCM_HIP_LIBRARY", "NYA_ROCM_CACHE_MIB"):
        monkeypatch.delenv(v, raising=False)


@pytest.mark.parametrize("chunk", [5, 20, 33])
def test_verify_matches_serial_steps(chunk):
    shape = fm.LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=96, vocabulary=1000,
                          seed=3)
    tokens = [(i * 37 + 11) % shape.vocabulary for i in range(2 * chunk + 3)]
    worst = verify_matches_steps(shape, tokens, chunk)
    print(f"chunk {chunk}: worst scaled logit error {worst:.3g}", flush=True)


@pytest.mark.parametrize("draft", ["other", "same", "swapped", "none"])
def test_generation_equals_target_decode(draft):
    types = {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K}
    target = fm.LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=96, vocabulary=1000,
                           types=types, seed=5 if draft == "swapped" else 3)
    other = fm.LlamaShape(embedding=256, heads=4, kv_heads=2, hidden=512, blocks=1, context=96, vocabulary=1000,
                          types={**types, "output": Q8_0}, seed=11)
    if draft == "swapped":
        # This shape's decode alternates two tokens (seed 5): a draft with
        # one of them swapped is right at every other position.
        target = fm.LlamaShape(context=96, types=types, seed=5)
    runs = generation_equals_target_decode(target, other if draft == "other" else None, PROMPT, limit=24,
                                           windows=(1, 4, 8), same_draft=draft == "same", swap=draft == "swapped")
    print(draft, runs, flush=True)
    if draft == "swapped":
        assert any(0 < stats["accepted"] < stats["draft_tokens"] for _, stats in runs), runs


def test_suppressed_tokens_are_skipped():
    suppressed_tokens_are_skipped(fm.LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=2, context=32,
                                                vocabulary=1000, seed=3), PROMPT)


SAMPLED_CASES = [(4, 1.0, 1.0, 0, 1), (1, 0.7, 0.9, 0, 7), (8, 1.5, 1.0, 5, 123), (5, 1.0, 0.5, 40, 99),
                 (16, 0.5, 1.0, 0, 3)]


@pytest.mark.parametrize("draft", ["other", "same", "none"])
def test_sampled_generation_matches_oracle(draft):
    types = {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K}
    target = fm.LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=96, vocabulary=1000,
                           types=types, seed=3)
    runs = sampled_generation_matches_oracle(target, draft, PROMPT, 24, SAMPLED_CASES)
    print(draft, runs, flush=True)
    if draft == "same":
        # The target's weights on the same kernels: equal distributions.
        assert all(r["accepted"] == r["draft_tokens"] for r in runs), runs


def test_sampled_first_token_distribution():
    p, count, accepted = first_token_follows_target(fm.LlamaShape(context=64, seed=3), PROMPT[:1], runs=400)
    print(f"p {p:.4f}: {count} of 400 leading, {accepted} accepted", flush=True)


GEMMA = dict(embedding=512, heads=8, kv_heads=4, width=256, local_width=128, hidden=1024, window=16, context=96,
             vocabulary=1000)


@pytest.mark.parametrize("chunk", [5, 33])
def test_gemma_verify_matches_serial_steps(chunk):
    """A Gemma target's batched verification (soft cap on every row, local
    windows across the chunk) against one step at a time."""
    shape = fm.GemmaShape(**GEMMA, seed=3)
    tokens = [(i * 37 + 11) % shape.vocabulary for i in range(2 * chunk + 3)]
    worst = verify_matches_steps(shape, tokens, chunk)
    print(f"gemma chunk {chunk}: worst scaled logit error {worst:.3g}", flush=True)


@pytest.mark.parametrize("draft", ["other", "same", "none"])
def test_gemma_generation_equals_target_decode(draft):
    target = fm.GemmaShape(**GEMMA, seed=3)
    other = fm.GemmaShape(**{**GEMMA, "local": (0,)}, shared_kv_layers=0, output_scales=(), seed=11)
    generation_equals_target_decode(target, other if draft == "other" else None, PROMPT, limit=40,
                                    same_draft=draft == "same")
