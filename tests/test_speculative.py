"""Batched verification and greedy speculative decoding on the CPU, against
the mock HIP runtime and kernel library (tests/mock/mock_hip.c computes the
resident steps and the greedy choice on the host); tests/speculative_check.py
holds the checks, which also run on an MI355X (tests/test_gpu_speculative.py):

- nya_compute_plan_verify over chunks of tokens gives the logits and greedy
  choices of one plan_token per token, and runs earlier positions again;
- nya_compute_generate_greedy emits the target's own serial greedy decode
  with a draft of other weights (proposals rejected), with the target's own
  weights as draft (every proposal accepted), with those weights but two
  rows of the output matrix swapped (some accepted, some rejected), and
  without a draft, at several windows; a stop token ends it after the token
  is emitted;
- nya_compute_generate_sampled emits the tokens of the engine's speculative
  sampling loop restated (oracle/speculative.py) over seeds, temperatures,
  top-k, top-p, windows and drafts (other weights, the target's own, none),
  with its counts of proposals and acceptances; over many seeds the first
  token follows the target's distribution, and top-p below the leading
  probability keeps only the leading token (the engine's own checks,
  backend/tests/test_generation.c:345-387);
- suppressed tokens are skipped by the device greedy choice;
- requests outside the plan's limits are refused without retiring it."""
import pytest

from fyodor_amd import Compute
from fyodor_amd import model as fm
from speculative_check import (first_token_follows_target, generation_equals_target_decode,
                               sampled_generation_matches_oracle, suppressed_tokens_are_skipped, verify_matches_steps)

PROMPT = [5, 17, 200, 3]


@pytest.fixture()
def mock_rocm(mock_paths, monkeypatch):
    good, _ = mock_paths
    monkeypatch.setenv("NYA_ROCM_HIP_LIBRARY", str(good))
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(good))
    monkeypatch.delenv("NYA_ROCM_CACHE_MIB", raising=False)


def test_verify_matches_serial_steps(mock_rocm):
    verify_matches_steps(fm.LlamaShape(context=32, seed=3), [5, 17, 200, 3, 42, 99, 250, 1, 7, 64, 128], chunk=5)


@pytest.mark.parametrize("draft", ["other", "same", "swapped", "none"])
def test_generation_equals_target_decode(mock_rocm, draft):
    # Random weights settle into short cycles: seed 5's decode alternates two
    # tokens, so a draft with one of them swapped is right at every other
    # position.
    target = fm.LlamaShape(context=64, seed=5 if draft == "swapped" else 3)
    other = fm.LlamaShape(context=64, seed=11, blocks=1)
    runs = generation_equals_target_decode(target, other if draft == "other" else None, PROMPT, limit=14,
                                           windows=(1, 3, 5), same_draft=draft == "same", swap=draft == "swapped")
    for window, stats in runs:
        if draft == "other":
            assert stats["accepted"] < stats["draft_tokens"]
    if draft == "swapped":
        # At window 1 the draft only proposes after the swapped token (the
        # round's bonus) and is right; longer windows reach it and are wrong.
        assert any(0 < stats["accepted"] < stats["draft_tokens"] for _, stats in runs), runs


SAMPLED_CASES = [(4, 1.0, 1.0, 0, 1), (1, 0.7, 0.9, 0, 7), (3, 1.5, 1.0, 5, 123), (5, 1.0, 0.5, 40, 99),
                 (2, 2.5, 1.0, 0, 0)]


@pytest.mark.parametrize("draft", ["other", "same", "none"])
def test_sampled_generation_matches_oracle(mock_rocm, draft):
    runs = sampled_generation_matches_oracle(fm.LlamaShape(context=64, seed=3), draft, PROMPT, 16, SAMPLED_CASES)
    if draft == "same":
        # Equal weights give equal distributions: every proposal is accepted.
        assert all(r["accepted"] == r["draft_tokens"] for r in runs), runs
    if draft == "other":
        assert any(r["accepted"] < r["draft_tokens"] for r in runs), runs


def test_sampled_stop_token(mock_rocm):
    sampled_generation_matches_oracle(fm.LlamaShape(context=64, seed=3), "other", PROMPT, 24,
                                      [(4, 3.0, 1.0, 0, s) for s in (1, 2, 3)], stops=(7, 100, 250))


def test_sampled_first_token_distribution(mock_rocm):
    # A one-token prompt needs no catch-up runs; at p = 3/4, 400 seeds put
    # the target's distribution and the reversed draft's 23 standard
    # deviations apart.
    p, count, accepted = first_token_follows_target(fm.LlamaShape(context=64, seed=3), PROMPT[:1], runs=400)
    assert abs(p - 0.75) < 0.01, p


def test_stop_token_ends_generation(mock_rocm):
    generation_equals_target_decode(fm.LlamaShape(context=64, seed=3), None, PROMPT, limit=12, windows=(4,),
                                    same_draft=True, stop_at=5)


def test_suppressed_tokens_are_skipped(mock_rocm):
    suppressed_tokens_are_skipped(fm.LlamaShape(context=16, seed=3), PROMPT)


def test_requests_outside_limits_are_refused(mock_rocm):
    shape = fm.LlamaShape(context=64, seed=3)
    compute = Compute("rocm")
    plan = fm.Plan(compute, fm.LlamaModel(shape), 64)
    try:
        limit = plan.verify_limit
        assert limit == 33
        with pytest.raises(RuntimeError):
            plan.verify(list(range(limit + 1)), 0)           # more tokens than one verification takes
        with pytest.raises(RuntimeError):
            plan.verify([1, 2], 5)                           # past the valid prefix
        with pytest.raises(RuntimeError):
            plan.verify([shape.vocabulary], 0)               # outside the vocabulary
        assert plan.verify([1, 2, 3], 0) and plan.verify([4], 3)   # the plan is still usable
        with pytest.raises(RuntimeError):
            fm.generate_greedy(plan, None, [1], 8, window=33)    # window above 32
    finally:
        plan.close()
        compute.close()


def test_gemma_verify_matches_serial_steps(mock_rocm):
    """Batched verification of a Gemma target (its soft cap on every row)
    against one step at a time."""
    verify_matches_steps(fm.GemmaShape(context=32, seed=3), [5, 17, 200, 3, 42, 99, 250, 1, 7, 64, 128], chunk=5)


@pytest.mark.parametrize("draft", ["none", "same", "other"])
def test_gemma_generation_equals_target_decode(mock_rocm, draft):
    """Greedy generation with batched verification on a Gemma target emits
    its serial greedy decode, with no draft, the target itself, or a
    one-block Gemma draft."""
    target = fm.GemmaShape(context=64, seed=3)
    other = fm.GemmaShape(context=64, seed=11, local=(0,), shared_kv_layers=0, output_scales=())
    generation_equals_target_decode(target, other if draft == "other" else None, PROMPT, limit=20,
                                    same_draft=draft == "same")
