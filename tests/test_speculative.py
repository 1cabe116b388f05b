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
- suppressed tokens are skipped by the device greedy choice;
- requests outside the plan's limits are refused without retiring it."""
import pytest

from fyodor_amd import Compute
from fyodor_amd import model as fm
from speculative_check import (generation_equals_target_decode, suppressed_tokens_are_skipped,
                               verify_matches_steps)

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
