"""Checks of batched verification and greedy speculative decoding
(nya_compute_plan_verify, nya_compute_generate_greedy), shared by the CPU
test on the mock HIP runtime (tests/test_speculative.py) and the MI355X test
(tests/test_gpu_speculative.py).

The oracle is the target plan's own serial decode: one nya_compute_plan_token
per token, with the engine's greedy rule applied to its logits (the first
largest value, backend/core/llm_cpu.c:896-904; numpy's argmax picks the first
of equal maxima). Greedy speculative decoding must emit exactly that
sequence, whatever the draft proposes (backend/core/llm_cpu.c:1274-1317).

Sampled generation (nya_compute_generate_sampled) is checked against
oracle/speculative.py, the engine's sampler and speculative sampling loop
restated (itself pinned to the engine's nya_llm_generate_draft in
tests/test_sampling_oracle.py), fed by a second pair of plans that make the
same provider calls as the C loop: equal logits, so equal tokens."""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from fyodor_amd import Compute, storage_bytes
from fyodor_amd import model as fm
from oracle import speculative as spec
from resident_check import LOGIT_BOUND


def serial_decode(plan: fm.Plan, prompt, limit: int, stops=()):
    """The target's greedy decode, one plan_token per step, and the logits
    each choice was made from."""
    logits = plan.prefill(prompt, 0).copy() if len(prompt) > 1 else plan.token(prompt[0], 0).copy()
    out, rows, position = [], [], len(prompt)
    while len(out) < limit:
        rows.append(logits)
        t = int(np.argmax(logits))
        out.append(t)
        if t in stops or len(out) == limit:
            break
        logits = plan.token(t, position).copy()
        position += 1
    return out, rows


def second_best_gap(row: np.ndarray) -> float:
    """How far the largest logit is above the next one, scaled like the
    engine's logit bound."""
    top = np.sort(row.astype(np.float64))[-2:]
    return float((top[1] - top[0]) / (1 + abs(top[1])))


def check_same_decode(got, ref, ref_rows, where: str):
    """got equals the serial decode, or differs first where the serial
    logits' two largest are within the logit bound of each other (a tie the
    batched and the serial arithmetic may resolve differently)."""
    for i, (a, b) in enumerate(zip(got, ref)):
        if a != b:
            gap = second_best_gap(ref_rows[i])
            assert gap <= 2 * LOGIT_BOUND, f"{where}: token {i} is {a}, the target's greedy choice is {b} (gap {gap:.3g})"
            return i
    assert len(got) == len(ref), f"{where}: {len(got)} tokens, the serial decode has {len(ref)}"
    return len(got)


def model_of(shape, tensors=None):
    """fyodor_amd.model's description of a LLaMA or Gemma shape."""
    if isinstance(shape, fm.GemmaShape):
        return fm.GemmaModel(shape, tensors)
    return fm.LlamaModel(shape, tensors)


def verify_matches_steps(shape, tokens: list[int], chunk: int):
    """plan_verify over chunks of `tokens` against plan_token one at a time:
    the same greedy choices and logits within the engine's bound; a chunk
    run again from an earlier position (a rejected proposal) as well."""
    compute = Compute("rocm")
    model = model_of(shape)
    serial, batched = fm.Plan(compute, model, shape.context), fm.Plan(compute, model, shape.context)
    worst = 0.0
    try:
        assert batched.verify_limit >= chunk
        ref = [serial.token(t, i).copy() for i, t in enumerate(tokens)]
        for at in range(0, len(tokens), chunk):
            part = tokens[at:at + chunk]
            ids, rows = batched.verify(part, at, logits=True)
            for i, row in enumerate(rows):
                r = ref[at + i]
                scaled = np.abs(row.astype(np.float64) - r) / (1 + np.abs(r.astype(np.float64)))
                worst = max(worst, float(scaled.max()))
                assert scaled.max() <= LOGIT_BOUND, f"position {at + i}: scaled logit error {scaled.max():.3g}"
                if ids[i] != int(np.argmax(r)):
                    assert second_best_gap(r) <= 2 * LOGIT_BOUND, f"position {at + i}: greedy {ids[i]}"
        # Run positions 2.. again with other tokens: the cache entries are
        # overwritten and the logits follow the new tokens.
        other = [(t * 7 + 1) % shape.vocabulary for t in tokens[2:2 + chunk]]
        ids, rows = batched.verify(other, 2, logits=True)
        fresh = fm.Plan(compute, model, shape.context)
        try:
            for i, t in enumerate(tokens[:2] + other):
                r = fresh.token(t, i)
                if i >= 2:
                    scaled = np.abs(rows[i - 2].astype(np.float64) - r) / (1 + np.abs(r.astype(np.float64)))
                    assert scaled.max() <= LOGIT_BOUND, f"rerun position {i}: scaled error {scaled.max():.3g}"
        finally:
            fresh.close()
        stats = batched.stats()
        assert stats["downloads"] > 0 and stats["external_matmul_calls"] > 0
    finally:
        serial.close()
        batched.close()
        compute.close()
    return worst


def swapped_output(shape: fm.LlamaShape, tensors, a: int, b: int):
    """The target's tensors with rows a and b of the output matrix swapped: a
    draft that proposes b where the target picks a (and a for b) and agrees
    with it elsewhere."""
    out = []
    for name, t, dims, data in tensors:
        if name == "output.weight":
            row = storage_bytes(t, 1, shape.embedding)
            data = data.copy()
            ra, rb = data[a * row:(a + 1) * row].copy(), data[b * row:(b + 1) * row].copy()
            data[a * row:(a + 1) * row], data[b * row:(b + 1) * row] = rb, ra
        out.append((name, t, dims, data))
    return out


def generation_equals_target_decode(target_shape, draft_shape, prompt,
                                    limit: int, windows=(1, 4), same_draft: bool = False, stop_at: int | None = None,
                                    swap: bool = False):
    """nya_compute_generate_greedy with the draft (or the target's own weights
    as draft, or those weights with two output rows swapped where `swap`, or
    none) at each window emits the serial greedy decode of the target;
    returns (window, counters) of every run."""
    compute = Compute("rocm")
    target_model = model_of(target_shape)
    capacity = len(prompt) + limit
    oracle = fm.Plan(compute, target_model, capacity)
    try:
        ref, rows = serial_decode(oracle, prompt, limit)
    finally:
        oracle.close()
    if swap:
        # The token the target emits most often, swapped with another.
        a = max(set(ref), key=ref.count)
        draft_model = fm.LlamaModel(target_shape, swapped_output(target_shape, target_model.arrays, a,
                                                                 (a + 1) % target_shape.vocabulary))
    else:
        draft_model = target_model if same_draft else (model_of(draft_shape) if draft_shape else None)
    stops = ()
    if stop_at is not None:
        stops = (ref[stop_at],)
        ref, rows = ref[:ref.index(ref[stop_at]) + 1], rows[:ref.index(ref[stop_at]) + 1]
    results = []
    try:
        for window in windows if draft_model is not None else (0,):
            target = fm.Plan(compute, target_model, capacity)
            draft = fm.Plan(compute, draft_model, capacity) if draft_model is not None else None
            try:
                got, stats = fm.generate_greedy(target, draft, prompt, limit, window=window, stops=stops)
            finally:
                target.close()
                if draft:
                    draft.close()
            agree = check_same_decode(got, ref, rows, f"window {window}")
            if agree == len(ref):
                assert stats["generated"] == len(got) == len(ref)
                assert stats["accepted"] <= stats["draft_tokens"]
                if same_draft and window:
                    # The draft is the target: every proposal is accepted
                    # unless the limit or a stop cut the round short.
                    assert stats["accepted"] >= stats["draft_tokens"] - stats["rounds"]
                    assert stats["rounds"] <= -(-len(ref) // (window + 1)) + 1
                if not window:
                    assert stats["rounds"] == len(ref) and stats["draft_tokens"] == 0
            results.append((window, stats))
    finally:
        compute.close()
    return results


def suppressed_tokens_are_skipped(shape: fm.LlamaShape, prompt):
    """With the target's first greedy choice suppressed, verification picks
    the best remaining token, as the engine masks suppressed tokens before
    sampling (backend/core/llm_cpu.c:570-574)."""
    compute = Compute("rocm")
    model = fm.LlamaModel(shape)
    plan = fm.Plan(compute, model, shape.context)
    try:
        logits = plan.prefill(prompt, 0).copy()
    finally:
        plan.close()
    first = int(np.argmax(logits))
    keep = (ctypes.c_uint32 * 2)(first, shape.vocabulary - 1)
    model.context.tokenizer.suppressed_tokens = ctypes.addressof(keep)
    model.context.tokenizer.suppressed_count = 2
    plan = fm.Plan(compute, model, shape.context)
    try:
        ids, rows = plan.verify(prompt, 0, logits=True)
        masked = logits.copy()
        masked[[first, shape.vocabulary - 1]] = -np.inf
        assert rows[-1][first] == -np.inf
        assert ids[-1] == int(np.argmax(masked)) or second_best_gap(masked) <= 2 * LOGIT_BOUND
        assert ids[-1] != first
    finally:
        plan.close()
        compute.close()
        del keep


class PlanSource:
    """Logits for the sampling oracle from a plan, through the calls
    nya_compute_generate_sampled makes: positions of the prefix not yet in
    the plan's cache (the first mismatch on) run as one catch-up (plan_token
    for one token, plan_prefill for more), then one verification of the
    batch returns its rows."""

    def __init__(self, plan: fm.Plan):
        self.plan, self.cache = plan, []

    def rows(self, prefix, batch):
        k = 0
        while k < min(len(self.cache), len(prefix)) and self.cache[k] == prefix[k]:
            k += 1
        part = list(prefix[k:])
        if len(part) == 1:
            self.plan.token(part[0], k, logits=False)
        elif part:
            self.plan.prefill(part, k)
        _, rows = self.plan.verify(list(batch), len(prefix), logits=True)
        self.cache = list(prefix) + list(batch)
        return rows

    def row(self, prefix, token):
        return self.rows(prefix, [token])[0]


def sampled_generation_matches_oracle(target_shape: fm.LlamaShape, draft: str, prompt, limit: int, cases,
                                      stops=()):
    """nya_compute_generate_sampled for each (window, temperature, top_p,
    top_k, seed) of `cases` emits the oracle's tokens, with its counts of
    proposals and accepted proposals; `draft` is "other" (other weights),
    "same" (the target's weights) or "none". Returns the counters."""
    compute = Compute("rocm")
    target_model = fm.LlamaModel(target_shape)
    draft_model = {"other": lambda: fm.LlamaModel(dataclasses.replace(target_shape, seed=11, blocks=1)),
                   "same": lambda: target_model, "none": lambda: None}[draft]()
    capacity = len(prompt) + limit
    out = []
    try:
        for window, temperature, top_p, top_k, seed in cases:
            plans = [fm.Plan(compute, target_model, capacity)]
            if draft_model is not None:
                plans.append(fm.Plan(compute, draft_model, capacity))
            try:
                got, stats = fm.generate_sampled(plans[0], plans[1] if len(plans) > 1 else None, prompt, limit,
                                                 temperature, top_p, top_k, seed, window=window, stops=stops)
                sources = [PlanSource(fm.Plan(compute, target_model, capacity))]
                if draft_model is not None:
                    sources.append(PlanSource(fm.Plan(compute, draft_model, capacity)))
                try:
                    ref, counts = spec.generate(sources[0].rows, sources[1].row if len(sources) > 1 else None, prompt,
                                                limit, window, temperature, top_p, top_k, seed, stops)
                finally:
                    for src in sources:
                        src.plan.close()
            finally:
                for plan in plans:
                    plan.close()
            where = f"window {window} T {temperature} top_p {top_p} top_k {top_k} seed {seed}"
            assert got == ref, f"{where}: {got} != {ref}"
            assert stats["generated"] == len(got)
            assert stats["accepted"] == counts["accepted"], where
            assert stats["draft_tokens"] == counts["draft_tokens"], where
            out.append(stats)
    finally:
        compute.close()
    return out


def first_token_follows_target(target_shape: fm.LlamaShape, prompt, runs: int, window: int = 4):
    """The engine's distribution check (backend/tests/test_generation.c
    :345-365) on the ROCm provider's plans: with top-k 2, a temperature giving the leading
    candidate p = 3/4, and a draft favouring the other candidate, the
    first token over `runs` seeds follows the target's two-candidate
    distribution (within five standard deviations), and both acceptance and
    rejection happen; with top_p below the leading probability only the
    leading token comes out (:377-387). Returns (p, count of the leading
    token, accepted proposals)."""
    compute = Compute("rocm")
    target_model = fm.LlamaModel(target_shape)
    capacity = len(prompt) + 1
    probe = fm.Plan(compute, target_model, capacity)
    try:
        row = probe.prefill(list(prompt), 0).copy()
    finally:
        probe.close()
    # The temperature that gives the leading candidate p = 3/4 of the two:
    # draws of the target's distribution and of the reversed draft's then
    # differ by half the runs.
    top2 = np.sort(row)[-2:]
    temperature = float(np.float32((top2[1] - top2[0]) / np.log(3.0))) if top2[1] > top2[0] else 1.0
    dense, cand = spec.distribution(row, temperature, 1.0, 2)
    lead, p = cand[0]
    # As the engine's test does, a draft that reverses the two candidates:
    # the target's weights with their output rows swapped.
    draft_model = fm.LlamaModel(target_shape, swapped_output(target_shape, target_model.arrays, lead, cand[1][0]))
    target, draft = fm.Plan(compute, target_model, capacity), fm.Plan(compute, draft_model, capacity)
    try:
        count = accepted = 0
        for seed in range(1, runs + 1):
            got, stats = fm.generate_sampled(target, draft, prompt, 1, temperature, 1.0, 2, seed, window=window)
            count += got[0] == lead
            accepted += stats["accepted"]
        sigma = (runs * p * (1 - p)) ** 0.5
        assert abs(count - runs * p) <= 4.5 * sigma, (count, runs, p)
        assert 0 < accepted < runs, accepted
        for seed in range(1, 33):
            got, _ = fm.generate_sampled(target, draft, prompt, 1, temperature, 0.9 * p, 2, seed, window=window)
            assert got == [lead], (seed, got, lead, p)
    finally:
        target.close()
        draft.close()
        compute.close()
    return p, count, accepted
