"""Pins oracle/speculative.py (the engine's sampler and speculative sampling
loop restated) to the engine itself: nya_llm_generate_draft and
nya_llm_generate compiled from the reference sources (backend/core/
llm_cpu.c:1155-1336, :940-1100, in oracle/_ref/libnya_dropin.so), run on
the engine's scalar reference path for a random-weight LLaMA GGUF target
and draft (tests/gguf_model.py).

The oracle gets its logits from the engine's own sessions, driven the way
the engine's loop drives its states (the prompt as one prefill, every later
token one forward step), so the logits are the engine's bit for bit; the
oracle must then give the engine's text (its tokens, decoded by the
engine's nya_llm_decode_token), its token count and its counts of proposals
and accepted proposals, over seeds, temperatures, top-k, top-p, windows and
drafts (other weights, the target itself, none)."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np
import pytest

from fyodor_amd.model import LlamaShape
from gguf_model import write
from oracle import speculative as spec
from resident_check import Model, Session, bind

STOPS = (2,)   # the test vocabulary's end-of-sequence token (tests/gguf_model.py)


class Request(ctypes.Structure):
    # nya_generation_request, backend/include/generation.h:22-52
    _fields_ = [("prompt", ctypes.c_char_p), ("max_tokens", ctypes.c_size_t), ("temperature", ctypes.c_float),
                ("top_p", ctypes.c_float), ("top_k", ctypes.c_size_t), ("seed", ctypes.c_uint64),
                ("max_output_bytes", ctypes.c_size_t), ("draft_model", ctypes.c_void_p),
                ("speculative_tokens", ctypes.c_size_t), ("soft_tokens", ctypes.c_void_p),
                ("soft_token_spans", ctypes.c_size_t)]


class Response(ctypes.Structure):
    # nya_generation_response, backend/include/generation.h:62-72
    _fields_ = [("text", ctypes.c_void_p), ("text_length", ctypes.c_size_t), ("prompt_tokens", ctypes.c_size_t),
                ("generated_tokens", ctypes.c_size_t), ("seed", ctypes.c_uint64), ("stop_reason", ctypes.c_int),
                ("draft_tokens", ctypes.c_size_t), ("accepted_draft_tokens", ctypes.c_size_t),
                ("target_steps", ctypes.c_size_t)]


_libc = ctypes.CDLL(ctypes.util.find_library("c"))
_libc.free.argtypes = [ctypes.c_void_p]


class Engine:
    def __init__(self, lib):
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        lib.nya_llm_generate_draft.argtypes = [vp, vp, ctypes.POINTER(Request), ctypes.POINTER(Response),
                                               ctypes.c_char_p, sz]
        lib.nya_llm_tokenize.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.POINTER(ctypes.c_uint32)),
                                         ctypes.POINTER(sz), ctypes.c_char_p, sz]
        lib.nya_llm_decode_token.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_char_p, sz,
                                             ctypes.POINTER(sz)]
        self.lib = lib

    def tokenize(self, model: Model, text: str) -> list[int]:
        p, n = ctypes.POINTER(ctypes.c_uint32)(), ctypes.c_size_t()
        err = ctypes.create_string_buffer(256)
        assert self.lib.nya_llm_tokenize(model.ptr, text.encode(), ctypes.byref(p), ctypes.byref(n), err, 256) == 0
        ids = [p[i] for i in range(n.value)]
        _libc.free(ctypes.cast(p, ctypes.c_void_p))
        return ids

    def decode(self, model: Model, previous: int, tokens, capacity: int = 4096) -> bytes:
        buf = ctypes.create_string_buffer(capacity + 1)
        length = ctypes.c_size_t(0)
        for t in tokens:
            assert self.lib.nya_llm_decode_token(model.ptr, previous, t, buf, capacity + 1, ctypes.byref(length)) == 0
            previous = t
        return buf.raw[:length.value]

    def generate(self, target: Model, draft: Model | None, prompt: str, limit: int, window: int, temperature: float,
                 top_p: float, top_k: int, seed: int):
        # Without a draft the engine takes no window (llm_cpu.c:1165-1170).
        req = Request(prompt.encode(), limit, temperature, top_p, top_k, seed, 4096, None, window if draft else 0,
                      None, 0)
        resp = Response()
        err = ctypes.create_string_buffer(512)
        rc = self.lib.nya_llm_generate_draft(target.ptr, draft.ptr if draft else None, ctypes.byref(req),
                                             ctypes.byref(resp), err, 512)
        assert rc == 0, err.value
        text = ctypes.string_at(resp.text, resp.text_length)
        out = {"text": text, "generated": resp.generated_tokens, "draft_tokens": resp.draft_tokens,
               "accepted": resp.accepted_draft_tokens, "prompt_tokens": resp.prompt_tokens}
        _libc.free(resp.text)
        return out


class SessionSource:
    """The engine's logits after a token sequence, from one of its sessions
    run as its generation loop runs a state: the prompt as one prefill (the
    session's batched run), every later token as one forward step; a
    sequence that leaves the session's tokens starts again from the prompt."""

    def __init__(self, session: Session, vocabulary: int, prompt_len: int):
        self.s, self.v, self.n0, self.tokens = session, vocabulary, prompt_len, None

    def after(self, seq) -> np.ndarray:
        seq = list(seq)
        if self.tokens is None or seq[:len(self.tokens)] != self.tokens:
            self.s.reset()
            assert self.s.run(seq[:self.n0], False) == 0
            self.tokens = seq[:self.n0]
        for t in seq[len(self.tokens):]:
            assert self.s.run([t], True) == 0
            self.tokens.append(t)
        return self.s.logits(self.v)

    def rows(self, prefix, batch):
        return np.stack([self.after(list(prefix) + list(batch[:j + 1])) for j in range(len(batch))])

    def row(self, prefix, token):
        return self.after(list(prefix) + [token])


@pytest.fixture(scope="module")
def engine(dropin_library, tmp_path_factory):
    lib = bind(dropin_library)
    d = tmp_path_factory.mktemp("sampling")
    target_shape = LlamaShape(context=64, seed=3)
    draft_shape = LlamaShape(context=64, seed=11, blocks=1)
    write(d / "target.gguf", target_shape)
    write(d / "draft.gguf", draft_shape)
    target, draft = Model(lib, d / "target.gguf", None), Model(lib, d / "draft.gguf", None)
    yield Engine(lib), target, draft, target_shape
    target.close()
    draft.close()


CASES = [  # window, temperature, top_p, top_k, seed
    (4, 1.0, 1.0, 0, 1), (1, 0.7, 0.9, 0, 7), (3, 1.5, 1.0, 5, 123), (5, 1.0, 0.5, 40, 99), (2, 2.5, 1.0, 0, 0),
    (8, 0.3, 0.95, 0, 5), (4, 4.0, 1.0, 3, 2**63 + 11),
]


@pytest.mark.parametrize("draft", ["other", "same", "none"])
def test_oracle_equals_engine(engine, draft):
    eng, target, other, shape = engine
    prompt_text = "p0002p0014p0197p0000p0040"
    prompt = eng.tokenize(target, prompt_text)
    assert len(prompt) >= 2
    limit = 16
    draft_model = {"other": other, "same": target, "none": None}[draft]
    mixed = False
    for window, temperature, top_p, top_k, seed in CASES:
        got = eng.generate(target, draft_model, prompt_text, limit, window, temperature, top_p, top_k, seed)
        assert got["prompt_tokens"] == len(prompt)
        tsrc = SessionSource(Session(target, shape.context), shape.vocabulary, len(prompt))
        dsrc = SessionSource(Session(draft_model, shape.context), shape.vocabulary, len(prompt)) if draft_model else None
        try:
            tokens, counts = spec.generate(tsrc.rows, dsrc.row if dsrc else None, prompt, limit, window, temperature,
                                           top_p, top_k, seed, STOPS)
        finally:
            tsrc.s.close()
            if dsrc:
                dsrc.s.close()
        where = f"draft {draft} window {window} T {temperature} top_p {top_p} top_k {top_k} seed {seed}"
        shown = [t for t in tokens if t not in STOPS]
        assert eng.decode(target, prompt[-1], shown) == got["text"], where
        assert got["generated"] == len(tokens), where
        if draft_model is not None:
            assert got["draft_tokens"] == counts["draft_tokens"], where
            assert got["accepted"] == counts["accepted"], where
            mixed |= 0 < counts["accepted"] < counts["draft_tokens"]
        if draft == "same":
            assert counts["accepted"] == counts["draft_tokens"], where
    if draft == "other":
        assert mixed
