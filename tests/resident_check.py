"""The engine's inference session (backend/core/llm_cpu.c, built from the
reference sources into oracle/_ref/libnya_dropin.so with this repository's
ROCm provider registered) driven from Python: the same model loaded twice,
one copy on the engine's scalar reference path (no compute context), one on
a named provider, and their logits and KV caches compared as the engine's
own inference test does (backend/tests/test_inference.c:9-33, :207-219):
every logit within 5e-4 (1 + |reference|) and every cached K/V value within
1.5e-4 (1 + |reference|)."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LOGIT_BOUND = 5e-4
KV_BOUND = 1.5e-4


class Stats(ctypes.Structure):
    # nya_compute_stats, backend/include/compute.h:12-22
    _fields_ = [("weights_bytes", ctypes.c_size_t), ("kv_bytes", ctypes.c_size_t),
                ("scratch_bytes", ctypes.c_size_t), ("prefill_batch", ctypes.c_size_t),
                ("external_matmul_bytes", ctypes.c_size_t), ("kernel_launches", ctypes.c_ulonglong),
                ("uploads", ctypes.c_ulonglong), ("downloads", ctypes.c_ulonglong),
                ("synchronizations", ctypes.c_ulonglong), ("external_matmul_calls", ctypes.c_ulonglong),
                ("graph_captures", ctypes.c_ulonglong), ("graph_replays", ctypes.c_ulonglong),
                ("external_matmul_kind", ctypes.c_uint), ("cutlass_matmul_calls", ctypes.c_ulonglong),
                ("tiled_attention_calls", ctypes.c_ulonglong)]


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.nya_llm_load.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(vp), ctypes.c_char_p, sz]
    lib.nya_llm_free.argtypes = [vp]
    lib.nya_llm_session_create.restype = vp
    lib.nya_llm_session_create.argtypes = [vp, sz, ctypes.c_char_p, sz]
    lib.nya_llm_session_free.argtypes = [vp]
    lib.nya_llm_session_reset.argtypes = [vp]
    lib.nya_llm_session_run.argtypes = [vp, ctypes.POINTER(ctypes.c_uint32), sz, ctypes.c_int]
    lib.nya_llm_session_logits.restype = ctypes.POINTER(ctypes.c_float)
    lib.nya_llm_session_logits.argtypes = [vp]
    lib.nya_llm_session_execution.restype = ctypes.c_char_p
    lib.nya_llm_session_execution.argtypes = [vp]
    lib.nya_llm_session_stats.argtypes = [vp, ctypes.POINTER(Stats)]
    fp = ctypes.POINTER(ctypes.c_float)
    lib.nya_llm_session_read_kv.argtypes = [vp, sz, sz, sz, fp, fp, sz]
    lib.nya_compute_free.argtypes = [vp]
    lib.nya_compute_name.restype = ctypes.c_char_p
    lib.nya_compute_name.argtypes = [vp]
    return lib


class Model:
    """A loaded model; provider None: the engine's scalar reference path."""

    def __init__(self, lib, path: Path, provider: str | None):
        self.lib = lib
        saved = os.environ.get("NYA_COMPUTE")
        os.environ["NYA_COMPUTE"] = provider or "cpu"
        try:
            self.ptr = ctypes.c_void_p()
            err = ctypes.create_string_buffer(512)
            rc = lib.nya_llm_load(str(path).encode(), path.stat().st_size, ctypes.byref(self.ptr), err, 512)
            assert rc == 0, err.value
        finally:
            if saved is None:
                os.environ.pop("NYA_COMPUTE", None)
            else:
                os.environ["NYA_COMPUTE"] = saved
        # nya_llm_context.compute is its first member (backend/core/llm_internal.h:123).
        self.compute = ctypes.c_void_p.from_address(self.ptr.value)
        if provider is None:
            lib.nya_compute_free(self.compute.value)
            self.compute.value = None

    def provider(self) -> str:
        return self.lib.nya_compute_name(self.compute.value).decode()

    def close(self):
        self.lib.nya_llm_free(self.ptr)


class Session:
    def __init__(self, model: Model, capacity: int):
        self.lib, self.model, self.capacity = model.lib, model, capacity
        err = ctypes.create_string_buffer(512)
        self.ptr = self.lib.nya_llm_session_create(model.ptr, capacity, err, 512)
        assert self.ptr, err.value

    def execution(self) -> str:
        return self.lib.nya_llm_session_execution(self.ptr).decode()

    def run(self, tokens, each: bool) -> int:
        arr = (ctypes.c_uint32 * len(tokens))(*tokens)
        return self.lib.nya_llm_session_run(self.ptr, arr, len(tokens), 1 if each else 0)

    def logits(self, vocabulary: int) -> np.ndarray:
        p = self.lib.nya_llm_session_logits(self.ptr)
        assert p, "no logits"
        return np.ctypeslib.as_array(p, shape=(vocabulary,)).copy()

    def kv(self, layer: int, position: int, count: int, width: int):
        n = count * width
        k, v = np.empty(n, np.float32), np.empty(n, np.float32)
        fp = ctypes.POINTER(ctypes.c_float)
        rc = self.lib.nya_llm_session_read_kv(self.ptr, layer, position, count, k.ctypes.data_as(fp),
                                              v.ctypes.data_as(fp), n)
        assert rc == 0
        return k, v

    def stats(self) -> Stats:
        s = Stats()
        self.lib.nya_llm_session_stats(self.ptr, ctypes.byref(s))
        return s

    def reset(self):
        self.lib.nya_llm_session_reset(self.ptr)

    def close(self):
        self.lib.nya_llm_session_free(self.ptr)


def check_logits(ref: np.ndarray, got: np.ndarray, where: str):
    same = ref == got   # includes -infinity masks
    assert np.all(np.isfinite(got) | same), f"{where}: non-finite logits"
    scaled = np.abs(got.astype(np.float64) - ref) / (1 + np.abs(ref.astype(np.float64)))
    scaled[same] = 0
    worst = int(np.argmax(scaled))
    assert scaled[worst] <= LOGIT_BOUND, f"{where}: logit {worst} {got[worst]} vs {ref[worst]} ({scaled[worst]:.3g})"
    return float(scaled.max())


def kv_widths(shape) -> list[int]:
    """Floats per cached position of each layer."""
    if hasattr(shape, "kv_widths"):
        return shape.kv_widths()
    return [shape.kv_heads * (shape.embedding // shape.heads)] * shape.blocks


def check_kv(ref: Session, got: Session, widths: list[int], count: int):
    worst = 0.0
    for layer, width in enumerate(widths):
        for a, b in zip(ref.kv(layer, 0, count, width), got.kv(layer, 0, count, width)):
            assert np.all(np.isfinite(b))
            scaled = np.abs(b.astype(np.float64) - a) / (1 + np.abs(a.astype(np.float64)))
            assert scaled.max() <= KV_BOUND, f"layer {layer}: KV scaled error {scaled.max():.3g}"
            worst = max(worst, float(scaled.max()))
    return worst


def compare(lib, path: Path, shape, provider: str, tokens: list[int], chunks=(5, 1, 1, 7, 1)) -> dict:
    """Token-by-token decode, then (after a reset) prefill chunks mixed with
    decode steps (`chunks`: tokens per session run; runs of more than one
    token are the plan's prefill), on the reference and on `provider`; every
    step's logits and the final KV caches compared. Returns the worst scaled
    errors."""
    ref_model, model = Model(lib, path, None), Model(lib, path, provider)
    assert model.provider() == provider
    ref, got = Session(ref_model, shape.context), Session(model, shape.context)
    widths = kv_widths(shape)
    out = {"execution": got.execution(), "logit": 0.0, "kv": 0.0}
    try:
        for i, t in enumerate(tokens):
            assert ref.run([t], True) == 0 and got.run([t], True) == 0
            out["logit"] = max(out["logit"], check_logits(ref.logits(shape.vocabulary), got.logits(shape.vocabulary),
                                                          f"decode position {i}"))
        out["kv"] = check_kv(ref, got, widths, len(tokens))
        # Reset, then prefill chunks (the plan's prefill) between decode steps.
        ref.reset()
        got.reset()
        at = 0
        for n in chunks:
            part = [(i * 7 + 3) % shape.vocabulary for i in range(at, at + n)]
            assert ref.run(part, n == 1) == 0 and got.run(part, n == 1) == 0
            at += n
            out["logit"] = max(out["logit"], check_logits(ref.logits(shape.vocabulary), got.logits(shape.vocabulary),
                                                          f"chunk ending at {at}"))
        out["kv"] = max(out["kv"], check_kv(ref, got, widths, at))
        out["stats"] = got.stats()
    finally:
        got.close()
        ref.close()
        model.close()
        ref_model.close()
    return out


def plan_against_engine(lib, tmp_path: Path, shape, tokens: list[int]) -> dict:
    """Decode `tokens` on a plan that fyodor_amd.model builds (no engine
    loader) through this repository's compute API, and on the engine's
    reference session of the same model written as GGUF; then one prefill
    chunk. Returns the worst scaled logit and KV errors."""
    from fyodor_amd import Compute
    from fyodor_amd import model as fm
    from gguf_model import write, write_gemma
    path = tmp_path / "model.gguf"
    gemma = isinstance(shape, fm.GemmaShape)
    (write_gemma if gemma else write)(path, shape)
    ref_model = Model(lib, path, None)
    ref = Session(ref_model, shape.context)
    compute = Compute("rocm")
    plan = fm.Plan(compute, fm.GemmaModel(shape) if gemma else fm.LlamaModel(shape), shape.context)
    worst = {"logit": 0.0, "kv": 0.0}
    try:
        for i, t in enumerate(tokens):
            assert ref.run([t], True) == 0
            got = plan.token(t, i)
            worst["logit"] = max(worst["logit"], check_logits(ref.logits(shape.vocabulary), got, f"position {i}"))
        chunk = [(7 * i + 3) % shape.vocabulary for i in range(4)]
        assert ref.run(chunk, False) == 0
        got = plan.prefill(chunk, len(tokens))
        worst["logit"] = max(worst["logit"], check_logits(ref.logits(shape.vocabulary), got, "prefill chunk"))
        n = len(tokens) + len(chunk)
        for layer, width in enumerate(kv_widths(shape)):
            for a, b in zip(ref.kv(layer, 0, n, width), plan.read_kv(layer, 0, n)):
                scaled = np.abs(b.astype(np.float64) - a) / (1 + np.abs(a.astype(np.float64)))
                assert scaled.max() <= KV_BOUND, f"layer {layer}: KV scaled error {scaled.max():.3g}"
                worst["kv"] = max(worst["kv"], float(scaled.max()))
        stats = plan.stats()
        assert stats["kernel_launches"] > 0 and stats["weights_bytes"] > 0 and stats["kv_bytes"] > 0
    finally:
        plan.close()
        compute.close()
        ref.close()
        ref_model.close()
    return worst
