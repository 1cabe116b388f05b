"""The engine's model description built in memory, and the resident plan on it.

The provider's resident plan reads the engine's ``nya_llm_context`` by
address (backend/include/compute_backend.h:18); ``fyodor_amd/core/llm_internal.h``
lays those types out as the engine does (checked against the engine's header
by tests/test_boundary.py). This module fills the same structures from
numpy arrays, so a plan can run without the engine's GGUF loader — the
benchmark times it this way — and drives it through the compute API's plan
functions (backend/include/compute.h:37-51).

``LlamaShape`` / ``llama_tensors`` describe a dense LLaMA with the tensor
names the engine's loader binds (backend/core/llm_gguf.c:1069-1077) and
seeded synthetic weights of real-model scale (fyodor_amd.synth).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import F32, Q4_K, Q6_K, Compute, ComputeStats, storage_bytes, synth

vp, u32, u64, sz, f32, i32 = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_float,
                              ctypes.c_int32)


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("type", u32), ("dimension_count", u32), ("dimensions", u64 * 4),
                ("relative_offset", u64), ("data", vp), ("data_size", sz), ("bound", ctypes.c_int)]


TP = ctypes.POINTER(Tensor)


class Layer(ctypes.Structure):
    _fields_ = [(n, TP) for n in ("attention_norm", "query", "key", "value", "attention_output", "feed_forward_norm",
                                  "feed_forward_gate", "feed_forward_down", "feed_forward_up", "query_norm",
                                  "key_norm", "attention_post_norm", "ffn_post_norm", "router", "router_scale",
                                  "expert_scale", "expert_gate", "expert_up", "expert_gate_up", "expert_down",
                                  "expert_pre_norm", "shared_post_norm", "expert_post_norm", "ple_gate",
                                  "ple_projection", "ple_norm", "output_scale", "rope_factors")] + \
               [(n, u32) for n in ("head_count", "kv_head_count", "head_dimension", "hidden_length",
                                   "expert_hidden_length", "sliding_window", "kv_source")] + [("cache_offset", sz)]


class Tokenizer(ctypes.Structure):
    _fields_ = [("pieces", vp), ("piece_lengths", vp), ("scores", vp), ("types", vp), ("sorted", vp),
                ("vocabulary_size", u32), ("maximum_piece_length", sz), ("byte_tokens", i32 * 256),
                ("unknown_token", u32), ("beginning_token", u32), ("end_token", u32),
                ("add_beginning_token", ctypes.c_int), ("add_end_token", ctypes.c_int),
                ("add_space_prefix", ctypes.c_int), ("uses_sentencepiece_space", ctypes.c_int),
                ("uses_merge_ranks", ctypes.c_int), ("merges", vp), ("merge_count", sz), ("stop_tokens", vp),
                ("suppressed_tokens", vp), ("suppressed_count", sz), ("special_tokens", vp), ("special_count", sz)]


class Mapping(ctypes.Structure):
    _fields_ = [("data", vp), ("size", sz), ("file_handle", ctypes.c_size_t), ("mapping_handle", ctypes.c_size_t)]


class Projector(ctypes.Structure):
    _fields_ = [("vision_type", ctypes.c_char * 32), ("audio_type", ctypes.c_char * 32)] + \
               [(n, u32) for n in ("vision_width", "audio_width", "output_width", "audio_output_width",
                                   "vision_blocks", "audio_blocks", "patch_size", "position_count")] + \
               [("vision_epsilon", f32), ("audio_epsilon", f32)] + \
               [(n, TP) for n in ("patch", "patch_bias", "position", "vision", "audio")] + \
               [("norm_weight", TP * 3), ("norm_bias", TP * 3)]


class Context(ctypes.Structure):
    _fields_ = [("compute", vp), ("mapping", Mapping), ("metadata_end", sz), ("file_type_begin", sz),
                ("file_type_end", sz), ("gguf_metadata_count", u64), ("tensor_alignment", u32), ("tensors", TP),
                ("tensor_count", sz), ("layers", ctypes.POINTER(Layer)), ("tokenizer", Tokenizer),
                ("projector", Projector), ("token_embedding", TP), ("output_norm", TP), ("output", TP)] + \
               [(n, u32) for n in ("embedding_length", "feed_forward_length", "block_count", "head_count",
                                   "key_value_head_count", "context_length", "rope_dimension_count")] + \
               [("norm_epsilon", f32), ("rope_frequency_base", f32), ("is_gemma", ctypes.c_int),
                ("is_assistant", ctypes.c_int), ("backbone_length", u32), ("nextn_layers", u32),
                ("nextn_pre", TP), ("nextn_post", TP)] + \
               [(n, u32) for n in ("head_dimension", "sliding_head_dimension", "sliding_window", "shared_kv_layers",
                                   "per_layer_embedding_length", "expert_count", "experts_used")] + \
               [("sliding_rope_base", f32), ("final_logit_softcap", f32), ("ple_embedding", TP),
                ("ple_projection", TP), ("ple_norm", TP), ("cache_width", sz), ("maximum_query_length", sz),
                ("maximum_hidden_length", sz)] + \
               [(n, u32 * 256) for n in ("layer_heads", "layer_kv_heads", "layer_hidden", "layer_expert_hidden",
                                         "layer_sliding")] + \
               [(n, u32) for n in ("heads_count", "kv_heads_count", "hidden_count", "expert_hidden_count",
                                   "sliding_count", "value_dimension", "sliding_value_dimension",
                                   "sliding_rope_dimension")]


@dataclass
class LlamaShape:
    embedding: int = 256
    heads: int = 4
    kv_heads: int = 2
    hidden: int = 512
    blocks: int = 2
    context: int = 64
    vocabulary: int = 300
    # GGML types of the embedding / output / attention / gate-up / down
    # matrices; optional "value" and "up" entries override the attention
    # type for v and the gate-up type for up.
    types: dict = field(default_factory=lambda: {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K,
                                                 "gate_up": Q4_K, "down": Q6_K})
    epsilon: float = 1e-5
    rope_base: float = 10000.0
    seed: int = 1


def llama_tensors(shape: LlamaShape, shared_blocks: bool = False) -> list[tuple[str, int, tuple[int, ...], np.ndarray]]:
    """(name, type, dims with the row length first, bytes) of every tensor:
    the engine's LLaMA tensor names, seeded weights (norm weights 1 + N(0, 0.1)).
    With `shared_blocks`, every block's tensors are block 0's host arrays (a
    plan still uploads each tensor to its own device memory), which builds a
    many-block model in the time of one block."""
    d, h, v = shape.embedding, shape.hidden, shape.vocabulary
    kv = shape.kv_heads * (d // shape.heads)
    rng = np.random.default_rng(shape.seed)
    seed = [shape.seed * 1000]

    def matrix(kind: str, rows: int, cols: int):
        seed[0] += 1
        t = shape.types[kind] if kind in shape.types else shape.types["attention" if kind == "value" else "gate_up"]
        return t, (cols, rows), synth.weights(t, rows, cols, seed[0])

    def norm(n: int):
        w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        return F32, (n,), w.view(np.uint8)

    out = [("token_embd.weight", *matrix("embedding", v, d)), ("output_norm.weight", *norm(d)),
           ("output.weight", *matrix("output", v, d))]
    for b in range(1 if shared_blocks else shape.blocks):
        out += [(f"blk.{b}.attn_norm.weight", *norm(d)),
                (f"blk.{b}.attn_q.weight", *matrix("attention", d, d)),
                (f"blk.{b}.attn_k.weight", *matrix("attention", kv, d)),
                (f"blk.{b}.attn_v.weight", *matrix("value", kv, d)),
                (f"blk.{b}.attn_output.weight", *matrix("attention", d, d)),
                (f"blk.{b}.ffn_norm.weight", *norm(d)),
                (f"blk.{b}.ffn_gate.weight", *matrix("gate_up", h, d)),
                (f"blk.{b}.ffn_down.weight", *matrix("down", d, h)),
                (f"blk.{b}.ffn_up.weight", *matrix("up", h, d))]
    if shared_blocks:
        first = out[3:]
        for b in range(1, shape.blocks):
            out += [(name.replace("blk.0.", f"blk.{b}.", 1), t, dims, data) for name, t, dims, data in first]
    for name, t, dims, data in out:
        rows = dims[1] if len(dims) > 1 else 1
        assert data.nbytes == storage_bytes(t, rows, dims[0]), name
    return out


@dataclass
class GemmaShape:
    """A Gemma 4 text model as the engine's loader binds it
    (backend/core/llm_gguf.c:852-990): local (sliding-window) and global
    layers of their own head widths, the last `shared_kv_layers` layers
    reading the cache of the last earlier layer of their kind, global
    layers without a value matrix (the key stands in) unless
    `global_value`, per-head q/k norms, post norms, optional per-layer
    output scales, rotary factors for the global layers, the output matrix
    tied to the embedding unless `tied_output` is false, and a final logit
    soft cap."""
    embedding: int = 256
    heads: int = 4
    kv_heads: int = 2
    width: int = 128          # global layers' head width
    local_width: int = 64     # local layers' head width
    hidden: int = 512
    local: tuple = (1, 1, 0, 1, 1, 0)
    shared_kv_layers: int = 2
    window: int = 8
    context: int = 64
    vocabulary: int = 300
    types: dict = field(default_factory=lambda: {"embedding": Q6_K, "output": Q6_K, "attention": Q4_K,
                                                 "gate_up": Q4_K, "down": Q6_K})
    epsilon: float = 1e-6
    rope_base: float = 1000000.0
    local_rope_base: float = 10000.0
    softcap: float = 30.0
    global_value: bool = False
    tied_output: bool = True
    output_scales: tuple = (None, 0.5, None, 1.25, None, 0.75)
    seed: int = 3

    @property
    def blocks(self) -> int:
        return len(self.local)

    def head_width(self, layer: int) -> int:
        return self.local_width if self.local[layer] else self.width

    def kv_widths(self) -> list[int]:
        """Floats per cached position of each layer (its source's for a
        shared layer)."""
        return [self.kv_heads * self.head_width(i) for i in range(self.blocks)]

    def shared(self, layer: int) -> bool:
        return layer >= self.blocks - self.shared_kv_layers

    def kv_source(self, layer: int) -> int:
        """The layer whose cache `layer` reads: itself, or for a shared layer
        the last earlier unshared layer of its kind (llm_gguf.c:925-930)."""
        if not self.shared(layer):
            return layer
        first_shared = self.blocks - self.shared_kv_layers
        return max(i for i in range(first_shared) if self.local[i] == self.local[layer])


def gemma_tensors(shape: GemmaShape, shared_blocks: bool = False):
    """(name, type, dims, bytes) of every tensor of `shape` with the engine's
    Gemma tensor names. With `shared_blocks`, every block reuses the host
    arrays of the first block of its kind (local or global) wherever the
    tensors' shapes agree (a many-block model in the time of two)."""
    d, h, v = shape.embedding, shape.hidden, shape.vocabulary
    rng = np.random.default_rng(shape.seed)
    seed = [shape.seed * 1000]

    def matrix(kind: str, rows: int, cols: int):
        seed[0] += 1
        t = shape.types[kind]
        return t, (cols, rows), synth.weights(t, rows, cols, seed[0])

    def norm(n: int, scale: float = 1.0):
        w = (scale * (1.0 + 0.1 * rng.standard_normal(n))).astype(np.float32)
        return F32, (n,), w.view(np.uint8)

    out = [("token_embd.weight", *matrix("embedding", v, d)), ("output_norm.weight", *norm(d))]
    if not shape.tied_output:
        out.append(("output.weight", *matrix("output", v, d)))
    # Rotary factors of the global layers: most near 1, a few large (those
    # pairs barely turn).
    factors = (1.0 + rng.random(shape.width // 2)).astype(np.float32)
    factors[-4:] = 1e6
    out.append(("rope_freqs.weight", F32, (shape.width // 2,), factors.view(np.uint8)))
    first_of = {}
    for b in range(shape.blocks):
        w = shape.head_width(b)
        q, kv = shape.heads * w, shape.kv_heads * w
        blk = f"blk.{b}."
        kind = (shape.local[b], shape.shared(b), shape.local[b] or shape.global_value)
        if shared_blocks and kind in first_of:
            src = first_of[kind]
            out += [(name.replace(src, blk, 1), t, dims, data) for name, t, dims, data in out
                    if name.startswith(src) and not name.endswith("layer_output_scale.weight")]
        else:
            first_of[kind] = blk
            # Gemma's attention is unscaled: q/k norm weights near
            # width^(-1/4) keep the scores near unit variance, as a trained
            # model's norms do (with weights near 1 the random model's
            # softmax is so peaked that the engine's two CPU paths already
            # differ past their inference-test bounds).
            qk = w ** -0.25
            out += [(blk + "attn_norm.weight", *norm(d)), (blk + "attn_q.weight", *matrix("attention", q, d)),
                    (blk + "attn_q_norm.weight", *norm(w, qk))]
            if not shape.shared(b):
                out += [(blk + "attn_k.weight", *matrix("attention", kv, d)),
                        (blk + "attn_k_norm.weight", *norm(w, qk))]
                if shape.local[b] or shape.global_value:
                    out.append((blk + "attn_v.weight", *matrix("attention", kv, d)))
            out += [(blk + "attn_output.weight", *matrix("attention", d, q)),
                    (blk + "post_attention_norm.weight", *norm(d)), (blk + "ffn_norm.weight", *norm(d)),
                    (blk + "ffn_gate.weight", *matrix("gate_up", h, d)),
                    (blk + "ffn_up.weight", *matrix("gate_up", h, d)),
                    (blk + "ffn_down.weight", *matrix("down", d, h)), (blk + "post_ffw_norm.weight", *norm(d))]
        scale = shape.output_scales[b] if b < len(shape.output_scales) else None
        if scale is not None:
            out.append((blk + "layer_output_scale.weight", F32, (1,), np.array([scale], np.float32).view(np.uint8)))
    for name, t, dims, data in out:
        rows = dims[1] if len(dims) > 1 else 1
        assert data.nbytes == storage_bytes(t, rows, dims[0]), name
    return out


def _tensor_table(arrays):
    n = len(arrays)
    table = (Tensor * n)()
    index = {}
    for i, (name, t, dims, data) in enumerate(arrays):
        tt = table[i]
        tt.name = name.encode()
        tt.type, tt.dimension_count = t, len(dims)
        for k, v in enumerate(dims):
            tt.dimensions[k] = v
        tt.data, tt.data_size, tt.bound = data.ctypes.data, data.nbytes, 1
        index[name] = ctypes.pointer(tt)
    return table, index


class LlamaModel:
    """A nya_llm_context for a dense LLaMA over `tensors` (kept referenced)."""

    def __init__(self, shape: LlamaShape, tensors=None):
        self.shape = shape
        self.arrays = tensors if tensors is not None else llama_tensors(shape)
        n = len(self.arrays)
        self.tensors, index = _tensor_table(self.arrays)
        d, hd = shape.embedding, shape.embedding // shape.heads
        kvd = shape.kv_heads * hd
        self.layers = (Layer * shape.blocks)()
        for b in range(shape.blocks):
            L = self.layers[b]
            for fld, name in [("attention_norm", "attn_norm"), ("query", "attn_q"), ("key", "attn_k"),
                              ("value", "attn_v"), ("attention_output", "attn_output"), ("feed_forward_norm", "ffn_norm"),
                              ("feed_forward_gate", "ffn_gate"), ("feed_forward_down", "ffn_down"),
                              ("feed_forward_up", "ffn_up")]:
                setattr(L, fld, index[f"blk.{b}.{name}.weight"])
            L.head_count, L.kv_head_count, L.head_dimension = shape.heads, shape.kv_heads, hd
            L.hidden_length, L.kv_source, L.cache_offset = shape.hidden, b, b * kvd
        c = self.context = Context()
        c.tensors, c.tensor_count = self.tensors, n
        c.layers = self.layers
        c.tokenizer.vocabulary_size = shape.vocabulary
        c.token_embedding, c.output_norm, c.output = (index["token_embd.weight"], index["output_norm.weight"],
                                                      index["output.weight"])
        c.embedding_length, c.feed_forward_length, c.block_count = d, shape.hidden, shape.blocks
        c.head_count, c.key_value_head_count, c.context_length = shape.heads, shape.kv_heads, shape.context
        c.rope_dimension_count, c.head_dimension = hd, hd
        c.norm_epsilon, c.rope_frequency_base = shape.epsilon, shape.rope_base
        c.cache_width, c.maximum_query_length, c.maximum_hidden_length = shape.blocks * kvd, d, shape.hidden

    @property
    def weight_bytes(self) -> int:
        return sum(a[3].nbytes for a in self.arrays)

    def kv_width(self, layer: int) -> int:
        return self.shape.kv_heads * (self.shape.embedding // self.shape.heads)


class GemmaModel:
    """A nya_llm_context for a Gemma 4 text model over `tensors` (kept
    referenced), the fields the engine's loader sets
    (backend/core/llm_gguf.c:852-990, :1496-1497)."""

    def __init__(self, shape: GemmaShape, tensors=None):
        self.shape = shape
        self.arrays = tensors if tensors is not None else gemma_tensors(shape)
        self.tensors, index = _tensor_table(self.arrays)
        d = shape.embedding
        self.layers = (Layer * shape.blocks)()
        cache_width, offsets = 0, []
        for b in range(shape.blocks):
            L = self.layers[b]
            w = shape.head_width(b)
            get = lambda name: index.get(f"blk.{b}.{name}.weight")
            for fld, name in [("attention_norm", "attn_norm"), ("query", "attn_q"), ("key", "attn_k"),
                              ("value", "attn_v"), ("attention_output", "attn_output"), ("feed_forward_norm", "ffn_norm"),
                              ("feed_forward_gate", "ffn_gate"), ("feed_forward_down", "ffn_down"),
                              ("feed_forward_up", "ffn_up"), ("query_norm", "attn_q_norm"),
                              ("key_norm", "attn_k_norm"), ("attention_post_norm", "post_attention_norm"),
                              ("ffn_post_norm", "post_ffw_norm"), ("output_scale", "layer_output_scale")]:
                t = get(name)
                if t is not None:
                    setattr(L, fld, t)
            if not shape.local[b]:
                L.rope_factors = index["rope_freqs.weight"]
            L.head_count, L.kv_head_count, L.head_dimension = shape.heads, shape.kv_heads, w
            L.hidden_length, L.sliding_window = shape.hidden, shape.window if shape.local[b] else 0
            L.kv_source = shape.kv_source(b)
            if L.kv_source == b:
                offsets.append(cache_width)
                cache_width += shape.kv_heads * w
            else:
                offsets.append(offsets[L.kv_source])
            L.cache_offset = offsets[b]
        c = self.context = Context()
        c.tensors, c.tensor_count = self.tensors, len(self.arrays)
        c.layers = self.layers
        c.tokenizer.vocabulary_size = shape.vocabulary
        c.token_embedding, c.output_norm = index["token_embd.weight"], index["output_norm.weight"]
        c.output = index["output.weight"] if not shape.tied_output else c.token_embedding
        c.embedding_length, c.feed_forward_length, c.block_count = d, shape.hidden, shape.blocks
        c.head_count, c.key_value_head_count, c.context_length = shape.heads, shape.kv_heads, shape.context
        c.rope_dimension_count, c.head_dimension = shape.width, shape.width
        c.sliding_head_dimension, c.sliding_window = shape.local_width, shape.window
        c.shared_kv_layers = shape.shared_kv_layers
        c.norm_epsilon, c.rope_frequency_base = shape.epsilon, shape.rope_base
        c.sliding_rope_base, c.final_logit_softcap = shape.local_rope_base, shape.softcap
        c.is_gemma = 1
        c.cache_width = cache_width
        c.maximum_query_length = shape.heads * max(shape.width, shape.local_width)
        c.maximum_hidden_length = shape.hidden

    @property
    def weight_bytes(self) -> int:
        return sum(a[3].nbytes for a in self.arrays)

    def kv_width(self, layer: int) -> int:
        return self.shape.kv_heads * self.shape.head_width(layer)


class Plan:
    """A resident plan of `model` on `compute` (nya_compute_plan_create)."""

    def __init__(self, compute: Compute, model: LlamaModel | GemmaModel, capacity: int):
        lib = compute._lib
        vp_, sz_ = ctypes.c_void_p, ctypes.c_size_t
        lib.nya_compute_plan_create.restype = vp_
        lib.nya_compute_plan_create.argtypes = [vp_, vp_, sz_]
        lib.nya_compute_plan_free.argtypes = [vp_]
        lib.nya_compute_plan_token.argtypes = [vp_, ctypes.c_uint, sz_, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
        lib.nya_compute_plan_prefill.argtypes = [vp_, ctypes.POINTER(ctypes.c_uint), sz_, sz_,
                                                 ctypes.POINTER(ctypes.c_float)]
        lib.nya_compute_plan_stats.argtypes = [vp_, ctypes.POINTER(ComputeStats)]
        self.lib, self.model, self.compute = lib, model, compute
        self.ptr = lib.nya_compute_plan_create(compute._ctx, ctypes.addressof(model.context), capacity)
        if not self.ptr:
            raise RuntimeError("the provider declined the resident plan (NYA_ROCM_DEBUG=1 prints why)")
        self.logits = np.empty(model.shape.vocabulary, np.float32)

    def token(self, token: int, position: int, logits: bool = True) -> np.ndarray | None:
        out = self.logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        if self.lib.nya_compute_plan_token(self.ptr, token, position, 1 if logits else 0, out if logits else None):
            raise RuntimeError(f"resident token failed at position {position}")
        return self.logits if logits else None

    def prefill(self, tokens, position: int) -> np.ndarray:
        arr = (ctypes.c_uint * len(tokens))(*tokens)
        out = self.logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        if self.lib.nya_compute_plan_prefill(self.ptr, arr, len(tokens), position, out):
            raise RuntimeError(f"resident prefill failed at position {position}")
        return self.logits

    def read_kv(self, layer: int, position: int, count: int) -> tuple[np.ndarray, np.ndarray]:
        """Keys and values of `count` cached positions of `layer`."""
        n = count * self.model.kv_width(layer)
        k, v = np.empty(n, np.float32), np.empty(n, np.float32)
        fp = ctypes.POINTER(ctypes.c_float)
        self.lib.nya_compute_plan_read_kv.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                                      ctypes.c_size_t, fp, fp, ctypes.c_size_t]
        if self.lib.nya_compute_plan_read_kv(self.ptr, layer, position, count, k.ctypes.data_as(fp),
                                             v.ctypes.data_as(fp), n):
            raise RuntimeError(f"resident KV read failed (layer {layer}, positions {position}..+{count})")
        return k, v

    def stats(self) -> dict:
        s = ComputeStats()
        self.lib.nya_compute_plan_stats(self.ptr, ctypes.byref(s))
        return s.as_dict()

    @property
    def verify_limit(self) -> int:
        self.lib.nya_compute_plan_verify_limit.restype = ctypes.c_size_t
        self.lib.nya_compute_plan_verify_limit.argtypes = [ctypes.c_void_p]
        return int(self.lib.nya_compute_plan_verify_limit(self.ptr))

    def verify(self, tokens, position: int, logits: bool = False):
        """Tokens [position, position + len(tokens)) in one batch
        (nya_compute_plan_verify): the target's greedy choice after each, and
        with `logits` the rows of logits too ([len(tokens)][vocabulary])."""
        n = len(tokens)
        arr = (ctypes.c_uint * n)(*tokens)
        ids = (ctypes.c_uint * n)()
        rows = np.empty((n, self.model.shape.vocabulary), np.float32) if logits else None
        fp = ctypes.POINTER(ctypes.c_float)
        self.lib.nya_compute_plan_verify.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint), ctypes.c_size_t,
                                                     ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint), fp]
        if self.lib.nya_compute_plan_verify(self.ptr, arr, n, position, ids,
                                            rows.ctypes.data_as(fp) if logits else None):
            raise RuntimeError(f"resident verification failed at position {position} ({n} tokens)")
        return (list(ids), rows) if logits else list(ids)

    def close(self):
        if self.ptr:
            self.lib.nya_compute_plan_free(self.ptr)
            self.ptr = None


class Speculation(ctypes.Structure):
    """nya_compute_speculation (include/compute.h)."""
    _fields_ = [(name, ctypes.c_size_t) for name in
                ("generated", "rounds", "draft_tokens", "accepted", "target_tokens", "draft_steps")]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def generate_greedy(target: Plan, draft: Plan | None, prompt, limit: int, window: int = 4, stops=()):
    """Greedy generation on `target` with batched speculative verification
    against `draft` (nya_compute_generate_greedy): (tokens, counters). Both
    plans must be empty and hold len(prompt) + limit positions."""
    lib = target.lib
    u = ctypes.POINTER(ctypes.c_uint)
    lib.nya_compute_generate_greedy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, u, ctypes.c_size_t, ctypes.c_size_t,
                                                ctypes.c_size_t, u, ctypes.c_size_t, u,
                                                ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(Speculation)]
    p = (ctypes.c_uint * len(prompt))(*prompt)
    st = (ctypes.c_uint * max(len(stops), 1))(*stops)
    out = (ctypes.c_uint * limit)()
    count, stats = ctypes.c_size_t(), Speculation()
    if lib.nya_compute_generate_greedy(target.ptr, draft.ptr if draft else None, p, len(prompt), window, limit, st,
                                       len(stops), out, ctypes.byref(count), ctypes.byref(stats)):
        raise RuntimeError("greedy generation failed")
    return list(out[:count.value]), stats.as_dict()


class Sampling(ctypes.Structure):
    """nya_compute_sampling (include/compute.h)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_size_t),
                ("seed", ctypes.c_uint64)]


def generate_sampled(target: Plan, draft: Plan | None, prompt, limit: int, temperature: float, top_p: float = 1.0,
                     top_k: int = 0, seed: int = 0, window: int = 4, stops=()):
    """Generation at `temperature` with the engine's exact speculative
    sampling over batched verification (nya_compute_generate_sampled):
    (tokens, counters). Both plans must be empty and hold len(prompt) + limit
    positions."""
    lib = target.lib
    u = ctypes.POINTER(ctypes.c_uint)
    lib.nya_compute_generate_sampled.argtypes = [ctypes.c_void_p, ctypes.c_void_p, u, ctypes.c_size_t,
                                                 ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(Sampling), u,
                                                 ctypes.c_size_t, u, ctypes.POINTER(ctypes.c_size_t),
                                                 ctypes.POINTER(Speculation)]
    p = (ctypes.c_uint * len(prompt))(*prompt)
    st = (ctypes.c_uint * max(len(stops), 1))(*stops)
    out = (ctypes.c_uint * limit)()
    count, stats = ctypes.c_size_t(), Speculation()
    s = Sampling(temperature, top_p, top_k, seed)
    if lib.nya_compute_generate_sampled(target.ptr, draft.ptr if draft else None, p, len(prompt), window, limit,
                                        ctypes.byref(s), st, len(stops), out, ctypes.byref(count),
                                        ctypes.byref(stats)):
        raise RuntimeError("sampled generation failed")
    return list(out[:count.value]), stats.as_dict()
