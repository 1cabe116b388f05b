"""Small random-weight LLaMA and Gemma models written as GGUF v3 files, for
inference parity tests of the resident plan against the engine's own CPU
session.

The file layout is the public GGUF v3 container: magic, version, tensor and
metadata counts; metadata as (key, type, value); tensor directory entries
(name, dimensions with the row length first, type, offset); then the tensor
data, each tensor aligned to `general.alignment`. The metadata keys and
tensor names are the ones the engine's loader binds for a dense LLaMA
(backend/core/llm_gguf.c:595-644, :1069-1077): embedding, output norm and
output, and per block the attention norm, q/k/v/output projections, the
feed-forward norm and gate/up/down projections, with every tensor used.

The shape and the tensors (seeded GGUF blocks of real-model scale, norm
weights 1 + N(0, 0.1)) are fyodor_amd.model's LlamaShape / llama_tensors; the
vocabulary is three control tokens and numbered pieces.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from fyodor_amd import F32, Q4_K, Q6_K, storage_bytes, synth
from fyodor_amd.model import LlamaShape, llama_tensors

# GGUF metadata value types.
U32, I32, F32_META, BOOL, STRING, ARRAY = 4, 5, 6, 7, 8, 9
ALIGNMENT = 32


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, kind: int, value) -> bytes:
    out = _string(key) + struct.pack("<I", kind)
    if kind == U32:
        return out + struct.pack("<I", value)
    if kind == F32_META:
        return out + struct.pack("<f", value)
    if kind == BOOL:
        return out + struct.pack("<B", 1 if value else 0)
    if kind == STRING:
        return out + _string(value)
    raise ValueError(kind)


def _array(key: str, elem: int, values) -> bytes:
    out = _string(key) + struct.pack("<IIQ", ARRAY, elem, len(values))
    if elem == STRING:
        return out + b"".join(_string(v) for v in values)
    fmt = {F32_META: "<f", I32: "<i", U32: "<I", BOOL: "<B"}[elem]
    return out + b"".join(struct.pack(fmt, v) for v in values)


tensors = llama_tensors


def _file(path: Path, meta: list[bytes], ts) -> int:
    directory, offset = [], 0
    for name, t, dims, data in ts:
        directory.append(_string(name) + struct.pack("<I", len(dims)) +
                         b"".join(struct.pack("<Q", n) for n in dims) + struct.pack("<IQ", t, offset))
        offset = (offset + data.nbytes + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    head = b"GGUF" + struct.pack("<IQQ", 3, len(ts), len(meta)) + b"".join(meta) + b"".join(directory)
    start = (len(head) + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)))
        at = 0
        for _, _, _, data in ts:
            f.write(data.tobytes())
            at += data.nbytes
            pad = (at + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT - at
            f.write(b"\0" * pad)
            at += pad
    return path.stat().st_size


@dataclass
class GemmaShape:
    """A small Gemma 4 text model as the engine's loader binds it
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


def gemma_tensors(shape: GemmaShape):
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
    for b in range(shape.blocks):
        w = shape.head_width(b)
        q, kv = shape.heads * w, shape.kv_heads * w
        blk = f"blk.{b}."
        # Gemma's attention is unscaled: q/k norm weights near width^(-1/4)
        # keep the scores near unit variance, as a trained model's norms do
        # (with weights near 1 the random model's softmax is so peaked that
        # the engine's two CPU paths already differ past the bounds).
        qk = w ** -0.25
        out += [(blk + "attn_norm.weight", *norm(d)), (blk + "attn_q.weight", *matrix("attention", q, d)),
                (blk + "attn_q_norm.weight", *norm(w, qk))]
        if not shape.shared(b):
            out += [(blk + "attn_k.weight", *matrix("attention", kv, d)), (blk + "attn_k_norm.weight", *norm(w, qk))]
            if shape.local[b] or shape.global_value:
                out.append((blk + "attn_v.weight", *matrix("attention", kv, d)))
        out += [(blk + "attn_output.weight", *matrix("attention", d, q)),
                (blk + "post_attention_norm.weight", *norm(d)), (blk + "ffn_norm.weight", *norm(d)),
                (blk + "ffn_gate.weight", *matrix("gate_up", h, d)), (blk + "ffn_up.weight", *matrix("gate_up", h, d)),
                (blk + "ffn_down.weight", *matrix("down", d, h)), (blk + "post_ffw_norm.weight", *norm(d))]
        scale = shape.output_scales[b] if b < len(shape.output_scales) else None
        if scale is not None:
            out.append((blk + "layer_output_scale.weight", F32, (1,), np.array([scale], np.float32).view(np.uint8)))
    for name, t, dims, data in out:
        rows = dims[1] if len(dims) > 1 else 1
        assert data.nbytes == storage_bytes(t, rows, dims[0]), name
    return out


def write_gemma(path: Path, shape: GemmaShape) -> int:
    """Writes the Gemma model (architecture "gemma4", its tokenizer model
    with one merge rule); returns its size in bytes."""
    pieces = ["<unk>", "<s>", "</s>"] + [f"p{i:04d}" for i in range(shape.vocabulary - 3)]
    g = "gemma4."
    meta = [
        _kv("general.architecture", STRING, "gemma4"),
        _kv("tokenizer.ggml.model", STRING, "gemma4"),
        _kv(g + "context_length", U32, shape.context),
        _kv(g + "embedding_length", U32, shape.embedding),
        _kv(g + "block_count", U32, shape.blocks),
        _kv(g + "attention.head_count", U32, shape.heads),
        _kv(g + "attention.head_count_kv", U32, shape.kv_heads),
        _kv(g + "feed_forward_length", U32, shape.hidden),
        _kv(g + "attention.key_length", U32, shape.width),
        _kv(g + "attention.value_length", U32, shape.width),
        _kv(g + "attention.key_length_swa", U32, shape.local_width),
        _kv(g + "attention.value_length_swa", U32, shape.local_width),
        _kv(g + "rope.dimension_count", U32, shape.width),
        _kv(g + "rope.dimension_count_swa", U32, shape.local_width),
        _kv(g + "attention.sliding_window", U32, shape.window),
        _kv(g + "attention.shared_kv_layers", U32, shape.shared_kv_layers),
        _array(g + "attention.sliding_window_pattern", BOOL, [1 if x else 0 for x in shape.local]),
        _kv(g + "attention.layer_norm_rms_epsilon", F32_META, shape.epsilon),
        _kv(g + "rope.freq_base", F32_META, shape.rope_base),
        _kv(g + "rope.freq_base_swa", F32_META, shape.local_rope_base),
        _kv(g + "final_logit_softcapping", F32_META, shape.softcap),
        _kv("tokenizer.ggml.unknown_token_id", U32, 0),
        _kv("tokenizer.ggml.bos_token_id", U32, 1),
        _kv("tokenizer.ggml.eos_token_id", U32, 2),
        _array("tokenizer.ggml.tokens", STRING, pieces),
        _array("tokenizer.ggml.scores", F32_META, [0.0] * len(pieces)),
        _array("tokenizer.ggml.token_type", I32, [3 if i in (1, 2) else 1 for i in range(len(pieces))]),
        _array("tokenizer.ggml.merges", STRING, ["p0000 p0001"]),
        _kv("general.alignment", U32, ALIGNMENT),
    ]
    return _file(path, meta, gemma_tensors(shape))


def write(path: Path, shape: LlamaShape, shared_blocks: bool = False) -> int:
    """Writes the model; returns its size in bytes. With `shared_blocks`
    every block stores block 0's tensor bytes (a many-block file in the
    generation time of one block)."""
    pieces = ["<unk>", "<s>", "</s>"] + [f"p{i:04d}" for i in range(shape.vocabulary - 3)]
    meta = [
        _kv("general.architecture", STRING, "llama"),
        _kv("tokenizer.ggml.model", STRING, "llama"),
        _kv("llama.embedding_length", U32, shape.embedding),
        _kv("llama.feed_forward_length", U32, shape.hidden),
        _kv("llama.block_count", U32, shape.blocks),
        _kv("llama.attention.head_count", U32, shape.heads),
        _kv("llama.attention.head_count_kv", U32, shape.kv_heads),
        _kv("llama.context_length", U32, shape.context),
        _kv("llama.attention.layer_norm_rms_epsilon", F32_META, shape.epsilon),
        _kv("llama.rope.freq_base", F32_META, shape.rope_base),
        _kv("tokenizer.ggml.unknown_token_id", U32, 0),
        _kv("tokenizer.ggml.bos_token_id", U32, 1),
        _kv("tokenizer.ggml.eos_token_id", U32, 2),
        _array("tokenizer.ggml.tokens", STRING, pieces),
        _array("tokenizer.ggml.scores", F32_META, [0.0] * len(pieces)),
        _array("tokenizer.ggml.token_type", I32, [3 if i in (1, 2) else 1 for i in range(len(pieces))]),
        _kv("tokenizer.ggml.add_eos_token", BOOL, False),
        _kv("general.alignment", U32, ALIGNMENT),
    ]
    return _file(path, meta, tensors(shape, shared_blocks=shared_blocks))
