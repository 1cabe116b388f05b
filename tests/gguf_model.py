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
from pathlib import Path

from fyodor_amd.model import GemmaShape, LlamaShape, gemma_tensors, llama_tensors

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
