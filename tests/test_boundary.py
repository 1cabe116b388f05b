"""The C-ABI boundary on the CPU: both native libraries load and export every
function their public headers declare, the host-side queries answer as
documented, and the weight packer is the byte permutation the device layout
specifies (fyodor_amd/csrc/formats.h). Nothing here launches GPU work."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, KERNEL_LIBRARY, PROVIDER_LIBRARY, Q4_0, Q4_K, Q6_K, Q8_0, storage_bytes, synth
from fyodor_amd.hip import Kernels

INCLUDE = Path(__file__).resolve().parent.parent / "include"


def declared(header: str) -> set:
    text = (INCLUDE / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nya_[a-z0-9_]+)\s*\(", text))


def exported(lib: Path) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_kernel_library_exports_its_header():
    want = declared("fyodor_hip.h")
    assert want == {"nya_hip_abi_version", "nya_hip_weight_bytes", "nya_hip_weight_layout", "nya_hip_weight_pack",
                    "nya_hip_workspace_bytes", "nya_hip_matmul", "nya_hip_matmul_static", "nya_hip_kernel_name",
                    "nya_hip_copy", "nya_hip_read", "nya_hip_read_shaped", "nya_hip_step", "nya_hip_embed", "nya_hip_rms_norm",
                    "nya_hip_rope_qkv", "nya_hip_attention", "nya_hip_attention_split", "nya_hip_silu_mul", "nya_hip_greedy",
                    "nya_hip_matvec_gated", "nya_hip_matvec_swiglu", "nya_hip_matvec_residual",
                    "nya_hip_matvec_swiglu_scaled", "nya_hip_silu_pairs",
                    "nya_hip_matvec_normed", "nya_hip_matvec_normed_rope", "nya_hip_matvec_scaled_rope",
                    "nya_hip_post_norm", "nya_hip_head_norm_rope", "nya_hip_gelu_mul", "nya_hip_softcap",
                    "nya_hip_matvec_geglu", "nya_hip_gelu_pairs", "nya_hip_matvec_rope_pair"}
    assert want <= exported(KERNEL_LIBRARY)


def test_provider_library_exports_compute_api():
    want = declared("compute.h") | declared("compute_backend.h")
    assert "nya_rocm_backend" in want and "nya_compute_matmul_typed" in want
    assert {"nya_compute_plan_verify", "nya_compute_generate_greedy", "nya_compute_generate_sampled",
            "nya_rocm_plan_verify"} <= want
    missing = want - exported(PROVIDER_LIBRARY)
    assert not missing, missing


def test_provider_needs_no_rocm_link():
    """The C provider resolves HIP at run time (rocm/rocm.c:155-166)."""
    out = subprocess.run(["ldd", str(PROVIDER_LIBRARY)], capture_output=True, text=True).stdout
    assert "amdhip64" not in out and "fyodor_hip" not in out


@pytest.fixture(scope="module")
def kernels():
    return Kernels()


@pytest.mark.parametrize("t,block_bytes", [(Q4_0, 18), (Q8_0, 34), (Q4_K, 144), (Q6_K, 210)])
def test_unaddressable_block_matrices_decline(kernels, t, block_bytes):
    """A block-format matrix above INT32_MAX bytes (the kernels' 32-bit
    buffer range and tile offsets) or rows above 2^26 columns are declined
    by every entry point before anything is enqueued; the largest one that
    fits is accepted. Dense types are addressed with 64-bit offsets."""
    L = kernels.lib
    b = ctypes.c_size_t()
    block = 32 if t in (Q4_0, Q8_0) else 256
    cols = 4096
    row = cols // block * block_bytes
    fits = (2**31 - 1) // row
    assert L.nya_hip_weight_bytes(t, fits, cols, ctypes.byref(b)) == 0 and b.value == fits * row <= 2**31 - 1
    for rows, c in [(fits + 1, cols), (1, (1 << 26) + block)]:
        assert L.nya_hip_weight_bytes(t, rows, c, ctypes.byref(b)) == 1
        assert L.nya_hip_workspace_bytes(t, rows, c, 1, ctypes.byref(b)) == 1
        assert L.nya_hip_weight_pack(16, 16, t, rows, c) == 1
        assert L.nya_hip_kernel_name(t, rows, c, 1) is None
        # Declined on the shape alone: the (never dereferenced) addresses are
        # aligned, so nothing else would refuse the call.
        assert L.nya_hip_matmul(1 << 20, t, rows, c, 1 << 20, 1 << 20, 1, 0, 0, 0) == 1
    assert L.nya_hip_weight_bytes(F32, 40000, 20000, ctypes.byref(b)) == 0 and b.value == 40000 * 20000 * 4


def test_queries(kernels):
    L = kernels.lib
    assert L.nya_hip_abi_version() == 2
    b = ctypes.c_size_t()
    for t, block, size in [(F32, 1, 4), (F16, 1, 2), (BF16, 1, 2), (Q4_0, 32, 18), (Q8_0, 32, 34),
                           (Q4_K, 256, 144), (Q6_K, 256, 210)]:
        assert L.nya_hip_weight_bytes(t, 3, 4 * block, ctypes.byref(b)) == 0 and b.value == 3 * 4 * size
        assert L.nya_hip_weight_bytes(t, 3, 4 * block + (block > 1), ctypes.byref(b)) == (1 if block > 1 else 0)
        assert L.nya_hip_weight_layout(t) == (0 if block == 1 else 1)
        assert L.nya_hip_workspace_bytes(t, 3, 4 * block, 2, ctypes.byref(b)) == 0
    assert L.nya_hip_weight_bytes(99, 3, 32, ctypes.byref(b)) == 1 and L.nya_hip_weight_layout(99) == -1
    assert L.nya_hip_weight_bytes(Q8_0, 0, 32, ctypes.byref(b)) == 1
    assert L.nya_hip_weight_bytes(Q8_0, 1 << 31, 32, ctypes.byref(b)) == 1
    assert L.nya_hip_matmul(0, Q8_0, 3, 32, 16, 16, 1, 0, 0, 0) == 1          # declined, nothing enqueued
    assert kernels.kernel_name(Q4_K, 14336, 4096, 1) == "matvec_rows"          # up to 64 rows per CU
    assert kernels.kernel_name(Q4_K, 20480, 4096, 1) == "matvec_rows"          # three tiles, up to 80 rows
    assert kernels.kernel_name(Q4_K, 20481, 4096, 1) == "matvec_q4k"
    assert kernels.kernel_name(Q4_K, 57344, 4096, 1) == "matvec_q4k"           # one workgroup per tile
    assert kernels.kernel_name(Q8_0, 4096, 800, 1) == "smalln_mfma"            # a short last group
    assert kernels.kernel_name(Q4_K, 14336, 4096, 8) == "smalln_rows"          # digits made in the kernel
    assert kernels.kernel_name(Q4_K, 4096, 14336, 8) == "smalln_rows"          # several groups per wavefront
    assert kernels.kernel_name(Q4_K, 14336, 8192, 8) == "smalln_mfma"          # that, at two tiles per CU
    assert kernels.kernel_name(Q6_K, 4096, 4096, 8) == "smalln_rows"
    assert kernels.kernel_name(Q6_K, 14336, 4096, 8) == "smalln_rows"          # one workgroup per tile
    assert kernels.kernel_name(Q6_K, 4096, 14336, 8) == "smalln_rows"          # wide Q6_K rows: eight wavefronts
    assert kernels.kernel_name(Q6_K, 4096, 14336, 1) == "matvec_rows"
    assert kernels.kernel_name(Q6_K, 128256, 4096, 1) == "matvec_rows"         # one tile per workgroup


def unpack_reference(dev: np.ndarray, t: int, rows: int, cols: int) -> np.ndarray:
    """Inverse of the tiled device layout, written from its specification:
    tiles of 32 rows, 256-column groups, fields stored [field][row]."""
    block, nbytes = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}[t]
    row_bytes = cols // block * nbytes
    out = np.empty((rows, row_bytes), dtype=np.uint8)
    groups = -(-cols // 256)
    for t0 in range(0, rows, 32):
        R = min(32, rows - t0)
        tile = dev[t0 * row_bytes:(t0 + R) * row_bytes]
        for g in range(groups):
            if t == Q4_K:
                grp = tile[144 * R * g:144 * R * (g + 1)]
                blk = out[t0:t0 + R, 144 * g:144 * (g + 1)]
                sl = grp[128 * R:144 * R].reshape(R, 16).view(np.uint32)   # [R, 4]
                for p in range(4):
                    blk[:, 16 + 32 * p:32 + 32 * p] = grp[32 * R * p:32 * R * p + 16 * R].reshape(R, 16)
                    blk[:, 32 + 32 * p:48 + 32 * p] = grp[32 * R * p + 16 * R:32 * R * (p + 1)].reshape(R, 16)
                    blk[:, p] = (sl[:, p] >> 24).astype(np.uint8)
                sc = [(sl[:, g2 // 2] >> (12 * (g2 % 2))) & 63 for g2 in range(8)]
                mn = [(sl[:, g2 // 2] >> (12 * (g2 % 2) + 6)) & 63 for g2 in range(8)]
                for k in range(4):
                    blk[:, 4 + k] = sc[k] | ((sc[k + 4] >> 4) << 6)
                    blk[:, 8 + k] = mn[k] | ((mn[k + 4] >> 4) << 6)
                    blk[:, 12 + k] = (sc[k + 4] & 15) | ((mn[k + 4] & 15) << 4)
            elif t == Q6_K:
                grp = tile[208 * R * g:208 * R * (g + 1)]
                blk = out[t0:t0 + R, 210 * g:210 * (g + 1)]
                sc = grp[192 * R:208 * R].reshape(R, 4, 4)
                for h in range(2):
                    for l16 in range(2):
                        p = 2 * h + l16
                        f = grp[48 * R * p:48 * R * (p + 1)].reshape(3, R, 16)
                        blk[:, 64 * h + 16 * l16:64 * h + 16 * l16 + 16] = f[0]
                        blk[:, 64 * h + 32 + 16 * l16:64 * h + 48 + 16 * l16] = f[1]
                        blk[:, 128 + 32 * h + 16 * l16:128 + 32 * h + 16 * l16 + 16] = f[2]
                        for q in range(4):
                            blk[:, 192 + 8 * h + 2 * q + l16] = sc[:, p, q]
                d = tile[208 * R * groups + 2 * R * g:208 * R * groups + 2 * R * (g + 1)].reshape(R, 2)
                blk[:, 208:210] = d
            else:
                quant = 32 if t == Q8_0 else 16
                nb = min(8, cols // 32 - 8 * g)
                grp = tile[(quant + 2) * 8 * R * g:(quant + 2) * 8 * R * g + (quant + 2) * nb * R]
                if nb == 8:
                    # Full group: the row's eight scales together; Q4_0 quants in
                    # units of two blocks (low nibble block 2p, high 2p + 1).
                    dd = grp[8 * quant * R:8 * quant * R + 16 * R].reshape(R, 8, 2)
                    for j in range(8):
                        c0 = (quant + 2) * (8 * g + j)
                        out[t0:t0 + R, c0:c0 + 2] = dd[:, j]
                        if t == Q8_0:   # two halves of 16 columns, each [row][16]
                            halves = grp[32 * R * j:32 * R * (j + 1)].reshape(2, R, 16)
                            out[t0:t0 + R, c0 + 2:c0 + 34] = np.concatenate([halves[0], halves[1]], axis=1)
                    if t == Q4_0:
                        for p in range(4):
                            u = grp[32 * R * p:32 * R * (p + 1)].reshape(2, R, 16)   # [half][row][n]
                            for m in range(2):
                                e = (u >> (4 * m)) & 15                              # element 16h + n of block 2p + m
                                c0 = 18 * (8 * g + 2 * p + m)
                                out[t0:t0 + R, c0 + 2:c0 + 18] = e[0] | (e[1] << 4)
                else:
                    for j in range(nb):
                        c0 = (quant + 2) * (8 * g + j)
                        q = grp[quant * R * j:quant * R * (j + 1)]
                        if t == Q8_0:
                            q = np.concatenate(list(q.reshape(2, R, 16)), axis=1)
                        out[t0:t0 + R, c0 + 2:c0 + 2 + quant] = q.reshape(R, quant)
                        out[t0:t0 + R, c0:c0 + 2] = grp[quant * R * nb + 2 * R * j:quant * R * nb + 2 * R * (j + 1)].reshape(R, 2)
    return out.reshape(-1)


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(5, 1024), (70, 768), (33, 256), (9, 800)])
def test_pack_is_the_specified_permutation(kernels, t, rows, cols):
    if cols % {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}[t]:
        pytest.skip("shape not representable")
    w = synth.weights(t, rows, cols, 21)   # random scale bytes: every 12-byte pattern
    dev = kernels.device_weights(w, t, rows, cols)
    assert dev.nbytes == w.nbytes and not np.shares_memory(dev, w)
    assert np.array_equal(unpack_reference(dev, t, rows, cols), w)


def test_prefill_dispatch_and_workspace():
    """Batch 1 needs no workspace; batches of 2..8 need the activation digits
    of a padded token count; batches above 8 go to the prefill GEMM: fp16
    activation pieces for Q4_K/Q8_0/Q4_0 (per token, rounded up to 64
    tokens: two fp16 planes, the 32-column block sums and the scale), int8
    digits for Q6_K (rounded up to 32 tokens) -- except small batches of
    matrices the row-balanced small-N kernel takes, which run 8 tokens per
    launch up to a break-even batch (20 tokens from 8192 rows on, else 32;
    Q6_K only on rows wider than 4096 columns, up to 56); dense types need
    none, and run batches above 8 on their own GEMM (nothing is launched)."""
    kern = Kernels()

    def pieces(cols, batch):
        np_ = -(-batch // 64) * 64
        return np_ * (4 * cols + cols // 32 * 4 + 4)

    for t in (Q4_0, Q8_0, Q4_K, Q6_K):
        assert kern.workspace_bytes(t, 4096, 4096, 1) == 0
        # The row-balanced kernel needs no workspace (rows wider than 4096
        # columns and Q6_K: one tile per CU); the tile kernel keeps digits for
        # 8 or 4 slots.
        rows_kernel = True
        assert kern.workspace_bytes(t, 4096, 4096, 8) == (0 if rows_kernel else 4096 // 32 * 136 * 8)
        assert kern.workspace_bytes(t, 4096, 4096, 3) == (0 if rows_kernel else 4096 // 32 * 136 * 4)
        assert kern.workspace_bytes(t, 4096, 8192, 3) == (0 if rows_kernel else 8192 // 32 * 136 * 4)
        assert kern.workspace_bytes(t, 16384, 8192, 3) == 8192 // 32 * 136 * 4
        assert kern.kernel_name(t, 4096, 4096, 8) == ("smalln_rows" if rows_kernel else "smalln_mfma")
    for t in (Q4_0, Q8_0, Q4_K):
        for batch in (9, 32):
            assert kern.workspace_bytes(t, 4096, 4096, batch) == 0
            assert kern.kernel_name(t, 4096, 4096, batch) == "smalln_rows"
        assert kern.workspace_bytes(t, 4096, 4096, 33) == pieces(4096, 33)
        assert kern.workspace_bytes(t, 14336, 4096, 20) == 0
        assert kern.workspace_bytes(t, 14336, 4096, 21) == pieces(4096, 21)
        assert kern.kernel_name(t, 14336, 4096, 21) == "prefill_f16"
        assert kern.workspace_bytes(t, 4096, 4096, 512) == pieces(4096, 512)
        assert kern.kernel_name(t, 4096, 4096, 512) == "prefill_f16"
    assert kern.workspace_bytes(Q6_K, 4096, 14336, 56) == 0
    assert kern.kernel_name(Q6_K, 4096, 14336, 56) == "smalln_rows"
    assert kern.kernel_name(Q6_K, 4096, 14336, 57) == "prefill_mfma"
    assert kern.workspace_bytes(Q6_K, 4096, 4096, 9) == 4096 // 32 * 136 * 32
    assert kern.workspace_bytes(Q6_K, 4096, 4096, 512) == 4096 // 32 * 136 * 512
    assert kern.kernel_name(Q6_K, 4096, 4096, 512) == "prefill_mfma"
    for t in (F32, F16, BF16):
        assert kern.workspace_bytes(t, 4096, 4096, 512) == 0
        assert kern.kernel_name(t, 4096, 4096, 8) == "skinny_dense"
        assert kern.kernel_name(t, 4096, 4096, 9) == "dense_gemm"
        assert kern.kernel_name(t, 4096, 4096, 512) == "dense_gemm"


def test_model_header_layout_matches_engine(tmp_path):
    """fyodor_amd/core/llm_internal.h lays out the engine's model types as
    backend/core/llm_internal.h does (the provider reads the engine's
    nya_llm_context by address): every member the resident plan reads, and
    the sizes of the structures, compiled against both headers."""
    ref_core = Path("/root/reference/backend/core")
    if not (ref_core / "llm_internal.h").exists():
        pytest.skip("reference sources not mounted")
    fields = {
        "nya_llm_context": ["compute", "tensors", "tensor_count", "layers", "tokenizer", "token_embedding",
                            "output_norm", "output", "embedding_length", "block_count", "context_length",
                            "norm_epsilon", "rope_frequency_base", "is_gemma", "is_assistant",
                            "per_layer_embedding_length", "expert_count", "final_logit_softcap", "cache_width",
                            "sliding_value_dimension"],
        "nya_llm_layer": ["attention_norm", "query", "key", "value", "attention_output", "feed_forward_norm",
                          "feed_forward_gate", "feed_forward_down", "feed_forward_up", "query_norm", "key_norm",
                          "attention_post_norm", "ffn_post_norm", "router", "ple_gate", "output_scale",
                          "rope_factors", "head_count", "kv_head_count", "head_dimension", "hidden_length",
                          "sliding_window", "kv_source", "cache_offset"],
        "nya_llm_tensor": ["type", "dimension_count", "dimensions", "data", "data_size"],
        "nya_llm_tokenizer": ["vocabulary_size", "suppressed_tokens", "suppressed_count"],
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "llm_internal.h"', "int main(void) {"]
    for struct, names in fields.items():
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        lines += [f'printf("{struct}.{n} %zu\\n", offsetof({struct}, {n}));' for n in names]
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    out = {}
    for name, inc in [("ours", [INCLUDE.parent / "fyodor_amd/core", INCLUDE]),
                      ("engine", [ref_core, ref_core.parent / "include"])]:
        exe = tmp_path / name
        subprocess.run(["gcc", "-std=c17", *[f"-I{p}" for p in inc], str(src), "-o", str(exe)], check=True)
        out[name] = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    assert out["ours"] == out["engine"]
