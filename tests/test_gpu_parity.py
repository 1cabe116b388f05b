"""GPU parity of the ROCm provider against the oracle, through the C ABI.

Restates the reference kernel contract backend/tests/test_quant_kernels.c:
138-213 (all seven storage types, 65 rows, three input passes, a double
oracle bound of 1e-6 * (1 + sum |w x|) per row, the first 17 rows within
1.5e-4 * (1 + |y|) of the scalar kernel, matmul batches {3, 17, 65, 32, 8}
with canaries on both sides of the output; batches above 8 of the quantized
types run the MFMA prefill GEMM), then checks the benchmark shapes at
relative L2 <= 1e-5 against the scalar oracle on seeded data.
"""
import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, synth
from checks import check_rows, rel_l2
from patterns import batch_inputs, pass_input, pattern_matrix

pytestmark = pytest.mark.gpu

ALL_TYPES = [F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q6_K]
REL_L2 = 1e-5   # fp32 activations, reordered fp32 accumulation


@pytest.mark.parametrize("type_id", ALL_TYPES, ids=lambda t: TYPE_NAMES[t])
def test_reference_kernel_contract(compute, oracle, type_id):
    rows, cols = 65, 1024
    w = pattern_matrix(type_id, rows, cols)
    for p in range(3):
        x = pass_input(cols, p)
        y = compute.matvec_typed(w, rows, cols, type_id, x)
        check_rows(oracle, w, type_id, x, rows, cols, y, oracle.matvec(w, type_id, x, rows, cols), 17)
    inputs = batch_inputs(65, cols)
    for batch in (3, 17, 65, 32, 8):
        out = np.full(batch * rows + 2, 12345, dtype=np.float32)
        compute.matmul_typed(w, rows, cols, type_id, inputs[:batch], batch, out=out[1:1 + batch * rows])
        assert out[0] == 12345 and out[-1] == 12345
        y = out[1:-1].reshape(batch, rows)
        for token in range(batch):
            scalar = oracle.matvec(w, type_id, inputs[token], rows, cols) if token < 3 else None
            check_rows(oracle, w, type_id, inputs[token], rows, cols, y[token], scalar, 17 if token < 3 else 0)
    assert compute.name == "rocm"


@pytest.mark.parametrize("type_id", ALL_TYPES, ids=lambda t: TYPE_NAMES[t])
def test_long_rows(compute, oracle, type_id):
    """8192 columns (NYA_TEST_NATIVE_LONG, test_quant_kernels.c:142)."""
    rows, cols = 65, 8192
    w = pattern_matrix(type_id, rows, cols)
    for p in range(3):
        x = pass_input(cols, p)
        check_rows(oracle, w, type_id, x, rows, cols, compute.matvec_typed(w, rows, cols, type_id, x))


CONFIG_SHAPES = [
    (Q8_0, 4096, 4096, 1),
    (Q4_0, 4096, 4096, 1), (Q4_0, 11008, 4096, 1), (Q4_0, 4096, 11008, 1),
    (Q4_K, 4096, 4096, 1), (Q4_K, 1024, 4096, 1), (Q4_K, 14336, 4096, 1),
    (Q4_K, 20480, 4096, 1), (Q4_K, 24576, 4096, 1), (Q4_K, 28672, 4096, 1),
    (Q6_K, 4096, 14336, 1),
    (Q4_K, 4096, 4096, 2), (Q4_K, 4096, 4096, 4), (Q4_K, 4096, 4096, 8),
    (Q4_K, 14336, 4096, 2), (Q4_K, 14336, 4096, 4), (Q4_K, 14336, 4096, 8),
]


@pytest.mark.parametrize("type_id,rows,cols,batch", CONFIG_SHAPES,
                         ids=[f"{TYPE_NAMES[t]}-{r}x{c}-n{b}" for t, r, c, b in CONFIG_SHAPES])
def test_config_shapes(compute, oracle, type_id, rows, cols, batch):
    seed = type_id * 1000003 + rows * 7 + cols
    w = synth.weights(type_id, rows, cols, seed)
    x = synth.activations(batch, cols, seed)
    y = compute.matmul_typed(w, rows, cols, type_id, x, batch)
    expected = oracle.matmul(w, type_id, x, rows, cols, batch, threads=8)
    assert np.all(np.isfinite(y))
    err = rel_l2(y, expected)
    assert err <= REL_L2, f"relative L2 {err:.3g}"


@pytest.mark.parametrize("rows", [20000, 16400, 20480, 20481])
def test_q4k_three_tiles(compute, oracle, rows):
    """Q4_K at 65..80 rows per CU (the row-balanced kernel with three
    32-row tiles per workgroup): every row within the contract bound, the
    last workgroup short (20000 = 253 x 79 + 13, 16400 = 252 x 65 + 20),
    80 rows per CU exactly, and one row past it (matvec_q4k)."""
    cols = 2048
    w = synth.weights(Q4_K, rows, cols, rows)
    x = synth.activations(1, cols, rows + 1)[0]
    check_rows(oracle, w, Q4_K, x, rows, cols, compute.matvec_typed(w, rows, cols, Q4_K, x))


def test_output_head_q6k(compute, oracle):
    """Q6_K 128256 x 4096 output head (431 MB of packed weights)."""
    rows, cols = 128256, 4096
    w = synth.weights(Q6_K, rows, cols, 14)
    x = synth.activations(1, cols, 14)
    y = compute.matmul_typed(w, rows, cols, Q6_K, x, 1)
    expected = oracle.matmul(w, Q6_K, x, rows, cols, 1, threads=16)
    assert rel_l2(y, expected) <= REL_L2
