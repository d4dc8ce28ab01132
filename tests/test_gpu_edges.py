"""Edge shapes through sgl_qlinear_forward against the reference CPU path (oracle dequant +
sgl_matmul_nt, or sgl_matmul_w8a16 for W8): a single output column, N below one 16-column
tile, K of one packed word (below one group), K below one MXFP4 block, many row blocks, and an
empty batch.  Tolerance (BASELINE): max|y - y_ref| / max|y_ref| <= 1e-3."""
import numpy as np
import pytest

from test_gpu_linear import _run

pytestmark = pytest.mark.gpu

MS = [1, 2, 9, 17, 40, 300]


def test_one_output_column(orc):
    """N = 1 (MXFP4 and W8 take any N)."""
    _run(orc, "mxfp4", 1, 256, MS)
    _run(orc, "w8", 1, 200, MS)


def test_n_below_one_tile(orc):
    """N = 8: every tile is partial."""
    _run(orc, "gptq4", 8, 512, MS)
    _run(orc, "awq4", 8, 384, MS)
    _run(orc, "gptq8", 8, 256, MS)


def test_k_of_one_word(orc):
    """K = 8 (one packed int4 word, far below one 128-element group), K = 3 for W8, and
    K = 20 for MXFP4 (below one 32-element block)."""
    _run(orc, "gptq4", 64, 8, MS)
    _run(orc, "w8", 48, 3, MS)
    _run(orc, "mxfp4", 48, 20, MS)


def test_many_row_blocks(orc):
    """5000 rows: many 128- and 256-row blocks, ragged at both ends of the grid."""
    _run(orc, "gptq4", 200, 512, [5000], dtypes=("bf16",))
    _run(orc, "w8", 96, 320, [3001], dtypes=("f32",))


@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4", "w8"])
def test_empty_batch(orc, fmt):
    """M = 0: nothing is read or written, and the call succeeds."""
    import torch
    from linear_cases import build, product
    kind, a = build(fmt, 64, 256, seed=5)
    ql = product(kind, a, 64, 256)
    y = ql.forward(torch.zeros((0, 256), dtype=torch.float32, device="cuda"))
    assert tuple(y.shape) == (0, 64)
