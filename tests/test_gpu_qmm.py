"""Dense quantized matmul (QmmCall, metal/lib.rs:357-380, 684-734) on the
GPU vs the oracle's sequential-FMA matvec per token row. Bar: max|d| /
max|ref| <= 1e-3 per token."""
import numpy as np
import pytest

from helpers import gen_quant_matrix, rel_err
from test_gpu_decode import dev, host, oracle_matvec, qweights

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.mark.parametrize("out_dim,in_dim,group,bits,n", [
    (512, 2048, 64, 4, 1),     # shared-expert gate/up shape, one token
    (2048, 512, 64, 4, 7),     # shared-expert down shape, ragged block
    (4096, 2048, 32, 4, 33),   # two 32-token blocks
    (1024, 1024, 128, 3, 64),  # packed 3-bit
    (256, 256, 64, 4, 100),    # four blocks, last ragged
    # Without GEMM tiles (one qmv per token row): Flash-Next's 640 and
    # 2560, a 7168-wide projection, a 96-input matrix.
    (640, 2560, 64, 4, 9), (2560, 640, 32, 3, 5), (300, 7168, 64, 4, 3), (64, 96, 32, 4, 17),
])
def test_qmm_matches_oracle(kernels, out_dim, in_dim, group, bits, n):
    import torch

    rng = np.random.default_rng(out_dim + 3 * in_dim + 7 * n + bits)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, group, bits)
    x = rng.standard_normal((n, in_dim)).astype(np.float32)
    w = qweights(codes, s, b, group, bits)
    y = torch.empty((n, out_dim), dtype=torch.float32, device="cuda")
    ws = torch.empty(kernels.qmm_workspace_size(in_dim, group, n), dtype=torch.uint8, device="cuda")
    assert kernels.qmm(w, dev(x), y, out_dim, in_dim, n, ws) == 0
    got = host(y)
    worst = 0.0
    for t in range(n):
        want, _ = oracle_matvec(codes, s, b, in_dim, out_dim, group, bits, x[t])
        worst = max(worst, rel_err(got[t], want))
    print(f"qmm {n}x{in_dim} -> {out_dim} g{group} {bits}-bit: worst rel_err {worst:.3e}")
    assert worst <= TOL


def test_qmm_argument_errors(kernels):
    import torch

    from streamoe_amd import _abi

    c = _abi.CODES
    rng = np.random.default_rng(5)
    codes, s, b = gen_quant_matrix(rng, 512, 2048, 64, 4)
    w = qweights(codes, s, b, 64, 4)
    x = torch.zeros((4, 2048), dtype=torch.float32, device="cuda")
    y = torch.zeros((4, 512), dtype=torch.float32, device="cuda")
    need = kernels.qmm_workspace_size(2048, 64, 4)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    small = torch.empty(need // 2, dtype=torch.uint8, device="cuda")
    assert kernels.qmm(w, x, y, 512, 2048, 4, small) == c["SMOE_ERR_WORKSPACE_TOO_SMALL"]
    assert kernels.qmm(w, x, y, 500, 2048, 4, ws) == 0  # out_dim % 256: one qmv per token row
    assert kernels.qmm(w, x, y, 512, 2048, 0, ws) == c["SMOE_ERR_INVALID_ARG"]
    assert kernels.qmm(w, x[:, 1:], y, 512, 2044, 4, ws) == c["SMOE_ERR_IN_DIM_NOT_MULTIPLE"]
