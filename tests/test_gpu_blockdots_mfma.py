"""Per-block int32 dots of the matrix-core (int8 MFMA) products, bit for bit.

The int8 MFMA kernels compute each Q4_0 x Q8_1 block as one v_mfma_i32 of the signed weights 16 (q - 8) against
the int8 activations, i.e. 16 (dot - 8 sum q_x), then scale it by d_w d_x / 16 in fp32 (the reference's MMQ
per-block formula, lab/qwen_batched.py:1099-1101, 1237-1243). To read every block's int32 value out of the fp32
output exactly, each weight row has ONE live block (the other blocks of the row carry the scale 0) and all
scales are powers of two: then y[t, n] = d_w d_x (dot - 8 sum q_x) is exact in fp32 and is compared with
oracle.quant.block_dots with np.array_equal. Rows of all-15 and all-0 nibbles and activations of +-127 are
included. The batch-1 GEMV (v_dot4 chains) is checked the same way.
"""
import numpy as np
import pytest

from lab import qwen_model as QM
from lab.hip import call, ptr
from oracle import quant as OQ

pytestmark = pytest.mark.gpu


def one_live_block_problem(N, K, T, seed):
    rng = np.random.default_rng(seed)
    nb = K // 32
    qs = rng.integers(0, 256, (N, nb, 16), dtype=np.uint8)
    qs[0] = 0xFF                                             # every weight 15 (value +7)
    qs[1] = 0x00                                             # every weight 0 (value -8)
    live = rng.integers(0, nb, N)
    dw = np.zeros((N, nb), np.float16)
    dw[np.arange(N), live] = (2.0 ** -rng.integers(2, 9, N)) * rng.choice([-1.0, 1.0], N)
    wb = np.concatenate([dw.view(np.uint8).reshape(N, nb, 2), qs], axis=2).reshape(-1, 18)
    xq = rng.integers(-127, 128, (T, K), dtype=np.int8)
    xq[0] = 127
    xq[min(1, T - 1)] = -127
    dx = (2.0 ** -rng.integers(2, 9, (T, nb))).astype(np.float16)
    # expected block values S = dot - 8 sum(q_x) of each row's live block, and y = d_w d_x S (exact)
    qw = OQ.q4_0_blocks(wb)[1].reshape(N, K)
    sq = xq.reshape(T, nb, 32).astype(np.int64).sum(axis=2)             # [T, nb]
    S = np.empty((T, N), np.int64)
    for b in np.unique(live):                                           # the live blocks' dots only
        rows = np.nonzero(live == b)[0]
        S[:, rows] = OQ.block_dots(qw[rows, 32 * b:32 * b + 32], xq[:, 32 * b:32 * b + 32])[:, :, 0] - 8 * sq[:, b:b + 1]
    y = (dw[np.arange(N), live].astype(np.float64)[None] * dx[:, live].astype(np.float64) * S)
    assert np.array_equal(y.astype(np.float32).astype(np.float64), y)   # exact in fp32 by construction
    return wb, xq, dx, S, y.astype(np.float32), dw[np.arange(N), live], live


def _run_mmq(cuda, N, K, T, seed):
    import torch
    wb, xq, dx, S, y_ref, dwl, live = one_live_block_problem(N, K, T, seed)
    W = QM.Q4Mat(wb, N, K, "cuda")
    xds = np.stack([dx, np.zeros_like(dx)], -1)
    xq_d, xds_d = torch.from_numpy(xq).cuda(), torch.from_numpy(xds).cuda()
    y = torch.full((T, N), float("nan"), device=cuda)
    call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq_d), ptr(xds_d), T, 0, ptr(y), None, None, None,
         None, None)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    # the int32 block values read back from the fp32 output
    s_got = got.astype(np.float64) / (dwl.astype(np.float64)[None] * dx[:, live].astype(np.float64))
    assert np.array_equal(s_got, S.astype(np.float64)), f"{int((s_got != S).sum())} block values differ"
    assert np.array_equal(got, y_ref)
    return T * N


@pytest.mark.parametrize("N,K,T", [(4096, 1536, 16),     # decode-batch kernel, one 16-token group
                                   (2048, 1536, 64),     # decode-batch kernel, four token groups
                                   (2048, 1536, 512),    # LDS-tiled prefill kernel (64-token tiles)
                                   (1536, 8960, 512)])   # LDS-tiled, the down projection's K
def test_mmq_block_dots_bitexact(cuda, N, K, T):
    n = _run_mmq(cuda, N, K, T, seed=N + K + T)
    assert n >= 65536


def test_gemv_block_dots_bitexact(cuda):
    """The batch-1 GEMV (v_dot4 int32 chains, f64 accumulation) on the same construction."""
    import torch
    N, K, T = 8960, 1536, 1
    wb, xq, dx, S, y_ref, dwl, live = one_live_block_problem(N, K, T, 7)
    W = QM.Q4Mat(wb, N, K, "cuda")
    xds = torch.from_numpy(np.stack([dx, np.zeros_like(dx)], -1)).cuda()
    xq_d = torch.from_numpy(xq).cuda()
    y = torch.full((T, N), float("nan"), device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq_d), ptr(xds), T, ptr(y), None, 0)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), y_ref)
