"""GPU parity of the fp16-activation batched decode path (q355_gemm_q4_0_f16, q355_rmsnorm_fix_f16,
q355_attn_decode_f16) against the oracle's fp16 forms (oracle/quant.py:gemv_q4_0_f16,
dequant_q4_0_f16; oracle/model.py rmsnorm / attn_decode rounded to fp16)."""
import math

import numpy as np
import pytest

from lab import gguf
from lab import qwen_model as QM
from lab.hip import HipError, call, ptr
from oracle import model as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
REL = 1e-4            # same fp16 products on both sides; only the fp32 summation order differs
_KEEP = []


@pytest.fixture(autouse=True)
def _keep_alive():
    yield
    _KEEP.clear()


def dev(a):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


def relerr(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def sync():
    import torch
    torch.cuda.synchronize()


def mat(N, K, seed):
    w = np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    b = gguf.quantize_q4_0(w)
    return QM.Q4Mat(b, N, K, "cuda"), b


def acts(T, K, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((T, K)) * scale).astype(np.float16)


@pytest.mark.parametrize("N,K,T", [(2048, 1536, 1), (1536, 1536, 8), (8960, 1536, 17), (1536, 8960, 32),
                                   (4096, 1536, 40), (1024, 1568, 64)])
def test_gemm_f16_store(cuda, N, K, T):
    import torch
    W, b = mat(N, K, N + K + T)
    x = acts(T, K, T)
    y = torch.zeros(T, N, device=cuda)
    call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), N, K, ptr(dev(x)), T, 0, ptr(y), None, None, None, None)
    sync()
    assert relerr(y.cpu().numpy(), OQ.gemv_q4_0_f16(b, N, K, x)) < REL


@pytest.mark.parametrize("N,K,T", [(1536, 8960, 32), (2048, 1536, 8), (1536, 1536, 33)])
def test_gemm_f16_resid_fix(cuda, N, K, T):
    W, b = mat(N, K, 7 * N + K)
    rng = np.random.default_rng(N)
    x = acts(T, K, K + T)
    h0 = rng.standard_normal((T, N), dtype=np.float32)
    h = dev(np.round(h0.astype(np.float64) * QM.FIX_SCALE).astype(np.int64))
    call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), N, K, ptr(dev(x)), T, 6, None, ptr(h), None, None, None)
    sync()
    got = h.cpu().numpy() / QM.FIX_SCALE - h0
    assert relerr(got, OQ.gemv_q4_0_f16(b, N, K, x)) < REL


@pytest.mark.parametrize("T", [5, 24, 64])
def test_gemm_f16_swiglu(cuda, T):
    import torch
    F, K = 8960, 1536
    g = np.random.default_rng(1).standard_normal((F, K), dtype=np.float32) * np.float32(0.02)
    u = np.random.default_rng(2).standard_normal((F, K), dtype=np.float32) * np.float32(0.02)
    gb, ub = gguf.quantize_q4_0(g), gguf.quantize_q4_0(u)
    gu = gguf.take_rows_q4_0(np.concatenate([gb, ub]), K, gguf.gate_up_row_order(F))
    W = QM.Q4Mat(gu, 2 * F, K, "cuda")
    x = acts(T, K, 3)
    m = torch.zeros(T, F, dtype=torch.float16, device=cuda)
    call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), 2 * F, K, ptr(dev(x)), T, 8, None, None, ptr(m), None, None)
    sync()
    ref = OM.silu_mul(OQ.gemv_q4_0_f16(gb, F, K, x), OQ.gemv_q4_0_f16(ub, F, K, x))
    got = m.cpu().numpy().astype(np.float64)
    assert relerr(got, ref) < 2e-3                   # fp16 output rounding (2^-11) + fp32 SiLU
    assert np.abs(got - ref).max() <= np.abs(ref).max() * 2e-3


@pytest.mark.parametrize("V,T", [(8192, 20), (4096, 33)])
def test_gemm_f16_logits_argmax(cuda, V, T):
    import torch
    K = 1536
    W, b = mat(V, K, 99)
    x = acts(T, K, 4)
    n = call("q355_mmq_nparts", V)
    y = torch.zeros(T, V, device=cuda)
    pm = torch.zeros(T, n, device=cuda)
    pi = torch.zeros(T, n, dtype=torch.int32, device=cuda)
    call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), V, K, ptr(dev(x)), T, 5, ptr(y), None, None, ptr(pm), ptr(pi))
    tok = torch.zeros(T, dtype=torch.int32, device=cuda)
    pos = torch.zeros(T, dtype=torch.int32, device=cuda)
    call("q355_finish", ptr(pm), ptr(pi), n, ptr(tok), ptr(pos), T)
    sync()
    yy = y.cpu().numpy()
    assert relerr(yy, OQ.gemv_q4_0_f16(b, V, K, x)) < REL
    assert tok.cpu().numpy().tolist() == [int(np.argmax(r)) for r in yy]


def test_gemm_f16_bad_args(cuda):
    with pytest.raises(HipError, match="epi"):
        call("q355_gemm_q4_0_f16", 1, 1, 64, 64, 1, 1, 3, None, None, None, None, None)
    with pytest.raises(HipError, match="multiple of 64"):
        call("q355_gemm_q4_0_f16", 1, 1, 48, 64, 1, 1, 0, 1, None, None, None, None)


@pytest.mark.parametrize("T", [1, 7, 32])
def test_rmsnorm_fix_f16(cuda, T):
    import torch
    H = 1536
    rng = np.random.default_rng(T)
    h = rng.standard_normal((T, H)) * 3
    hf = np.round(h * QM.FIX_SCALE).astype(np.int64)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    xh = torch.zeros(T, H, dtype=torch.float16, device=cuda)
    call("q355_rmsnorm_fix_f16", ptr(dev(hf)), ptr(dev(w)), ptr(xh), T, H, 1e-6)
    sync()
    ref = OM.rmsnorm(hf / QM.FIX_SCALE, w, 1e-6).astype(np.float16)
    got = xh.cpu().numpy()
    # one f64 -> fp16 rounding on both sides: equal but for last-ulp ties of the f64 sum order
    ulp = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1 and (ulp > 0).mean() < 1e-3


@pytest.mark.parametrize("positions", [[0, 63], [64, 511], [1000, 5, 700, 130]])
def test_attn_decode_f16(cuda, positions):
    import torch
    c = QM.Config(L=1, V=1024)
    T = len(positions)
    max_chunks = 16
    rng = np.random.default_rng(sum(positions))
    n_pages = T * max_chunks
    kc = rng.standard_normal((n_pages, c.NKV, 64, c.HD)).astype(np.float16)
    vc = rng.standard_normal((n_pages, c.NKV, 64, c.HD)).astype(np.float16)
    bt = rng.permutation(n_pages).astype(np.int32).reshape(T, max_chunks)
    q = (rng.standard_normal((T, c.NH * c.HD)) * 2).astype(np.float16)
    pos = np.array(positions, np.int32)
    part = torch.zeros(T, c.NH, max_chunks, c.HD + 2, dtype=torch.float64, device=cuda)
    oh = torch.zeros(T, c.NH * c.HD, dtype=torch.float16, device=cuda)
    call("q355_attn_decode_f16", ptr(dev(q)), ptr(dev(kc)), ptr(dev(vc)), ptr(dev(pos)), ptr(dev(bt)), max_chunks,
         c.NH, c.NKV, max_chunks, 1 / math.sqrt(c.HD), ptr(part), ptr(oh), T)
    sync()
    for j in range(T):
        K = np.concatenate([kc[bt[j, p]] for p in range(max_chunks)], axis=1)
        V = np.concatenate([vc[bt[j, p]] for p in range(max_chunks)], axis=1)
        ref = OM.attn_decode(q[j].reshape(c.NH, c.HD), K, V, int(pos[j]) + 1, c.NH, c.NKV)
        assert relerr(oh[j].float().cpu().numpy(), ref) < 2e-3   # fp16 P on the matrix cores, fp16 output


@pytest.mark.parametrize("T", [5, 8, 20, 32])
def test_gemm_f16_qkv_rope_equals_finish(cuda, T):
    """QKV with bias, RoPE and the K/V write in the fp16 product's epilogue equals the K-split product into the
    int64 accumulator followed by q355_qkv_finish (one token per sequence, scattered pages)."""
    import torch
    c = QM.Config(L=1, V=1024)
    N, K = c.nqkv, c.H
    W, _ = mat(N, K, 40 + T)
    rng = np.random.default_rng(T)
    x = dev(acts(T, K, T + 1))
    bias = dev(rng.standard_normal(N).astype(np.float32))
    maxlen, bt_stride = 1024, 8
    ang = np.arange(maxlen)[:, None] * (1e6 ** (-np.arange(64) * 2 / 128))[None, :]
    cos, sin = dev(np.cos(ang).astype(np.float32)), dev(np.sin(ang).astype(np.float32))
    pos = dev(rng.integers(0, bt_stride * 64, T).astype(np.int32))
    table = dev(rng.permutation(T * bt_stride).astype(np.int32).reshape(T, bt_stride))
    outs = []
    for fused in (True, False):
        kc = torch.zeros(T * bt_stride, c.NKV, 64, 128, dtype=torch.float16, device=cuda)
        vc = torch.zeros_like(kc)
        q = torch.zeros(T, c.NH * 128, dtype=torch.float16, device=cuda)
        if fused:
            call("q355_gemm_f16_qkv_rope", ptr(W.qs), ptr(W.d), N, K, ptr(x), T, ptr(bias), ptr(cos), ptr(sin),
                 ptr(pos), ptr(table), bt_stride, 1, ptr(kc), ptr(vc), ptr(q), c.NH, c.NKV)
        else:
            acc = torch.zeros(T, N, dtype=torch.int64, device=cuda)
            call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), N, K, ptr(x), T, 6, None, ptr(acc), None, None, None)
            call("q355_qkv_finish", ptr(acc), ptr(bias), ptr(cos), ptr(sin), ptr(pos), ptr(table), bt_stride, 1,
                 ptr(kc), ptr(vc), ptr(q), c.NH, c.NKV, T)
        sync()
        outs.append([t.cpu().numpy() for t in (q, kc, vc)])
    # the fused product sums all of K in one fp32 accumulator, the split one in K slices: the fp32 sums differ
    # in their last bits, so an fp16 output may round one or two ulps apart
    for a, b in zip(*outs):
        ulp = np.abs(a.view(np.int16).astype(np.int32) - b.view(np.int16).astype(np.int32))
        assert ulp.max() <= 2 and (ulp > 0).mean() < 1e-3
        assert relerr(a.astype(np.float32), b.astype(np.float32)) < 2e-3
    with pytest.raises(HipError, match="T <= 32"):
        call("q355_gemm_f16_qkv_rope", ptr(W.qs), ptr(W.d), N, K, ptr(x), 33, ptr(bias), ptr(cos), ptr(sin),
             ptr(pos), ptr(table), bt_stride, 1, ptr(kc), ptr(vc), ptr(q), c.NH, c.NKV)
