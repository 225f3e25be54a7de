"""GPU edge cases: extreme shapes and positions, all-zero blocks, single-token prefill, decode batches up
to 64 sequences, the end of the KV cache."""
import math

import numpy as np
import pytest

from lab import gguf
from lab import qwen_batched as QB
from lab import qwen_model as QM
from lab.hip import call, ptr
from oracle import model as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
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


def q8(x):
    q, d, s = OQ.quantize_q8_1(x)
    return dev(q), dev(np.stack([d, s], -1)), q, d


@pytest.mark.parametrize("N,K,T", [(16, 32, 1), (64, 9216, 2), (48, 64, 4)])
def test_gemv_extreme_shapes(cuda, N, K, T):
    """Smallest tile / block, the largest K of the GEMV (9216), and T = 4."""
    import torch
    rng = np.random.default_rng(N * K + T)
    wb = gguf.quantize_q4_0(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    W = QM.Q4Mat(wb, N, K, "cuda")
    xq, xds, q, d = q8(rng.standard_normal((T, K), dtype=np.float32))
    y = torch.zeros(T, N, device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(y), None, 0)
    dots = torch.zeros(T, N, K // 32, dtype=torch.int32, device=cuda)
    call("q355_gemv_blockdots", ptr(W.qs), N, K, ptr(xq), T, ptr(dots))
    torch.cuda.synchronize()
    assert np.array_equal(dots.cpu().numpy(), OQ.block_dots(OQ.q4_0_blocks(wb)[1].reshape(N, K), q))
    assert relerr(y.cpu().numpy(), OQ.gemv_q4_0_q8_1(wb, N, K, q, d)) < 1e-3


def test_gemv_all_zero_activation_blocks(cuda):
    """Zero activation blocks quantize to d = 0 and contribute exactly 0; all-zero input gives y == 0."""
    import torch
    N, K = 64, 256
    rng = np.random.default_rng(5)
    wb = gguf.quantize_q4_0(rng.standard_normal((N, K), dtype=np.float32))
    W = QM.Q4Mat(wb, N, K, "cuda")
    x = rng.standard_normal((2, K), dtype=np.float32)
    x[0] = 0
    x[1, 64:128] = 0
    xq, xds, q, d = q8(x)
    assert d[0].max() == 0 and d[1, 2:4].max() == 0
    y = torch.zeros(2, N, device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), 2, ptr(y), None, 0)
    torch.cuda.synchronize()
    yy = y.cpu().numpy()
    assert np.all(yy[0] == 0)
    assert relerr(yy[1], OQ.gemv_q4_0_q8_1(wb, N, K, q, d)[1]) < 1e-3


@pytest.mark.parametrize("fp32", [0, 1])
@pytest.mark.parametrize("nh,nkv", [(8, 2), (16, 2), (12, 3)])
def test_attn_decode_gqa_groups(cuda, nh, nkv, fp32):
    """GQA groups of 4 and 8 query heads per KV head (the model's is 6): each group size has its own
    instantiation of the f64 kernel, one query head per workgroup. Positions cover one page, a page plus one
    key and three full pages."""
    import torch
    mc = 4
    rng = np.random.default_rng(nh * 10 + nkv + fp32)
    pos = np.array([0, 64, 255], np.int32)
    T = len(pos)
    kc = rng.standard_normal((T * mc, nkv, 64, 128)).astype(np.float16)
    vc = rng.standard_normal((T * mc, nkv, 64, 128)).astype(np.float16)
    bt = rng.permutation(T * mc).astype(np.int32).reshape(T, mc)
    q = (rng.standard_normal((T, nh * 128)) * 2).astype(np.float16)
    part = torch.zeros(T, nh, mc, 130, dtype=torch.float64, device=cuda)
    oq = torch.zeros(T, nh * 128, dtype=torch.int8, device=cuda)
    ods = torch.zeros(T, nh * 4, 2, dtype=torch.float16, device=cuda)
    o32 = torch.zeros(T, nh * 128, device=cuda)
    call("q355_attn_decode", ptr(dev(q)), ptr(dev(kc)), ptr(dev(vc)), ptr(dev(pos)), ptr(dev(bt)), mc, nh, nkv, mc,
         1 / math.sqrt(128), ptr(part), ptr(oq), ptr(ods), ptr(o32), T, fp32)
    torch.cuda.synchronize()
    for j in range(T):
        K = np.concatenate([kc[bt[j, p]] for p in range(mc)], axis=1)
        V = np.concatenate([vc[bt[j, p]] for p in range(mc)], axis=1)
        ref = OM.attn_decode(q[j].reshape(nh, 128), K, V, int(pos[j]) + 1, nh, nkv)
        # f64 scores/softmax/P.V rounded once to fp32 (fp32 = 0); fp16 P on the matrix cores (fp32 = 1)
        assert relerr(o32[j].cpu().numpy(), ref) < (1e-6 if fp32 == 0 else 1e-3), (nh, nkv, j)


@pytest.mark.parametrize("fp32", [0, 1])
def test_attn_decode_longest_context(cuda, fp32):
    """max_chunks = 64 pages: the last position of a 4096-token cache, and position 0 beside it."""
    import torch
    nh, nkv, mc = 12, 2, 64
    rng = np.random.default_rng(64 + fp32)
    kc = rng.standard_normal((2 * mc, nkv, 64, 128)).astype(np.float16)
    vc = rng.standard_normal((2 * mc, nkv, 64, 128)).astype(np.float16)
    bt = rng.permutation(2 * mc).astype(np.int32).reshape(2, mc)
    q = rng.standard_normal((2, nh * 128)).astype(np.float16)
    pos = np.array([64 * mc - 1, 0], np.int32)
    part = torch.zeros(2, nh, mc, 130, dtype=torch.float64, device=cuda)
    oq = torch.zeros(2, nh * 128, dtype=torch.int8, device=cuda)
    ods = torch.zeros(2, nh * 4, 2, dtype=torch.float16, device=cuda)
    o32 = torch.zeros(2, nh * 128, device=cuda)
    call("q355_attn_decode", ptr(dev(q)), ptr(dev(kc)), ptr(dev(vc)), ptr(dev(pos)), ptr(dev(bt)), mc, nh, nkv, mc,
         1 / math.sqrt(128), ptr(part), ptr(oq), ptr(ods), ptr(o32), 2, fp32)
    torch.cuda.synchronize()
    for j in range(2):
        K = np.concatenate([kc[bt[j, p]] for p in range(mc)], axis=1)
        V = np.concatenate([vc[bt[j, p]] for p in range(mc)], axis=1)
        ref = OM.attn_decode(q[j].reshape(nh, 128), K, V, int(pos[j]) + 1, nh, nkv)
        assert relerr(o32[j].cpu().numpy(), ref) < 1e-3


def test_attn_decode_fp32_splits(cuda):
    """The fp32 path's two-level merge (4 pages inside a workgroup, then the splits): contexts of 1 to 9
    splits, one scratch buffer reused by calls with different T, fp16 and Q8_1 outputs."""
    import torch
    nh, nkv, mc = 12, 2, 36
    rng = np.random.default_rng(7)
    Tmax = 6
    kc = rng.standard_normal((Tmax * mc, nkv, 64, 128)).astype(np.float16)
    vc = rng.standard_normal((Tmax * mc, nkv, 64, 128)).astype(np.float16)
    bt = rng.permutation(Tmax * mc).astype(np.int32).reshape(Tmax, mc)
    q = rng.standard_normal((Tmax, nh * 128)).astype(np.float16)
    part = torch.full((Tmax, nh, mc, 130), float('nan'), dtype=torch.float64, device=cuda)
    kcd, vcd, btd, qd = dev(kc), dev(vc), dev(bt), dev(q)
    for T, positions in [(6, [64 * mc - 1, 0, 255, 256, 1000, 2047]), (2, [300, 1500]), (5, [70, 2200, 9, 511, 512])]:
        pos = np.array(positions, np.int32)
        oq = torch.zeros(T, nh * 128, dtype=torch.int8, device=cuda)
        ods = torch.zeros(T, nh * 4, 2, dtype=torch.float16, device=cuda)
        o32 = torch.zeros(T, nh * 128, device=cuda)
        oh = torch.zeros(T, nh * 128, dtype=torch.float16, device=cuda)
        posd = dev(pos)
        call("q355_attn_decode", ptr(qd), ptr(kcd), ptr(vcd), ptr(posd), ptr(btd), mc, nh, nkv, mc,
             1 / math.sqrt(128), ptr(part), ptr(oq), ptr(ods), ptr(o32), T, 1)
        call("q355_attn_decode_f16", ptr(qd), ptr(kcd), ptr(vcd), ptr(posd), ptr(btd), mc, nh, nkv, mc,
             1 / math.sqrt(128), ptr(part), ptr(oh), T)
        torch.cuda.synchronize()
        for j in range(T):
            K = np.concatenate([kc[bt[j, p]] for p in range(mc)], axis=1)
            V = np.concatenate([vc[bt[j, p]] for p in range(mc)], axis=1)
            ref = OM.attn_decode(q[j].reshape(nh, 128), K, V, int(pos[j]) + 1, nh, nkv)
            assert relerr(o32[j].cpu().numpy(), ref) < 1e-3, (T, j)
            assert relerr(oh[j].float().cpu().numpy(), ref) < 2e-3, (T, j)
        rq, rd, _ = OQ.quantize_q8_1(o32.cpu().numpy())
        assert np.array_equal(oq.cpu().numpy(), rq)
        assert np.array_equal(ods.cpu().numpy()[..., 0], rd.astype(np.float16))


@pytest.mark.parametrize("T", [1, 64])
def test_mmq_decode_batch_extremes(cuda, T):
    """The int8 MFMA product at one token and at 64 tokens (four 16-token workgroups)."""
    import torch
    N, K = 1536, 8960
    rng = np.random.default_rng(T)
    wb = gguf.quantize_q4_0(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    W = QM.Q4Mat(wb, N, K, "cuda")
    xq, xds, q, d = q8(rng.standard_normal((T, K), dtype=np.float32))
    y = torch.zeros(T, N, device=cuda)
    call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, 0, ptr(y), None, None, None, None, None)
    torch.cuda.synchronize()
    assert relerr(y.cpu().numpy(), OQ.gemv_q4_0_q8_1(wb, N, K, q, d)) < 1e-3


CFG_S = QM.Config(L=2, V=4096)


@pytest.fixture(scope="module")
def small(cuda):
    w = QM.random_weights(CFG_S, seed=21)
    return w, QM.DeviceModel(w, CFG_S, maxlen=512)


def test_prefill_single_token_equals_decode_step(small):
    """A one-token prefill chunk (the MMQ path) and one decode step (the f64 GEMV path) agree on the hidden
    state and the next token."""
    w, dm = small
    a = QM.Decoder(dm, T=1, max_ctx=128)
    QB.Prefill(a, max_chunk=16).chunk([77], 0)
    b = QM.Decoder(dm, T=1, max_ctx=128)
    b.tok.fill_(77)
    b.step()
    assert int(a.pos.item()) == int(b.pos.item()) == 1
    lg_a, lg_b = a.logits[0].cpu().numpy(), b.logits[0].cpu().numpy()
    assert relerr(lg_a, lg_b) < 2e-2
    top2 = np.partition(lg_b, -2)[-2:]
    if top2[1] - top2[0] > 1e-2:
        assert int(a.tok.item()) == int(b.tok.item())


def test_decode_at_last_cache_position(small):
    """Decoding the last position a cache holds (pos = 64 max_chunks - 1) works and matches the oracle."""
    import torch
    w, dm = small
    om = OM.Model(OM.Config(L=2, V=4096), w, maxlen=512)
    dec = QM.Decoder(dm, T=1, max_ctx=128)
    prompt = list(np.random.default_rng(8).integers(0, CFG_S.V, 127))
    QB.Prefill(dec, max_chunk=128).chunk(prompt[:-1], 0)
    dec.tok.fill_(int(prompt[-1]))
    assert int(dec.pos.item()) == 126
    dec.step()                                  # position 126
    dec.tok.fill_(5)
    dec.step()                                  # position 127 = the last slot
    torch.cuda.synchronize()
    assert int(dec.pos.item()) == 128
    cache = om.new_cache()
    om.forward(prompt, 0, cache)
    h = om.forward([5], 127, cache)
    assert relerr(dec.logits[0].cpu().numpy(), om.logits(h)[0]) < 5e-2


@pytest.mark.parametrize("N,K,T,epi", [(8960, 1536, 1, 0), (1536, 8960, 2, 1), (2048, 1536, 4, 2)])
def test_gemv_bf16_reference_parity_mode(cuda, N, K, T, epi):
    """Q4_0 x bf16 activations in fp32 (the reference's decode arithmetic) against the f64 dequantized product."""
    import torch
    rng = np.random.default_rng(N + K + T)
    wb = gguf.quantize_q4_0(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    W = QM.Q4Mat(wb, N, K, "cuda")
    xb = OQ.f32_to_bf16(rng.standard_normal((T, K), dtype=np.float32))
    bias = rng.standard_normal(N, dtype=np.float32)
    y0 = rng.standard_normal((T, N), dtype=np.float32) if epi == 1 else np.zeros((T, N), np.float32)
    y = dev(y0.copy())
    call("q355_gemv_q4_0_bf16", ptr(W.qs), ptr(W.d), N, K, ptr(dev(xb.view(np.int16))), T, ptr(y),
         ptr(dev(bias)), epi)
    torch.cuda.synchronize()
    ref = OQ.gemv_q4_0_bf16(wb, N, K, xb)
    if epi == 1:
        ref = ref + y0
    elif epi == 2:
        ref = ref + bias
    assert relerr(y.cpu().numpy(), ref) < 1e-5
