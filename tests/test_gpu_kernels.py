"""GPU parity of each libqwen355 kernel against the numpy oracle (same seeded inputs).

Bars: integer outputs (per-block int32 dots, Q8_1 of identical fp32 inputs) bit-exact; fp32 outputs
within 1e-3 relative (max |gpu - oracle| / max |oracle|, the reference's norm-error metric of
lab/experiments/gemv5.py:66-69); fp16 outputs within one fp16 ulp-scale tolerance stated per test.
"""
import math

import numpy as np
import pytest

from lab import gguf, hip
from lab import qwen_model as QM
from lab.hip import call, ptr
from oracle import model as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

REL = 1e-3


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


_KEEP = []


@pytest.fixture(autouse=True)
def _keep_alive():
    """Device copies made with to_dev() stay alive until the test ends (a pointer taken from a temporary
    tensor would otherwise be recycled by the caching allocator before the kernel reads it)."""
    yield
    _KEEP.clear()


def to_dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    t = t.cuda() if dtype is None else t.to(dtype).cuda()
    _KEEP.append(t)
    return t


def sync():
    import torch
    torch.cuda.synchronize()


def q8_dev(x):
    """Upload the oracle's Q8_1 quantization of x [T, K] (xq, xds as half2 pairs)."""
    q, d, s = OQ.quantize_q8_1(x)
    ds = np.stack([d, s], -1)
    return to_dev(q), to_dev(ds.view(np.int16)), (q, d, s)


def mat_dev(N, K, seed):
    w = np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    b = gguf.quantize_q4_0(w)
    return QM.Q4Mat(b, N, K, "cuda"), b


# --------------------------------------------------------------------------------------------------

def test_quant_q8_1_bitexact(cuda):
    import torch
    rng = np.random.default_rng(1)
    T, K = 3, 1536
    x = rng.standard_normal((T, K), dtype=np.float32)
    x[0, :32] = 0.0                                   # d = 0 block
    x[1, 32:64] = np.float32(0.5) * np.arange(32)     # exact halves after scaling
    x[2, 64:96] = -x[2, 64:96] * 1e-30                # tiny values (fp16 d underflow)
    x[2, 96:128] = x[2, 96:128] * 1e-4                # small values (fp16-subnormal d)
    xq = torch.zeros(T, K, dtype=torch.int8, device=cuda)
    xds = torch.zeros(T, K // 32, 2, dtype=torch.float16, device=cuda)
    call("q355_quant_q8_1", ptr(to_dev(x)), ptr(xq), ptr(xds), T, K)
    sync()
    q, d, s = OQ.quantize_q8_1(x)
    assert np.array_equal(xq.cpu().numpy(), q)
    g = xds.cpu().numpy()
    assert np.array_equal(g[..., 0].view(np.uint16), d.view(np.uint16))
    assert np.array_equal(g[..., 1].view(np.uint16), s.view(np.uint16))


def test_rmsnorm_q8_1(cuda):
    import torch
    rng = np.random.default_rng(2)
    T, H = 4, 1536
    h = rng.standard_normal((T, H), dtype=np.float32) * 3
    w = (1 + 0.01 * rng.standard_normal(H)).astype(np.float32)
    xq = torch.zeros(T, H, dtype=torch.int8, device=cuda)
    xds = torch.zeros(T, H // 32, 2, dtype=torch.float16, device=cuda)
    call("q355_rmsnorm_q8_1", ptr(to_dev(h)), ptr(to_dev(w)), ptr(xq), ptr(xds), T, H, 1e-6)
    sync()
    q, d, _ = OQ.quantize_q8_1(OM.rmsnorm(h, w, 1e-6).astype(np.float32))
    gq = xq.cpu().numpy().astype(np.int32)
    # fp32 RMSNorm vs float64: a rounding tie can flip by one step, rarely
    assert np.abs(gq - q).max() <= 1
    assert (gq != q).mean() < 1e-3
    assert relerr(xds.cpu().numpy()[..., 0], d) < 1e-3


def test_blockdots_bitexact(cuda):
    import torch
    rng = np.random.default_rng(3)
    N, K, T = 64, 256, 2
    qw = rng.integers(0, 16, (N, K), dtype=np.uint8)
    qw[0] = 15
    qx = rng.integers(-127, 128, (T, K), dtype=np.int8)
    qx[0, :32] = 127
    qx[1, :32] = -127
    # GGUF bytes from nibbles (d arbitrary)
    blk = qw.reshape(N * K // 32, 32)
    b = np.zeros((N * K // 32, 18), np.uint8)
    b[:, 2:] = blk[:, :16] | (blk[:, 16:] << 4)
    qs, _ = gguf.tile_q4_0(b, N, K)
    out = torch.zeros(T, N, K // 32, dtype=torch.int32, device=cuda)
    call("q355_gemv_blockdots", ptr(to_dev(qs.reshape(-1))), N, K, ptr(to_dev(qx)), T, ptr(out))
    sync()
    assert np.array_equal(out.cpu().numpy(), OQ.block_dots(qw, qx))


@pytest.mark.parametrize("N,K,T", [(8960, 1536, 1), (1536, 8960, 1), (2048, 1536, 4), (1536, 1536, 3)])
def test_gemv_store(cuda, N, K, T):
    """BASELINE config 0 (8960 x 1536, batch 1) and the other layer shapes."""
    import torch
    W, b = mat_dev(N, K, seed=N + K)
    x = np.random.default_rng(7).standard_normal((T, K), dtype=np.float32)
    xq, xds, (q, d, _) = q8_dev(x)
    y = torch.zeros(T, N, dtype=torch.float32, device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(y), None, 0)
    sync()
    ref = OQ.gemv_q4_0_q8_1(b, N, K, q, d)
    assert relerr(y.cpu().numpy(), ref) < REL


def test_gemv_resid_bias(cuda):
    import torch
    N, K, T = 1536, 8960, 2
    W, b = mat_dev(N, K, seed=11)
    x = np.random.default_rng(8).standard_normal((T, K), dtype=np.float32)
    xq, xds, (q, d, _) = q8_dev(x)
    h0 = np.random.default_rng(9).standard_normal((T, N), dtype=np.float32)
    h = to_dev(h0)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(h), None, 1)
    bias = np.random.default_rng(10).standard_normal(N).astype(np.float32)
    yb = torch.zeros(T, N, dtype=torch.float32, device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(yb), ptr(to_dev(bias)), 2)
    sync()
    ref = OQ.gemv_q4_0_q8_1(b, N, K, q, d)
    assert relerr(h.cpu().numpy() - h0, ref) < REL
    assert relerr(yb.cpu().numpy(), ref + bias) < REL


def test_gemv_bad_shape_raises(cuda):
    import torch
    y = torch.zeros(16, device=cuda)
    with pytest.raises(hip.HipError, match="N=24"):
        call("q355_gemv_q4_0_q8_1", ptr(y), ptr(y), 24, 32, ptr(y), ptr(y), 1, ptr(y), None, 0)
    with pytest.raises(hip.HipError, match="T=5"):
        call("q355_gemv_q4_0_q8_1", ptr(y), ptr(y), 16, 32, ptr(y), ptr(y), 5, ptr(y), None, 0)


# --------------------------------------------------------------------------------------------------
# fused layer ops against the oracle layer

CFG1 = QM.Config(L=1, V=1024)


@pytest.fixture(scope="module")
def one_layer(cuda):
    w = QM.random_weights(CFG1, seed=5)
    dm = QM.DeviceModel(w, CFG1, maxlen=1024)
    om = OM.Model(OM.Config(L=1, V=1024), w, maxlen=1024)
    return w, dm, om


def test_qkv_rope_kv(one_layer):
    import torch
    w, dm, om = one_layer
    c = CFG1
    T = 2
    dec = QM.Decoder(dm, T=T, max_ctx=1024)
    h = np.random.default_rng(12).standard_normal((T, c.H), dtype=np.float32)
    dec.set_h(h)
    pos = np.array([77, 513], np.int32)
    dec.pos.copy_(to_dev(pos))
    L = dm.layers[0]
    call("q355_qkv_rope_kv", ptr(L["qkv"].qs), ptr(L["qkv"].d), c.H, ptr(dec.h), ptr(L["ln1"]), c.eps,
         ptr(L["qkv_b"]), ptr(dm.cos), ptr(dm.sin), ptr(dec.pos), ptr(dec.block_table), dec.max_chunks, 1,
         ptr(dec.kc[0]), ptr(dec.vc[0]), ptr(dec.q), c.NH, c.NKV, T)
    sync()
    WL, lin = w["layers"][0], om.lin[0]
    for j in range(T):
        x = OM.rmsnorm(h[j:j + 1], WL["ln1"], c.eps).astype(np.float32)
        q = lin["q"](x)[0] + WL["bq"]
        k = lin["k"](x)[0] + WL["bk"]
        v = lin["v"](x)[0] + WL["bv"]
        p = int(pos[j])
        qr = OM.rope(q.reshape(c.NH, c.HD), om.cos[p], om.sin[p]).reshape(-1)
        kr = OM.rope(k.reshape(c.NKV, c.HD), om.cos[p], om.sin[p])
        assert relerr(dec.q[j].float().cpu().numpy(), qr) < REL
        page = dec.block_table[j, p // 64].item()
        kg = dec.kc[0][page, :, p % 64].float().cpu().numpy()
        vg = dec.vc[0][page, :, p % 64].float().cpu().numpy()
        assert relerr(kg, kr) < REL
        assert relerr(vg, v.reshape(c.NKV, c.HD)) < REL


def test_ffn_gate_up_down(one_layer):
    import torch
    w, dm, om = one_layer
    c = CFG1
    T = 3
    dec = QM.Decoder(dm, T=T, max_ctx=128)
    h = np.random.default_rng(13).standard_normal((T, c.H), dtype=np.float32)
    dec.set_h(h)
    L = dm.layers[0]
    call("q355_ffn_gate_up", ptr(L["gu"].qs), ptr(L["gu"].d), L["gu"].N, c.H, ptr(dec.h), ptr(L["ln2"]), c.eps,
         ptr(dec.mlp), T)
    sync()
    WL, lin = w["layers"][0], om.lin[0]
    x = OM.rmsnorm(h, WL["ln2"], c.eps).astype(np.float32)
    m = OM.silu_mul(lin["g"](x), lin["u"](x)).astype(np.float32)
    gm = dec.mlp.cpu().numpy()
    assert relerr(gm, m) < REL
    # down: Q8_1(m) per K slice + GEMV + fixed-point residual add (4 K slices)
    call("q355_ffn_down", ptr(L["down"].qs), ptr(L["down"].d), c.H, c.FFN, ptr(dec.mlp), ptr(dec.h), T)
    sync()
    ref = lin["d"](gm)
    assert relerr(dec.h_f32().cpu().numpy() - h, ref) < REL


@pytest.mark.parametrize("fp32", [0, 1])
@pytest.mark.parametrize("positions,max_chunks", [([0, 63], 16), ([64, 511], 16), ([1000, 5], 16),
                                                  # chunk counts that are not a multiple of 8: the batch-1
                                                  # grid pads its chunk slots to 8, the padding must exit
                                                  ([319, 200, 0], 5), ([831, 64], 13)])
def test_attn_decode(cuda, positions, max_chunks, fp32):
    import torch
    c = CFG1
    T = len(positions)
    rng = np.random.default_rng(sum(positions))
    n_pages = T * max_chunks
    kc = rng.standard_normal((n_pages, c.NKV, 64, c.HD)).astype(np.float16)
    vc = rng.standard_normal((n_pages, c.NKV, 64, c.HD)).astype(np.float16)
    bt = rng.permutation(n_pages).astype(np.int32).reshape(T, max_chunks)   # scattered pages
    q = (rng.standard_normal((T, c.NH * c.HD)) * 2).astype(np.float16)
    pos = np.array(positions, np.int32)
    part = torch.zeros(T, c.NH, max_chunks, c.HD + 2, dtype=torch.float64, device=cuda)
    oq = torch.zeros(T, c.NH * c.HD, dtype=torch.int8, device=cuda)
    ods = torch.zeros(T, c.NH * c.HD // 32, 2, dtype=torch.float16, device=cuda)
    o32 = torch.zeros(T, c.NH * c.HD, device=cuda)
    for rep in range(2):   # repeated calls give identical results (no state carried between calls)
        call("q355_attn_decode", ptr(to_dev(q)), ptr(to_dev(kc)), ptr(to_dev(vc)), ptr(to_dev(pos)), ptr(to_dev(bt)),
             max_chunks, c.NH, c.NKV, max_chunks, 1 / math.sqrt(c.HD), ptr(part), ptr(oq), ptr(ods), ptr(o32), T, fp32)
        sync()
        for j in range(T):
            K = np.concatenate([kc[bt[j, p]] for p in range(max_chunks)], axis=1)     # [nkv, ctx, hd]
            V = np.concatenate([vc[bt[j, p]] for p in range(max_chunks)], axis=1)
            ref = OM.attn_decode(q[j].reshape(c.NH, c.HD), K, V, int(pos[j]) + 1, c.NH, c.NKV)
            assert relerr(o32[j].cpu().numpy(), ref) < REL
            rq, rd, _ = OQ.quantize_q8_1(o32[j:j + 1].cpu().numpy())
            assert np.array_equal(oq[j:j + 1].cpu().numpy(), rq)
    if fp32:
        return                       # the fp32 path merges in its own launch; part is then its workspace
    # fused merge + Q8_1 + O projection + residual (the decode path) against the merged output
    W, b = mat_dev(c.H, c.NH * c.HD, seed=31)
    h0 = rng.standard_normal((T, c.H), dtype=np.float32)
    h = to_dev(np.round(h0.astype(np.float64) * QM.FIX_SCALE).astype(np.int64))
    call("q355_attn_o_resid", ptr(W.qs), ptr(W.d), c.H, ptr(part), max_chunks, ptr(to_dev(pos)), c.NH, ptr(h), T)
    sync()
    rq, rd, _ = OQ.quantize_q8_1(o32.cpu().numpy())
    ref = OQ.gemv_q4_0_q8_1(b, c.H, c.NH * c.HD, rq, rd)
    assert relerr(h.cpu().numpy() / QM.FIX_SCALE - h0, ref) < REL


def test_finish_ties(cuda):
    import torch
    pm = np.array([[1.0, 3.0, 3.0, -1.0], [2.0, 2.0, 2.0, 2.0]], np.float32)
    pi = np.array([[5, 9, 7, 1], [40, 30, 20, 10]], np.int32)
    tok = torch.zeros(2, dtype=torch.int32, device=cuda)
    pos = torch.tensor([3, 4], dtype=torch.int32, device=cuda)
    call("q355_finish", ptr(to_dev(pm)), ptr(to_dev(pi)), 4, ptr(tok), ptr(pos), 2)
    sync()
    assert tok.tolist() == [7, 10]
    assert pos.tolist() == [4, 5]


def test_embed_head(one_layer):
    import torch
    w, dm, om = one_layer
    c = CFG1
    T = 2
    dec = QM.Decoder(dm, T=T, max_ctx=128)
    toks = np.array([3, 1000], np.int32)
    dec.tok.copy_(to_dev(toks))
    dec.embed()
    sync()
    assert np.array_equal(dec.h_f32().cpu().numpy(), om.embed(toks))
    h = np.random.default_rng(14).standard_normal((T, c.H), dtype=np.float32)
    dec.set_h(h)
    dec.head()
    sync()
    ref = om.logits(h)
    assert relerr(dec.logits.cpu().numpy(), ref) < REL
    assert dec.tok.cpu().numpy().tolist() == [int(np.argmax(r)) for r in dec.logits.cpu().numpy()]


def test_qkv_with_embedding_equals_embed_then_qkv(one_layer):
    """q355_qkv_rope_kv_embed (layer 0's QKV with the embedding in its prologue) gives bit-equal h, q and K/V
    cache rows to q355_embed_q4_0 followed by q355_qkv_rope_kv, at T = 1 and 3."""
    import torch
    w, dm, om = one_layer
    for T in (1, 3):
        a = QM.Decoder(dm, T=T, max_ctx=128)
        b = QM.Decoder(dm, T=T, max_ctx=128)
        toks = np.array([3, 1000, 1023][:T], np.int32)
        for d in (a, b):
            d.tok.copy_(to_dev(toks))
            d.pos.copy_(to_dev(np.array([5, 70, 127][:T], np.int32)))
            d.h.fill_(12345)                      # stale residual: both paths must overwrite it
        a.embed()
        a.layer(0)
        b.layer(0, embed=True)
        sync()
        assert torch.equal(a.q, b.q)
        assert torch.equal(a.kc[0], b.kc[0]) and torch.equal(a.vc[0], b.vc[0])
        assert torch.equal(a.h, b.h)


# --------------------------------------------------------------------------------------------------
# one decoder layer, decode at batch 1 with 512 past positions of N(0,1) fp16 KV

def test_layer_config1(one_layer):
    import torch
    w, dm, om = one_layer
    c = CFG1
    dec = QM.Decoder(dm, T=1, max_ctx=1024)
    rng = np.random.default_rng(15)
    past = 512
    Kp = rng.standard_normal((c.NKV, past, c.HD)).astype(np.float16)
    Vp = rng.standard_normal((c.NKV, past, c.HD)).astype(np.float16)
    for p0 in range(0, past, 64):
        pg = dec.block_table[0, p0 // 64].item()
        dec.kc[0][pg] = to_dev(Kp[:, p0:p0 + 64])
        dec.vc[0][pg] = to_dev(Vp[:, p0:p0 + 64])
    h = rng.standard_normal((1, c.H), dtype=np.float32)
    dec.set_h(h)
    dec.pos.fill_(past)
    dec.layer(0)
    sync()
    cache = om.new_cache()
    cache["K"][0, :, :past] = Kp
    cache["V"][0, :, :past] = Vp
    ref = om.layer(0, h, past, cache)
    got = dec.h_f64().cpu().numpy()
    # north_star's bound is 1e-3 relative; the f64 layer (fixed-point residual) holds the layer's update to 1e-9
    assert relerr(got - h, ref - h) < 1e-9
    assert relerr(got, ref) < 1e-9


# --------------------------------------------------------------------------------------------------
# small whole-model greedy decode and graph replay

CFG_S = QM.Config(L=2, V=4096)


@pytest.fixture(scope="module")
def small_model(cuda):
    w = QM.random_weights(CFG_S, seed=21)
    return w, QM.DeviceModel(w, CFG_S, maxlen=512), OM.Model(OM.Config(L=2, V=4096), w, maxlen=512)


def test_greedy_small_model(small_model):
    w, dm, om = small_model
    prompt = list(np.random.default_rng(22).integers(0, CFG_S.V, 8))
    ref, margins = om.greedy(prompt, 24)
    dec = QM.Decoder(dm, T=1, max_ctx=512)
    dec.prefill_tokens(prompt)
    got = dec.generate(24)[0].tolist()
    first_bad = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), None)
    assert first_bad is None, f"diverged at {first_bad} (oracle top-2 margin {margins[first_bad]:.3g})"


def test_graph_replay_matches_eager(small_model):
    import torch
    w, dm, om = small_model
    prompt = [5, 6, 7]
    a = QM.Decoder(dm, T=2, max_ctx=256)
    a.prefill_tokens(np.array([prompt, prompt[::-1]]))
    b = QM.Decoder(dm, T=2, max_ctx=256)
    b.prefill_tokens(np.array([prompt, prompt[::-1]]))
    ga = a.generate(12, use_graph=True)
    gb = b.generate(12, use_graph=False)
    assert np.array_equal(ga, gb)
    assert torch.equal(a.h, b.h)            # bitwise: fixed reduction order, no atomics on this path
