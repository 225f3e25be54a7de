"""GPU parity of the prefill path: causal flash attention on fp16 MFMA and the chunked
prefill driver (MMQ GEMMs + attention), against the numpy oracle."""
import math

import numpy as np
import pytest

from lab import qwen_batched as QB
from lab import qwen_model as QM
from lab.hip import call, ptr
from oracle import model as OM

pytestmark = pytest.mark.gpu
ATT_TOL = 3e-3          # fp16 P (as BASELINE config 4: fp16 inputs, fp32 accumulation) vs the f64 oracle
NEAR_TIE = 1e-2


def relerr(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("P,pos0,nh,nkv", [(1, 0, 12, 2), (64, 0, 12, 2), (100, 0, 12, 2), (200, 37, 12, 2),
                                           (130, 64, 8, 2), (17, 250, 12, 2), (700, 0, 12, 2), (300, 555, 16, 2),
                                           (77, 1500, 12, 2), (64, 4100, 12, 2), (130, 2000, 8, 2),
                                           (2048, 0, 12, 2), (1024, 3000, 12, 2), (100, 1500, 16, 2)])
def test_attn_prefill_matches_oracle(cuda, P, pos0, nh, nkv, split):
    """Without and with the workspace. With it, contexts past 1024 keys run the persistent form over key splits
    of 1024 keys: pos0 = 4100 merges 5 splits; pos0 = 2000 makes a query block straddle a split boundary, so
    some of its queries see no key of the last split; P = 2048 and (1024, 3000) give 384 and 512 items, two
    rounds per workgroup; (100, 1500, 16, 2) runs the 640-thread form (8 query heads per KV head). Two calls in
    a row reuse the self-resetting counters and give the same bits."""
    import torch
    rng = np.random.default_rng(P * 1000 + pos0)
    n = pos0 + P
    n_pages = (n + 63) // 64 + 3
    K = rng.standard_normal((nkv, n_pages * 64, 128)).astype(np.float16)
    V = rng.standard_normal((nkv, n_pages * 64, 128)).astype(np.float16)
    q = (rng.standard_normal((P, nh, 128)) * 0.5).astype(np.float16)
    # scattered pages: logical page c of the sequence lives in physical page table[c]
    table = rng.permutation(n_pages).astype(np.int32)
    kc = np.zeros((n_pages, nkv, 64, 128), np.float16)
    vc = np.zeros_like(kc)
    for c in range(n_pages):
        kc[table[c]] = K[:, 64 * c:64 * (c + 1)]
        vc[table[c]] = V[:, 64 * c:64 * (c + 1)]
    # positions past the context hold garbage that the mask must ignore
    kc_t = torch.from_numpy(kc).cuda()
    vc_t = torch.from_numpy(vc).cuda()
    out = torch.zeros(P, nh * 128, device=cuda)
    q_t = torch.from_numpy(q.reshape(P, -1)).cuda()
    table_t = torch.from_numpy(table).cuda()
    ws, nb = None, 0
    if split:
        nb = call("q355_attn_prefill_ws_bytes", P, n, nh, nkv)
        ws = torch.zeros(nb // 4, dtype=torch.float32, device=cuda)
    ref = OM.attn_prefill(q, K, V, pos0, nh, nkv)
    first = None
    for rep in range(2 if split else 1):                  # the second call reuses the self-resetting counters
        out.zero_()
        call("q355_attn_prefill", ptr(q_t), ptr(kc_t), ptr(vc_t), ptr(table_t), pos0, P, nh, nkv,
             1.0 / math.sqrt(128), ptr(out), ptr(ws) if split else None, nb)
        torch.cuda.synchronize()
        assert relerr(out.cpu().numpy(), ref) < ATT_TOL
        if first is None:
            first = out.clone()
        else:                                             # merged in split order whatever the arrival order
            assert torch.equal(out.view(torch.int32), first.view(torch.int32))
    if split:
        cnt = ws[-((P + 15) // 16) * nkv * (nh // nkv):].view(torch.int32)   # [query blocks][KV heads][heads]
        assert int(cnt.abs().sum()) == 0
    # the Q8_1-output form quantizes exactly the values the fp32 form stores
    oq = torch.zeros(P, nh * 128, dtype=torch.int8, device=cuda)
    ods = torch.zeros(P, nh * 4, 2, dtype=torch.float16, device=cuda)
    call("q355_attn_prefill_q8_1", ptr(q_t), ptr(kc_t), ptr(vc_t), ptr(table_t), pos0, P, nh, nkv,
         1.0 / math.sqrt(128), ptr(oq), ptr(ods), ptr(ws) if split else None, nb)
    xq = torch.zeros_like(oq)
    xds = torch.zeros_like(ods)
    call("q355_quant_q8_1", ptr(out), ptr(xq), ptr(xds), P, nh * 128)
    torch.cuda.synchronize()
    assert torch.equal(oq, xq) and torch.equal(ods, xds)


def test_attn_prefill_bad_args(cuda):
    from lab.hip import HipError
    with pytest.raises(HipError, match="attn_prefill"):
        call("q355_attn_prefill", 1, 1, 1, 1, 0, 0, 12, 2, 0.1, 1, None, 0)
    with pytest.raises(HipError, match="workspace"):
        call("q355_attn_prefill", 1, 1, 1, 1, 0, 2048, 12, 2, 0.1, 1, 1, 100)
    with pytest.raises(HipError, match="null output"):
        call("q355_attn_prefill_q8_1", 1, 1, 1, 1, 0, 16, 12, 2, 0.1, None, 1, None, 0)
    with pytest.raises(HipError, match="mmq_qkv_rope"):        # N must be (nh + 2 nkv) * 128
        call("q355_mmq_qkv_rope", 16, 16, 1024, 1536, 16, 16, 64, 16, 16, 16, 16, 16, 4, 0, 16, 16, 16, None, 12, 2)
    with pytest.raises(HipError, match="mmq_qkv_rope"):        # seq_stride is 0 or 1
        call("q355_mmq_qkv_rope", 16, 16, 2048, 1536, 16, 16, 64, 16, 16, 16, 16, 16, 4, 2, 16, 16, 16, None, 12, 2)


CFG_S = QM.Config(L=2, V=4096)


@pytest.fixture(scope="module")
def small(cuda):
    w = QM.random_weights(CFG_S, seed=21)
    return w, QM.DeviceModel(w, CFG_S, maxlen=512), OM.Model(OM.Config(L=2, V=4096), w, maxlen=512)


def test_prefill_matches_oracle(small):
    """A 150-token prompt in one chunk: final hidden states, the K cache and the next token match the oracle."""
    import torch
    w, dm, om = small
    prompt = np.random.default_rng(5).integers(0, CFG_S.V, 150)
    dec = QM.Decoder(dm, T=1, max_ctx=512)
    pf = QB.Prefill(dec, max_chunk=256)
    pf.chunk(prompt, 0)
    torch.cuda.synchronize()
    cache = om.new_cache()
    h = om.forward(list(prompt), 0, cache)
    assert relerr(pf.hidden_f64(150).cpu().numpy(), h) < 2e-2
    k_gpu = dec.kc[1][0:3].permute(1, 0, 2, 3).reshape(2, 192, 128)[:, :150].float().cpu().numpy()
    assert relerr(k_gpu, cache["K"][1][:, :150]) < 2e-2
    lg = om.logits(h[-1:])[0]
    top2 = np.partition(lg, -2)[-2:]
    if top2[1] - top2[0] >= NEAR_TIE:
        assert int(dec.tok.item()) == int(np.argmax(lg))
    assert int(dec.pos.item()) == 150


def test_prefill_then_decode_greedy(small):
    """Prefill, then greedy decode continues from the prefilled cache: tokens match the oracle up to its first
    near-tie."""
    w, dm, om = small
    prompt = list(np.random.default_rng(6).integers(0, CFG_S.V, 70))
    dec = QM.Decoder(dm, T=1, max_ctx=256)
    QB.Prefill(dec, max_chunk=128).chunk(prompt, 0)
    got = dec.generate(12)[0]
    ref, margins = om.greedy(prompt, 12)
    for i, (x, y) in enumerate(zip(got, ref)):
        if margins[i] < NEAR_TIE:
            break
        assert x == y, f"token {i}: {x} vs {y} (margin {margins[i]:.3g})"


def test_prefill_chunked_equals_one_chunk(small):
    """Two chunks (64 + 61 tokens, the second at pos0 = 64) leave the same cache and next token as one chunk."""
    import torch
    w, dm, om = small
    prompt = np.random.default_rng(7).integers(0, CFG_S.V, 125)
    a = QM.Decoder(dm, T=1, max_ctx=256)
    QB.Prefill(a, max_chunk=128).chunk(prompt, 0)
    b = QM.Decoder(dm, T=1, max_ctx=256)
    pb = QB.Prefill(b, max_chunk=128)
    pb.chunk(prompt[:64], 0)
    pb.chunk(prompt[64:], 64)
    torch.cuda.synchronize()
    for i in range(CFG_S.L):
        assert relerr(b.kc[i][:2].float().cpu().numpy(), a.kc[i][:2].float().cpu().numpy()) < 1e-2
    assert int(a.pos.item()) == int(b.pos.item()) == 125
    lg = om.logits(om.forward(list(prompt), 0, om.new_cache())[-1:])[0]
    top2 = np.partition(lg, -2)[-2:]
    if top2[1] - top2[0] >= NEAR_TIE:
        assert int(a.tok.item()) == int(b.tok.item())


@pytest.mark.parametrize("T,seq_stride", [(1100, 0), (8, 1), (32, 1), (5, 1), (20, 1)])
def test_mmq_qkv_rope_equals_finish(cuda, T, seq_stride):
    """The QKV product with the finish in its epilogue (tiled kernel for a prefill chunk, register-resident for
    decode batches of one token per sequence) writes the same q and K/V cache rows as the K-split product into
    the int64 accumulator followed by q355_qkv_finish (both round once from f64)."""
    import torch
    c = QM.Config(L=1, V=1024)
    N, K = c.nqkv, c.H
    rng = np.random.default_rng(11 + T)
    from lab import gguf
    W = QM.Q4Mat(gguf.quantize_q4_0(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)), N, K, "cuda")
    x = torch.from_numpy(rng.standard_normal((T, K), dtype=np.float32)).cuda()
    xq = torch.zeros(T, K, dtype=torch.int8, device=cuda)
    xds = torch.zeros(T, K // 32, 2, dtype=torch.float16, device=cuda)
    call("q355_quant_q8_1", ptr(x), ptr(xq), ptr(xds), T, K)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda()
    maxlen = 1216
    ang = np.arange(maxlen)[:, None] * (1e6 ** (-np.arange(64) * 2 / 128))[None, :]
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).cuda()
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).cuda()
    if seq_stride == 0:                                       # one sequence, positions 37 .. 37 + T - 1
        pos_np = np.arange(37, 37 + T, dtype=np.int32)
        bt_stride = n_pages = maxlen // 64
        table_np = rng.permutation(n_pages).astype(np.int32)
    else:                                                     # one token per sequence, scattered pages
        bt_stride = 8
        n_pages = T * bt_stride
        pos_np = rng.integers(0, bt_stride * 64, T).astype(np.int32)
        table_np = rng.permutation(n_pages).astype(np.int32).reshape(T, bt_stride)
    pos = torch.from_numpy(pos_np).cuda()
    table = torch.from_numpy(table_np).cuda()
    outs = []
    for fused in (True, False):
        kc = torch.zeros(n_pages, c.NKV, 64, 128, dtype=torch.float16, device=cuda)
        vc = torch.zeros_like(kc)
        q = torch.zeros(T, c.NH * 128, dtype=torch.float16, device=cuda)
        if fused:
            call("q355_mmq_qkv_rope", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(bias), ptr(cos), ptr(sin),
                 ptr(pos), ptr(table), bt_stride, seq_stride, ptr(kc), ptr(vc), ptr(q), None, c.NH, c.NKV)
        else:
            acc = torch.zeros(T, N, dtype=torch.int64, device=cuda)
            call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), N, K, ptr(xq), ptr(xds), T, 6, None, ptr(acc),
                 None, None, None, None)
            call("q355_qkv_finish", ptr(acc), ptr(bias), ptr(cos), ptr(sin), ptr(pos), ptr(table), bt_stride,
                 seq_stride, ptr(kc), ptr(vc), ptr(q), c.NH, c.NKV, T)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (q, kc, vc)])
    for a, b in zip(*outs):
        ulp = np.abs(a.view(np.int16).astype(np.int32) - b.view(np.int16).astype(np.int32))
        assert ulp.max() <= 1 and (ulp > 0).mean() < 1e-3
    # exactly the cache rows of the T (sequence, position) pairs were written
    rows = np.abs(outs[0][1]).sum(axis=(1, 3)) > 0                 # [page, slot]
    want = np.zeros_like(rows)
    for j, p in enumerate(pos_np):
        pg = table_np[p // 64] if seq_stride == 0 else table_np[j, p // 64]
        want[pg, p % 64] = True
    assert np.array_equal(rows, want)


def test_prefill_fused_qkv_equals_split(small, monkeypatch):
    """A chunk long enough for the fused QKV epilogue leaves the same cache, hidden state and next token as the
    accumulator + finish path (forced by raising the threshold)."""
    import torch
    w, dm, om = small
    dm2 = QM.DeviceModel(w, CFG_S, maxlen=1216)
    prompt = np.random.default_rng(8).integers(0, CFG_S.V, 1100)
    res = []
    for thr in (QB.QKV_FUSED_MIN_P, 1 << 30):
        monkeypatch.setattr(QB, "QKV_FUSED_MIN_P", thr)
        dec = QM.Decoder(dm2, T=1, max_ctx=1216)
        pf = QB.Prefill(dec, max_chunk=1100)
        pf.chunk(prompt, 0)
        torch.cuda.synchronize()
        res.append((pf.hidden_f64(1100).cpu().numpy(), [dec.kc[i].float().cpu().numpy() for i in range(CFG_S.L)],
                    int(dec.tok.item())))
        del pf, dec
    assert relerr(res[0][0], res[1][0]) < 1e-3
    for a, b in zip(res[0][1], res[1][1]):
        assert relerr(a, b) < 1e-3
    assert res[0][2] == res[1][2]
