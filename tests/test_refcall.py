"""Reference-order launches (lab/refcall.py): a decode step written the way the reference's host code writes it.

RefStep below mirrors FusedQwen.gemv / rms / step (scripts/qwen_fused.py:104-145) line for line: the same kernel
names (gemv_source(epi), RMSNORM_F32W_1P, EMBED_F32, ATTN4 % {...}, FINISH_MB), the same launch argument lists
(W, S, X, Y, AUX, N, K etc.) built from tensor.data_ptr() and ctypes scalars. The CPU test checks which library
calls those launches become (the call layer is replaced by a recorder); the GPU test runs the step and requires
bit-equal residual streams and equal tokens against lab.qwen_model.Decoder.step.
"""
import ctypes
import math

import numpy as np
import pytest

from lab import qwen_batched as QB
from lab import qwen_kernels as KS
from lab import qwen_model as QM
from lab import refcall
from lab.hip import Kern

SPLIT = {"qkv": 2, "o": 2, "gu": 4, "down": 8, "head": 4}


class RefStep:
    """FusedQwen's step over this build's buffers (device-resident model `dm`, decode state of `dec`)."""

    def __init__(self, dm, dec):
        c = dm.cfg
        self.H, self.nh, self.nkv, self.hd, self.inter, self.V, self.eps = c.H, c.NH, c.NKV, c.HD, c.FFN, c.V, c.eps
        self.L = [{"ln1": L["ln1"], "ln2": L["ln2"], "qkv_b": L["qkv_b"], "qkv": (L["qkv"].qs, L["qkv"].d),
                   "o": (L["o"].qs, L["o"].d), "gu": (L["gu"].qs, L["gu"].d), "down": (L["down"].qs, L["down"].d)}
                  for L in dm.layers]
        self.embed, self.norm, self.head = dm.embed, dm.norm, (dm.embed.qs, dm.embed.d)
        self.cos, self.sin = dm.cos, dm.sin
        self.kc, self.vc = dec.kc, dec.vc
        dev = dec.h.device
        self.h, self.tok, self.pos = dec.h, dec.tok, dec.pos
        self.x = refcall.NormedAct(1, self.H, dev)
        self.xm = dec.mlp
        self.qkv = refcall.QKVOut(1, self.nh, self.hd, dec.block_table, dev)
        self.att = refcall.AttnOut(1, self.nh, self.hd, dec.max_chunks, dev)
        self.logits = refcall.Logits(1, self.V, dev)
        self.k = {name: Kern(KS.gemv_source(SPLIT[name], epi)) for name, epi in
                  (("qkv", "bias"), ("o", "resid"), ("gu", "swiglu"), ("down", "resid"), ("head", "logits"))}
        self.k_rms, self.k_emb = Kern(KS.RMSNORM_F32W_1P), Kern(KS.EMBED_F32)
        self.k_attn, self.k_fin = Kern(KS.ATTN4 % {"maxlen": 2048}), Kern(KS.FINISH_MB)

    def gemv(self, name, wsplit, X, Y, aux, N, K):
        W, S = wsplit
        self.k[name].launch((N + 3) // 4, 32 * SPLIT[name],
                            [W.data_ptr(), S.data_ptr(), X.data_ptr(), Y.data_ptr(), aux, ctypes.c_int32(N),
                             ctypes.c_int32(K)])

    def rms(self, w, out):
        self.k_rms.launch(1, 512, [self.h.data_ptr(), w.data_ptr(), out.data_ptr(), ctypes.c_int32(self.H),
                                   ctypes.c_float(self.eps)])

    def step(self):
        H, nq = self.H, (self.nh + 2 * self.nkv) * self.hd
        self.k_emb.launch(4, 512, [self.embed.data_ptr(), self.tok.data_ptr(), self.h.data_ptr(), ctypes.c_int32(H)])
        scale = ctypes.c_float(1.0 / math.sqrt(self.hd))
        for i, L in enumerate(self.L):
            self.rms(L["ln1"], self.x)
            self.gemv("qkv", L["qkv"], self.x, self.qkv, L["qkv_b"].data_ptr(), nq, H)
            aargs = [self.qkv.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(), self.pos.data_ptr(),
                     self.kc[i].data_ptr(), self.vc[i].data_ptr(), self.att.data_ptr(), ctypes.c_int32(self.nh),
                     ctypes.c_int32(self.nkv), scale]
            self.k_attn.launch(self.nh, 128, aargs)
            self.gemv("o", L["o"], self.att, self.h, 0, H, self.nh * self.hd)
            self.rms(L["ln2"], self.x)
            self.gemv("gu", L["gu"], self.x, self.xm, 0, 2 * self.inter, H)
            self.gemv("down", L["down"], self.xm, self.h, 0, H, self.inter)
        self.rms(self.norm, self.x)
        self.gemv("head", self.head, self.x, self.logits, 0, self.V, H)
        nb = 8
        self.k_fin.launch(nb, 256, [self.logits.data_ptr(), ctypes.c_int32(self.V), self.tok.data_ptr(),
                                    self.pos.data_ptr(), 0, 0, 0])


class RefBatched:
    """Batched.step (scripts/qwen_batched_decode.py:106-187) over this build's buffers: batchify'd EMBED_F32 /
    RMSNORM_F32W_1P / ATTN4 launched over grid.y = B, gemv_v2_source GEMVs with (W, S, X, Y, aux, N, K, ws, cnt),
    head_v2_source on pack_q6_mma's head with (*head, x, logits, V, H), then the argmax and pos += 1 in torch,
    as the reference does them. The decode state (h, tok, pos, paged caches) is BatchedDecoder `bd`'s."""

    CONFIG2 = {8: {"qkv": (1, 4, 1, 4), "o": (1, 8, 1, 2), "gu": (4, 2, 2, 1), "down": (1, 4, 1, 4)},
               32: {"qkv": (2, 4, 1, 2), "o": (2, 4, 1, 1), "gu": (2, 4, 1, 1), "down": (2, 2, 1, 4)}}

    def __init__(self, dm, bd):
        c, B = dm.cfg, bd.B
        self.B, self.H, self.nh, self.nkv, self.hd, self.inter, self.V, self.eps = B, c.H, c.NH, c.NKV, c.HD, c.FFN, c.V, c.eps
        self.nq = (self.nh + 2 * self.nkv) * self.hd
        self.L = [{"ln1": L["ln1"], "ln2": L["ln2"], "qkv_b": L["qkv_b"], "qkv": (L["qkv"].qs, L["qkv"].d),
                   "o": (L["o"].qs, L["o"].d), "gu": (L["gu"].qs, L["gu"].d), "down": (L["down"].qs, L["down"].d)}
                  for L in dm.layers]
        self.embed, self.norm, self.cos, self.sin = dm.embed, dm.norm, dm.cos, dm.sin
        self.head_packed = QB.pack_q6_mma(dm.head_q6k if dm.head_q6k is not None else dm.embed)
        self.h, self.tok, self.pos, self.kc, self.vc = bd.h, bd.tok, bd.pos, bd.kc, bd.vc
        dev = bd.h.device
        self.x = refcall.BatchAct(B, self.H, dev)
        self.qkv = refcall.BatchQKV(B, self.nh, self.hd, bd.block_table, dev)
        self.att = refcall.BatchAttn(B, self.nh, self.nkv, self.hd, bd.max_chunks, dev)
        self.xm = bd.mh
        self.logits = refcall.Logits(B, self.V, dev, batched=True)
        cfg = self.CONFIG2[8 if B <= 8 else 32]
        self.cfg = cfg
        self.g = {name: Kern(QB.gemv_v2_source(cfg[name][0], cfg[name][1], cfg[name][2], B, epi, 1, cfg[name][3]))
                  for name, epi in (("qkv", "biasf"), ("o", "resid"), ("gu", "swiglu"), ("down", "resid"))}
        self.ws, self.cnt = 0, 0
        self.k_emb = Kern(QB.batchify(KS.EMBED_F32, "tok += b_; h += (size_t)b_ * H;"))
        self.k_rms = Kern(QB.batchify(KS.RMSNORM_F32W_1P, "h += (size_t)b_ * H; out += (size_t)b_ * H;"))
        self.k_attn = Kern(QB.batchify(KS.ATTN4 % {"maxlen": 4096}, "qkv += ...;"))
        self.k_head = Kern(QB.head_v2_source(8, 1, 1, B))

    def gemv(self, name, X, Y, aux, N, K):
        W, S = self.L[self.layer][name]
        WM, WK, MT, KS_ = self.cfg[name]
        R = 16 * MT * WM
        self.g[name].launch(((N + R - 1) // R, KS_), 32 * WM * WK,
                            [W.data_ptr(), S.data_ptr(), X.data_ptr(), Y.data_ptr(), aux, ctypes.c_int32(N),
                             ctypes.c_int32(K), self.ws, self.cnt])

    def rms(self, w):
        self.k_rms.launch((1, self.B), 512, [self.h.data_ptr(), w.data_ptr(), self.x.data_ptr(),
                                             ctypes.c_int32(self.H), ctypes.c_float(self.eps)])

    def step(self):
        B, H = self.B, self.H
        self.k_emb.launch((4, B), 512, [self.embed.data_ptr(), self.tok.data_ptr(), self.h.data_ptr(), ctypes.c_int32(H)])
        scale = ctypes.c_float(1.0 / math.sqrt(self.hd))
        for i, L in enumerate(self.L):
            self.layer = i
            self.rms(L["ln1"])
            self.gemv("qkv", self.x, self.qkv, L["qkv_b"].data_ptr(), self.nq, H)
            self.k_attn.launch((self.nh, B), 512, [self.qkv.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                                                   self.pos.data_ptr(), self.kc[i].data_ptr(), self.vc[i].data_ptr(),
                                                   self.att.data_ptr(), ctypes.c_int32(self.nh),
                                                   ctypes.c_int32(self.nkv), scale])
            self.gemv("o", self.att, self.h, 0, H, self.nh * self.hd)
            self.rms(L["ln2"])
            self.gemv("gu", self.x, self.xm, 0, 2 * self.inter, H)
            self.gemv("down", self.xm, self.h, 0, H, self.inter)
        self.rms(self.norm)
        self.k_head.launch(self.V // 128, 256, [*(t.data_ptr() for t in self.head_packed), self.x.data_ptr(),
                                                 self.logits.data_ptr(), ctypes.c_int32(self.V), ctypes.c_int32(H)])
        self.tok.copy_(self.logits.logits.argmax(-1))
        self.pos += 1


CFG = QM.Config(L=2, V=4096)


def _model(device):
    w = QM.random_weights(CFG, seed=23)
    return QM.DeviceModel(w, CFG, maxlen=128, device=device)


def test_reference_order_launches_map_to_fused_calls(monkeypatch):
    """CPU: the reference-shaped step issues exactly the fused entry points Decoder.step issues, in order, with the
    epilogue the generator chose."""
    import torch
    calls = []
    monkeypatch.setattr(refcall, "call", lambda name, *a: calls.append((name, a)) or (8 if name.endswith("nparts") else 0))
    monkeypatch.setattr(QM, "call", lambda name, *a: 8 if name.endswith("nparts") else 0)
    dm = _model("cpu")
    dec = QM.Decoder(dm, T=1, max_ctx=128)
    RefStep(dm, dec).step()
    names = [n for n, _ in calls]
    layer = ["q355_qkv_rope_kv", "q355_attn_decode", "q355_attn_o_resid", "q355_ffn_gate_up", "q355_ffn_down"]
    assert names == ["q355_head_nparts", "q355_embed_q4_0"] + layer * CFG.L + ["q355_head_logits", "q355_finish"]
    qkv = calls[2][1]
    L0 = dm.layers[0]
    # q355_qkv_rope_kv(qs, d, K, h, ln1, eps, bias, cos, sin, pos, block_table, bt_stride, 1, kc, vc, q, nh, nkv, T)
    assert qkv[0] == L0["qkv"].qs.data_ptr() and qkv[2] == CFG.H and qkv[3] == dec.h.data_ptr()
    assert qkv[4] == L0["ln1"].data_ptr() and qkv[6] == L0["qkv_b"].data_ptr() and qkv[16:19] == (CFG.NH, CFG.NKV, 1)
    down = calls[6][1]
    assert down[:4] == (L0["down"].qs.data_ptr(), L0["down"].d.data_ptr(), CFG.H, CFG.FFN)
    assert down[4] == dec.mlp.data_ptr() and down[5] == dec.h.data_ptr()


def test_reference_order_errors():
    """Wrong shapes and missing producers are reported, not launched."""
    spec = KS.gemv_source(2, "resid")
    assert spec.params["epi_name"] == "resid" and spec.ref == "gemv"
    assert KS.ATTN4 % {"maxlen": 4096} is KS.ATTN4
    with pytest.raises(ValueError):
        KS.gemv_source(2, "bogus")


def test_reference_order_down_is_batch_one(monkeypatch):
    """The down product over plain pointers (no row count) runs one token; a spec asking for more is rejected."""
    import dataclasses
    from lab.hip import HipError
    calls = []
    monkeypatch.setattr(refcall, "call", lambda name, *a: calls.append((name, a)) or 0)
    dm = _model("cpu")
    W = dm.layers[0]["down"]
    refcall.register(W.qs, W)
    spec = KS.gemv_source(2, "resid")
    refcall.launch_gemv(spec, [W.qs, W.d, 1000, 2000, 0, CFG.H, CFG.FFN])
    assert calls and calls[-1][0] == "q355_ffn_down" and calls[-1][1][-1] == 1
    wide = dataclasses.replace(spec, params={**spec.params, "T": 4})
    with pytest.raises(HipError, match="batch 1"):
        refcall.launch_gemv(wide, [W.qs, W.d, 1000, 2000, 0, CFG.H, CFG.FFN])


@pytest.mark.gpu
def test_reference_order_step_equals_decoder(cuda):
    """GPU: prompt + greedy steps through RefStep and through Decoder.step give bit-equal h and equal tokens."""
    import torch
    dm = _model("cuda")
    a = QM.Decoder(dm, T=1, max_ctx=128)
    b = QM.Decoder(dm, T=1, max_ctx=128)
    ref = RefStep(dm, b)
    prompt = [7, 4000, 123, 9, 3071]
    for t in prompt + [None] * 6:
        if t is not None:
            a.tok.fill_(t)
            b.tok.fill_(t)
        a.step()
        ref.step()
        torch.cuda.synchronize()
        assert torch.equal(a.h, b.h)
        assert int(a.tok.item()) == int(b.tok.item()) and int(a.pos.item()) == int(b.pos.item())


def test_reference_order_typed_arguments():
    """The reference allocates tok/pos as torch.long; the kernels read int32, so a tensor of another dtype is
    rejected; the GGUF script's quant name "g32f16" (GGUF Q4_0) is accepted."""
    import torch
    from lab.hip import HipError
    with pytest.raises(HipError, match="int32"):
        refcall.launch_embed(KS.EMBED_F32, [0, torch.zeros(1, dtype=torch.long), 0, 1536])
    with pytest.raises(HipError, match="int32"):
        refcall.launch_finish(KS.FINISH, [0, 4096, torch.zeros(1, dtype=torch.int32), torch.zeros(1, dtype=torch.long)])
    assert KS.gemv_source(2, "resid", "g32f16") == KS.gemv_source(2, "resid")
    with pytest.raises(ValueError):
        KS.gemv_source(2, "resid", "g128f32")


def test_batched_reference_order_launches_map_to_fused_calls(monkeypatch):
    """CPU: Batched.step's launches issue the entry points BatchedDecoder(act="f16").step issues, in order."""
    calls = []
    fake = lambda name, *a: calls.append((name, a)) or (8 if name.endswith("nparts") else 0)
    monkeypatch.setattr(refcall, "call", fake)
    monkeypatch.setattr(QM, "call", fake)
    monkeypatch.setattr(QB, "call", fake)
    dm = _model("cpu")
    for B in (8, 32):
        bd = QB.BatchedDecoder(dm, B=B, max_ctx=128, act="f16", keep_logits=True)
        calls.clear()
        bd.step()
        want = [n for n, _ in calls if not n.endswith("nparts")]
        ref = RefBatched(dm, bd)
        calls.clear()
        ref.step()
        got = [n for n, _ in calls if not n.endswith("nparts")]
        want = [n for n in want if n != "q355_finish"]   # the reference takes the argmax in torch
        assert got == want, (B, got[:8], want[:8])


@pytest.mark.gpu
@pytest.mark.parametrize("B", [8, 32])
def test_batched_reference_order_step_equals_decoder(cuda, B):
    """GPU: prompts + greedy steps through RefBatched and through BatchedDecoder(act="f16").step give bit-equal
    residual streams and logits and equal tokens (B = 8: split merge inside the O product; B = 32: its own
    launch)."""
    import torch
    dm = _model("cuda")
    a = QB.BatchedDecoder(dm, B=B, max_ctx=128, page_seed=B, act="f16", keep_logits=True)
    b = QB.BatchedDecoder(dm, B=B, max_ctx=128, page_seed=B, act="f16")
    ref = RefBatched(dm, b)
    prompts = np.random.default_rng(B).integers(0, CFG.V, (B, 4)).astype(np.int32)
    for t in range(10):
        if t < prompts.shape[1]:
            a.tok.copy_(torch.from_numpy(prompts[:, t]))
            b.tok.copy_(torch.from_numpy(prompts[:, t]))
        a.step()
        ref.step()
        torch.cuda.synchronize()
        assert torch.equal(a.h, b.h), t
        assert torch.equal(a.logits, ref.logits.logits), t
        assert torch.equal(a.tok, b.tok) and torch.equal(a.pos, b.pos), t
