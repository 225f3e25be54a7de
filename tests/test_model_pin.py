"""Pins the composition of oracle.model.Model with an independently written float64 forward in torch.

The forward below follows the reference's decode step order (scripts/qwen_fused.py:113-145):
embed -> per layer [RMSNorm(ln1) -> QKV GEMV + bias -> RoPE(q, k) + K/V write -> GQA attention ->
O GEMV + residual -> RMSNorm(ln2) -> gate/up GEMV -> SwiGLU -> down GEMV + residual] -> RMSNorm(norm) ->
tied head. It shares no code with oracle/: the Q4_0 decoder, the Q8_1 rounding points (the reference's
QUANT_Q8 rule, lab/qwen_batched.py:1032-1033, with the fp16 stored scale), RMSNorm, the NeoX RoPE pairing
(d, d + 64), softmax attention and SiLU are written here in torch from their definitions. Both activation
modes are pinned: "q8" (Q8_1 layer inputs) and "f16" (the reference's batched arithmetic, gemv_v2_source,
lab/qwen_batched.py:467-680: fp16 layer inputs times the fp16 weights d (q - 8), the LM head on Q8_1). A model with a
swapped norm weight, a dropped bias or a misplaced residual gives logits that differ far beyond the
tolerance (checked by the mutation cases at the end).
"""
import math

import numpy as np
import pytest
import torch

from lab import qwen_model as QM
from oracle import model as OM

H, NH, NKV, HD, FFN, V = 1536, 12, 2, 128, 8960, 1024


def dq4(b: np.ndarray, n: int, k: int) -> torch.Tensor:
    """GGUF Q4_0 bytes -> float64 [n, k]: per 18-byte block, fp16 scale then 16 bytes whose low nibbles are
    weights 0..15 and high nibbles weights 16..31, value = d (q - 8)."""
    t = torch.from_numpy(np.asarray(b, np.uint8).reshape(-1, 18).copy())
    d = t[:, :2].contiguous().view(torch.float16).to(torch.float64)
    qs = t[:, 2:].to(torch.int64)
    q = torch.cat([qs & 15, qs >> 4], 1).to(torch.float64) - 8
    return (d * q).reshape(n, k)


def q8(x: torch.Tensor) -> torch.Tensor:
    """Q8_1 round trip of fp32 activations: d = fp32(amax / 127), q = round-half-even(fp32(x / d)), value q * fp16(d)."""
    xb = x.to(torch.float32).reshape(x.shape[0], -1, 32)
    d = xb.abs().amax(-1, keepdim=True) / 127.0
    q = torch.where(d > 0, torch.round(xb / torch.where(d > 0, d, torch.ones_like(d))), torch.zeros_like(xb))
    return (q.to(torch.float64) * d.to(torch.float16).to(torch.float64)).reshape(x.shape)


def f16(x: torch.Tensor) -> torch.Tensor:
    """fp16 layer input: the fp32 activation rounded to fp16."""
    return x.to(torch.float32).to(torch.float16).to(torch.float64)


def w16(wq: torch.Tensor) -> torch.Tensor:
    """The fp16 weight of the batched arithmetic: d (q - 8), an exact float64 product, rounded once to fp16."""
    return wq.to(torch.float16).to(torch.float64)


def rms(h, w, eps=1e-6):
    return h / torch.sqrt((h * h).mean(-1, keepdim=True) + eps) * torch.as_tensor(w, dtype=torch.float64)


class Ref:
    def __init__(self, w, maxlen=64, mutate=None, act="q8"):
        self.w, self.mut = w, mutate or ""
        self.a = q8 if act == "q8" else f16
        i = torch.arange(0, HD, 2, dtype=torch.float64) / HD
        ang = torch.arange(maxlen, dtype=torch.float64)[:, None] * (1e6 ** -i)[None]
        self.cos, self.sin = torch.cos(ang).to(torch.float32).double(), torch.sin(ang).to(torch.float32).double()
        self.E = dq4(w["embed"], V, H)
        self.L = []
        for L in w["layers"]:
            self.L.append({k: (dq4(L[k], *s) if act == "q8" else w16(dq4(L[k], *s))) for k, s in
                           (("wq", (NH * HD, H)), ("wk", (NKV * HD, H)), ("wv", (NKV * HD, H)), ("wo", (H, NH * HD)),
                            ("wg", (FFN, H)), ("wu", (FFN, H)), ("wd", (H, FFN)))})
        self.K = [torch.zeros(NKV, maxlen, HD, dtype=torch.float64) for _ in w["layers"]]
        self.V = [torch.zeros(NKV, maxlen, HD, dtype=torch.float64) for _ in w["layers"]]

    def rot(self, x, p):
        # pairs (d, d + 64) rotated by the angle of frequency d: (a, b) -> (a c - b s, a s + b c)
        a, b = x[..., :64], x[..., 64:]
        c, s = self.cos[p], self.sin[p]
        return torch.cat([a * c - b * s, a * s + b * c], -1)

    def step(self, tok, p):
        h = self.E[tok][None].to(torch.float32).double()
        for i, (Lw, Ld) in enumerate(zip(self.w["layers"], self.L)):
            ln1, ln2 = (Lw["ln2"], Lw["ln1"]) if self.mut == "swap_norms" else (Lw["ln1"], Lw["ln2"])
            x = self.a(rms(h, ln1).to(torch.float32))
            bq = 0 if self.mut == "no_bias" else torch.as_tensor(Lw["bq"], dtype=torch.float64)
            q = x @ Ld["wq"].T + bq
            k = x @ Ld["wk"].T + torch.as_tensor(Lw["bk"], dtype=torch.float64)
            v = x @ Ld["wv"].T + torch.as_tensor(Lw["bv"], dtype=torch.float64)
            q = self.rot(q.reshape(NH, HD), p).to(torch.float16).double()
            self.K[i][:, p] = self.rot(k.reshape(NKV, HD), p).to(torch.float16).double()
            self.V[i][:, p] = v.reshape(NKV, HD).to(torch.float16).double()
            att = torch.empty(NH, HD, dtype=torch.float64)
            for hh in range(NH):
                kv = hh // (NH // NKV)
                s = self.K[i][kv, :p + 1] @ q[hh] / math.sqrt(HD)
                att[hh] = torch.softmax(s, 0) @ self.V[i][kv, :p + 1]
            o = self.a(att.reshape(1, -1).to(torch.float32)) @ Ld["wo"].T
            h = o if self.mut == "no_resid" else h + o
            x = self.a(rms(h, ln2).to(torch.float32))
            m = torch.nn.functional.silu(x @ Ld["wg"].T) * (x @ Ld["wu"].T)
            h = h + self.a(m.to(torch.float32)) @ Ld["wd"].T
        x = q8(rms(h, self.w["norm"]).to(torch.float32))
        return (x @ self.E.T).to(torch.float32)[0]


@pytest.fixture(scope="module")
def weights():
    return QM.random_weights(QM.Config(L=2, V=V), seed=31)


def _oracle_logits(w, toks, act="q8"):
    m = OM.Model(OM.Config(L=2, V=V), w, maxlen=64, act=act)
    cache = m.new_cache()
    out = []
    for p, t in enumerate(toks):
        out.append(m.logits(m.forward([t], p, cache))[0])
    return np.stack(out)


def _ref_logits(w, toks, mutate=None, act="q8"):
    r = Ref(w, mutate=mutate, act=act)
    return np.stack([r.step(t, p).numpy() for p, t in enumerate(toks)])


TOKS = [5, 900, 17, 333, 1023, 64]


@pytest.mark.parametrize("act", ["q8", "f16"])
def test_model_matches_independent_forward(weights, act):
    """2 layers at full width, 6 decode positions: the oracle's logits equal the independent forward's."""
    a, b = _oracle_logits(weights, TOKS, act), _ref_logits(weights, TOKS, act=act)
    err = np.abs(a - b).max() / np.abs(b).max()
    assert err < 1e-6, err


@pytest.mark.parametrize("mutate", ["swap_norms", "no_bias", "no_resid"])
def test_forward_detects_composition_mistakes(weights, mutate):
    """The comparison above is sensitive: each plausible composition mistake moves the logits by > 1e-3."""
    a, b = _oracle_logits(weights, TOKS[:3]), _ref_logits(weights, TOKS[:3], mutate)
    assert np.abs(a - b).max() / np.abs(a).max() > 1e-3


def test_forward_detects_activation_mode_mistake(weights):
    """The two modes' rounding points are distinguishable: the "f16" oracle against the "q8" forward (Q8_1
    inputs instead of fp16, unrounded weights) differs by > 1e-3."""
    a, b = _oracle_logits(weights, TOKS[:3], "f16"), _ref_logits(weights, TOKS[:3], act="q8")
    assert np.abs(a - b).max() / np.abs(a).max() > 1e-3
