"""Oracle: the Qwen2.5-1.5B-shape Q4_0 model (numpy). TEST INFRASTRUCTURE ONLY.

Restates the reference's decode step (scripts/qwen_fused.py:113-145, kernels in lab/qwen_kernels.py)
with this build's operand formats (Q8_1 activations, fp16 KV cache, tied Q4_0 embedding/head):

  h = E[tok]                                   EMBED_F32 (lab/qwen_kernels.py:284-290), Q4_0 row dequant
  per layer:
    x = Q8_1(rmsnorm(h) * ln1)                 RMSNORM_F32W_1P (lab/qwen_kernels.py:683-705),
                                               rmsnorm_q8 (lab/qwen_batched.py:1044-1091)
    qkv = Wqkv x + b                           gemv 'biasf' epilogue (lab/qwen_kernels.py:33)
    q, k = RoPE(q, k) (pairs d, d+64)          ATTN4 (lab/qwen_kernels.py:532-546), tables
                                               scripts/qwen_gguf.py:108-113 (theta = 1e6)
    K[pos], V[pos] = fp16(k), fp16(v); q = fp16(q)
    att = softmax(q K^T / sqrt(128)) V per head, GQA group NH/NKV    (ATTN4 :547-603)
    h += Wo Q8_1(att)                          'resid' epilogue (:34)
    x = Q8_1(rmsnorm(h) * ln2)
    m = silu(g) * u, (g, u) = (Wg x, Wu x)     'swiglu' epilogue (:21-28), swiglu_q8 (qwen_batched.py:1363-1396)
    h += Wd Q8_1(m)
  logits = E Q8_1(rmsnorm(h) * norm); tok = argmax (lowest index wins ties); pos += 1
                                               FINISH / FINISH_MB (lab/qwen_kernels.py:222-282)

Rounding points follow the product: every GEMV input is Q8_1 of an fp32 value (x, att, m) -- with
act "f16" (the batched decode path) the layer GEMV inputs are instead rounded to fp16 and the weights are
the fp16 values d (q - 8) (gemv_v2_source, lab/qwen_batched.py:467-680); the LM head keeps Q8_1 -- q/K/V are
rounded f64 -> fp16 once (round to nearest even), logits are fp32; everything else (GEMV outputs, the residual stream h,
RMSNorm, RoPE, attention, SwiGLU) is float64.
GEMVs use gemv_q4_0_q8_1 semantics; mode "f64" computes them as a float64 BLAS product of the
exactly dequantized operands (identical mathematics, pinned against the int32 block-dot form on
small shapes), which makes full-model runs practical on the CPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import quant as Q


@dataclass
class Config:
    H: int = 1536
    NH: int = 12
    NKV: int = 2
    HD: int = 128
    FFN: int = 8960
    L: int = 28
    V: int = 151936
    eps: float = 1e-6
    theta: float = 1e6


def rope_tables(maxlen: int, hd: int = 128, theta: float = 1e6):
    """cos/sin fp32 [maxlen, hd/2]: inv_i = theta^(-2i/hd) and angles in float64, then rounded to fp32
    (scripts/qwen_gguf.py:108-113).
    pinned by: closed form at pos 0 (cos 1, sin 0) and pos 1 (cos/sin of inv_i computed by math.cos)."""
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.arange(maxlen, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rmsnorm(h: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """h [T, H] -> h * 1/sqrt(mean(h^2) + eps) * w in float64 (RMSNORM_F32W_1P, lab/qwen_kernels.py:683-705).
    pinned by: closed form on a constant vector (h = c -> c/sqrt(c^2 + eps) w) and scale invariance."""
    h = np.asarray(h, np.float64)
    r = 1.0 / np.sqrt((h * h).mean(axis=-1, keepdims=True) + eps)
    return h * r * np.asarray(w, np.float64)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., hd] at one position (cos/sin [hd/2] rows): NeoX half-split rotation, pairs (i, i + hd/2):
    out_i = a c - b s, out_{i+hd/2} = b c + a s (lab/qwen_kernels.py:163-169; scripts/qwen_e2e.py:139-143).
    pinned by: equality with complex multiplication (a + ib) e^{i angle} and norm preservation."""
    half = x.shape[-1] // 2
    a, b = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    c, s = cos.astype(np.float64), sin.astype(np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(g) * u = g / (1 + exp(-g)) * u (lab/qwen_kernels.py:27).
    pinned by: closed values (silu(0) = 0, silu(large) -> g) and scipy.special.expit."""
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def argmax_lowest(logits: np.ndarray) -> int:
    """Index of the maximum, lowest index on ties (FINISH_MB tie rule, lab/qwen_kernels.py:230, 277).
    pinned by: hand cases with ties."""
    return int(np.argmax(logits))       # numpy returns the first occurrence


def attn_decode(q: np.ndarray, K: np.ndarray, V: np.ndarray, n_ctx: int, nh: int, nkv: int) -> np.ndarray:
    """One decode token. q [nh, hd] (fp16 values), K/V [nkv, >=n_ctx, hd] fp16; attends to positions
    0..n_ctx-1 (the new token's K/V already written at n_ctx-1). Returns fp32 [nh*hd].
    Semantics of ATTN4 (lab/qwen_kernels.py:517-605): s = q.k / sqrt(hd), softmax with max subtraction,
    o = sum p v / sum p.
    pinned by: uniform keys -> mean of V; a single dominant key -> its V row; equality with prefill
    causal attention at the last row (attn_prefill, an independently written masked form)."""
    hd = q.shape[-1]
    grp = nh // nkv
    out = np.empty((nh, hd), np.float64)
    for g in range(nkv):                                 # K/V widened once per KV head
        k = K[g, :n_ctx].astype(np.float64)
        v = V[g, :n_ctx].astype(np.float64)
        for h in range(g * grp, (g + 1) * grp):
            s = k @ q[h].astype(np.float64) / math.sqrt(hd)
            p = np.exp(s - s.max())
            out[h] = p @ v / p.sum()
    return out.reshape(-1).astype(np.float32)


def attn_prefill(q: np.ndarray, K: np.ndarray, V: np.ndarray, pos0: int, nh: int, nkv: int) -> np.ndarray:
    """Causal GQA attention for P tokens at positions pos0..pos0+P-1 (flash_prefill_v3 semantics,
    lab/qwen_batched.py:1795-2037, and the torch reference of scripts/flash_bench.py:51-65).
    q [P, nh, hd] fp16 values; K/V [nkv, >= pos0+P, hd]. Row t attends to keys 0..pos0+t. -> fp32 [P, nh*hd]."""
    P, _, hd = q.shape
    grp = nh // nkv
    n = pos0 + P
    mask = np.arange(n)[None, :] > (pos0 + np.arange(P))[:, None]           # [P, n] True = masked
    out = np.empty((P, nh, hd), np.float64)
    for h in range(nh):
        k = K[h // grp, :n].astype(np.float64)
        v = V[h // grp, :n].astype(np.float64)
        s = q[:, h].astype(np.float64) @ k.T / math.sqrt(hd)
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p @ v) / p.sum(axis=1, keepdims=True)
    return out.reshape(P, nh * hd).astype(np.float32)


class LinearQ6K:
    """A Q6_K matrix (llama.cpp's output.weight) applied to Q8_1 activations, float64."""

    def __init__(self, wbytes: np.ndarray, N: int, K: int):
        self.b, self.N, self.K = wbytes, N, K
        self._w = None

    def __call__(self, x: np.ndarray) -> np.ndarray:
        if self._w is None:
            self._w = Q.dequant_q6_k(self.b, (self.N, self.K))
        qx, dx, _ = Q.quantize_q8_1(np.asarray(x, np.float32))
        return Q.dequant_q8_1(qx, dx).astype(np.float64) @ self._w.T


class Linear:
    """One Q4_0 matrix W [N, K] from GGUF bytes, applied to Q8_1 activations (act "q8"), or, as the batched
    decode does (gemv_v2_source, lab/qwen_batched.py:467-680), as fp16-dequantized weights to fp16
    activations (act "f16")."""

    def __init__(self, wbytes: np.ndarray, N: int, K: int, mode: str = "f64", act: str = "q8"):
        self.b, self.N, self.K, self.mode, self.act = wbytes, N, K, mode, act
        self._w = None

    def dense(self):
        if self._w is None:
            if self.act == "f16":
                self._w = Q.dequant_q4_0_f16(self.b, (self.N, self.K)).astype(np.float64)
            else:
                self._w = Q.dequant_q4_0(self.b, (self.N, self.K)).astype(np.float64)
        return self._w

    def __call__(self, x: np.ndarray) -> np.ndarray:
        """x [T, K] -> Q8_1 (or fp16) activations -> y float64 [T, N]."""
        if self.act == "f16":
            return np.asarray(x).astype(np.float16).astype(np.float64) @ self.dense().T
        qx, dx, _ = Q.quantize_q8_1(np.asarray(x, np.float32))
        if self.mode == "int":
            return Q.gemv_q4_0_q8_1(self.b, self.N, self.K, qx, dx, out_dtype=np.float64)
        xf = Q.dequant_q8_1(qx, dx).astype(np.float64)
        return xf @ self.dense().T


@dataclass
class Model:
    """Random-weight model in oracle form. `w` is the dict produced by the weight generator:
    embed (GGUF Q4_0 bytes of E [V, H]), norm [H], layers[i] with ln1, ln2, wq, wk, wv, bq, bk, bv, wo, wg, wu, wd."""
    cfg: Config
    w: dict
    maxlen: int = 2048
    mode: str = "f64"
    act: str = "q8"              # "q8": Q8_1 activations (batch 1, prefill); "f16": the batched decode path
    lin: list = field(default_factory=list)

    def __post_init__(self):
        c = self.cfg
        self.cos, self.sin = rope_tables(self.maxlen, c.HD, c.theta)
        md, ac = self.mode, self.act
        for L in self.w["layers"]:
            self.lin.append({
                "q": Linear(L["wq"], c.NH * c.HD, c.H, md, ac), "k": Linear(L["wk"], c.NKV * c.HD, c.H, md, ac),
                "v": Linear(L["wv"], c.NKV * c.HD, c.H, md, ac), "o": Linear(L["wo"], c.H, c.NH * c.HD, md, ac),
                "g": Linear(L["wg"], c.FFN, c.H, md, ac), "u": Linear(L["wu"], c.FFN, c.H, md, ac),
                "d": Linear(L["wd"], c.H, c.FFN, md, ac)})
        # the LM head takes Q8_1 activations in both modes (the batched decode's head is the int8 kernel)
        self.head = (LinearQ6K(self.w["head_q6k"], c.V, c.H) if "head_q6k" in self.w
                     else Linear(self.w["embed"], c.V, c.H, md))

    def new_cache(self):
        c = self.cfg
        shape = (c.L, c.NKV, self.maxlen, c.HD)
        return {"K": np.zeros(shape, np.float16), "V": np.zeros(shape, np.float16)}

    def embed(self, toks) -> np.ndarray:
        c = self.cfg
        nb = c.H // Q.QK
        rows = [Q.dequant_q4_0(self.w["embed"][t * nb:(t + 1) * nb], (c.H,)) for t in toks]
        return np.stack(rows).astype(np.float32)

    def layer(self, i: int, h: np.ndarray, pos0: int, cache) -> np.ndarray:
        """One decoder layer for P tokens at positions pos0..pos0+P-1 of one sequence; h [P, H] -> new h (float64).
        Writes the layer's K/V rows into cache["K"][i], cache["V"][i]."""
        c = self.cfg
        L, lin = self.w["layers"][i], self.lin[i]
        P = h.shape[0]
        x = rmsnorm(h, L["ln1"], c.eps).astype(np.float32)
        q = lin["q"](x) + L["bq"]
        k = lin["k"](x) + L["bk"]
        v = lin["v"](x) + L["bv"]
        qh = np.empty((P, c.NH, c.HD), np.float16)
        for t in range(P):
            p = pos0 + t
            cs, sn = self.cos[p], self.sin[p]
            qh[t] = rope(q[t].reshape(c.NH, c.HD), cs, sn).astype(np.float16)
            cache["K"][i, :, p] = rope(k[t].reshape(c.NKV, c.HD), cs, sn).astype(np.float16)
            cache["V"][i, :, p] = v[t].reshape(c.NKV, c.HD).astype(np.float16)
        if P == 1:
            att = attn_decode(qh[0], cache["K"][i], cache["V"][i], pos0 + 1, c.NH, c.NKV)[None]
        else:
            att = attn_prefill(qh, cache["K"][i], cache["V"][i], pos0, c.NH, c.NKV)
        self.last = {"q": qh, "att": att}
        h = np.asarray(h, np.float64) + lin["o"](att)
        x = rmsnorm(h, L["ln2"], c.eps).astype(np.float32)
        m = silu_mul(lin["g"](x), lin["u"](x)).astype(np.float32)
        self.last["m"] = m
        return h + lin["d"](m)

    def forward(self, toks, pos0: int, cache) -> np.ndarray:
        """P tokens at positions pos0..pos0+P-1 of one sequence (P = 1: decode step; P > 1: prefill).
        Writes K/V rows into `cache`; returns the final hidden state h float64 [P, H]."""
        h = self.embed(toks)
        for i in range(len(self.w["layers"])):
            h = self.layer(i, h, pos0, cache)
        return h

    def decode_batch(self, toks, positions, caches) -> np.ndarray:
        """One decode token for each of S independent sequences: token toks[s] at position positions[s] of the
        sequence whose cache is caches[s] (the batched step, scripts/qwen_batched_decode.py:156-187). Each row
        follows Model.layer's single-token arithmetic (the same rounding points); only the GEMV products of the
        S rows are evaluated as one matrix product. Writes each sequence's K/V rows; returns h float64 [S, H].
        pinned by: equality (1e-12) with Model.forward run per sequence (tests/test_oracle.py)."""
        c = self.cfg
        S = len(toks)
        h = self.embed(toks).astype(np.float64)
        for i, (L, lin) in enumerate(zip(self.w["layers"], self.lin)):
            x = rmsnorm(h, L["ln1"], c.eps).astype(np.float32)
            q = lin["q"](x) + L["bq"]
            k = lin["k"](x) + L["bk"]
            v = lin["v"](x) + L["bv"]
            att = np.empty((S, c.NH * c.HD), np.float32)
            for r in range(S):
                p, cache = int(positions[r]), caches[r]
                cs, sn = self.cos[p], self.sin[p]
                qh = rope(q[r].reshape(c.NH, c.HD), cs, sn).astype(np.float16)
                cache["K"][i, :, p] = rope(k[r].reshape(c.NKV, c.HD), cs, sn).astype(np.float16)
                cache["V"][i, :, p] = v[r].reshape(c.NKV, c.HD).astype(np.float16)
                att[r] = attn_decode(qh, cache["K"][i], cache["V"][i], p + 1, c.NH, c.NKV)
            h = h + lin["o"](att)
            x = rmsnorm(h, L["ln2"], c.eps).astype(np.float32)
            m = silu_mul(lin["g"](x), lin["u"](x)).astype(np.float32)
            h = h + lin["d"](m)
        return h

    def logits(self, h: np.ndarray) -> np.ndarray:
        """Final RMSNorm + tied Q4_0 head -> fp32 [T, V]."""
        x = rmsnorm(h, self.w["norm"], self.cfg.eps).astype(np.float32)
        return self.head(x).astype(np.float32)

    def greedy(self, prompt, n_gen: int, cache=None):
        """Prefill the prompt (one forward over all prompt tokens), then n_gen greedy decode steps.
        Returns (tokens [n_gen], top-2 margins [n_gen]). Token 0 is the argmax after the prompt."""
        cache = cache if cache is not None else self.new_cache()
        h = self.forward(list(prompt), 0, cache)
        toks, margins = [], []
        pos = len(prompt)
        lg = self.logits(h[-1:])[0]
        for step in range(n_gen):
            t = argmax_lowest(lg)
            top2 = np.partition(lg, -2)[-2:]
            toks.append(t)
            margins.append(float(top2[1] - top2[0]))
            if step == n_gen - 1:
                break
            h = self.forward([t], pos, cache)
            pos += 1
            lg = self.logits(h)[0]
        return toks, margins
