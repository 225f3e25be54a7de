"""Qwen2.5-1.5B-shape Q4_0 model on one MI355X: synthetic weights, device layout, decode engine.

The decode step is the reference's FusedQwen.step (scripts/qwen_fused.py:113-145, GGUF variant
scripts/qwen_gguf.py:63-144) re-cut for gfx950 into 5 fused launches per layer:

  qkv_rope_kv   RMSNorm(ln1) + Q8_1 + QKV GEMV + bias + RoPE + fp16 K/V cache write   (fused prologue/epilogue)
  attn_decode   split-K GQA attention over 64-position pages -> per-chunk partials
  attn_o_resid  merge of the partials + Q8_1 + O GEMV (3 K slices), h += ...
  ffn_gate_up   RMSNorm(ln2) + Q8_1 + gate_up GEMV + SwiGLU -> m (fp32)
  ffn_down      Q8_1(m) + down GEMV (4 K slices), h += ...
The residual stream h is int64 fixed point (value * 2^48): the K-sliced projections add into it with
integer atomics, so results do not depend on workgroup timing. GEMV accumulation, RMSNorm, RoPE, attention
and SwiGLU run in f64 on this batch-1 path, so every Q8_1 quantizer input agrees with the f64 oracle to
~1e-14 and greedy decoding reproduces the oracle's tokens.
then head_logits (final RMSNorm + tied Q4_0 head + per-workgroup argmax partials) and finish
(argmax, tok <- idx, pos += 1). The whole step is captured once in a torch.cuda.CUDAGraph (a hipGraph)
and replayed per token, as run_fused does (scripts/qwen_fused.py:148-180).
"""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np

from . import gguf
from .hip import call, ptr

PAGE = 64
FIX_SCALE = 2.0 ** 48        # residual stream: int64 fixed point, value * 2^48


@dataclass(frozen=True)
class Config:
    """Qwen2.5-1.5B shape."""
    H: int = 1536
    NH: int = 12
    NKV: int = 2
    HD: int = 128
    FFN: int = 8960
    L: int = 28
    V: int = 151936
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def nqkv(self):
        return (self.NH + 2 * self.NKV) * self.HD


QWEN15 = Config()

# tensor ids for the per-tensor seeded generators
_TID = {"wq": 0, "wk": 1, "wv": 2, "wo": 3, "wg": 4, "wu": 5, "wd": 6, "bq": 7, "bk": 8, "bv": 9,
        "ln1": 10, "ln2": 11, "embed": 100, "norm": 101}


def _normal(seed: int, layer: int, name: str, n: int, std: float, mean: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng([seed, layer, _TID[name]])
    x = rng.standard_normal(n, dtype=np.float32)
    x *= np.float32(std)
    if mean:
        x += np.float32(mean)
    return x


def random_weights(cfg: Config = QWEN15, seed: int = 0, workers: int | None = None) -> dict:
    """Synthetic weights of BASELINE configs 1-4: every matrix fp32 N(0, 0.02) from its own seeded
    generator, quantized with the Q4_0 rule to GGUF bytes; QKV biases fp32 N(0, 0.02); RMSNorm weights
    1 + N(0, 0.01). The embedding is tied to the output head. Returns a dict of numpy arrays:
    embed, norm, layers[i] = {ln1, ln2, wq, wk, wv, bq, bk, bv, wo, wg, wu, wd}."""
    H, F = cfg.H, cfg.FFN
    shapes = {"wq": (cfg.NH * cfg.HD, H), "wk": (cfg.NKV * cfg.HD, H), "wv": (cfg.NKV * cfg.HD, H),
              "wo": (H, cfg.NH * cfg.HD), "wg": (F, H), "wu": (F, H), "wd": (H, F)}

    def mat(layer, name, rows, cols):
        return gguf.quantize_q4_0(_normal(seed, layer, name, rows * cols, 0.02))

    jobs = {}
    with ThreadPoolExecutor(max_workers=workers or min(16, os.cpu_count() or 4)) as ex:
        jobs["embed"] = ex.submit(mat, 1000, "embed", cfg.V, H)
        for i in range(cfg.L):
            for name, (r, c) in shapes.items():
                jobs[(i, name)] = ex.submit(mat, i, name, r, c)
        w = {"embed": jobs["embed"].result(), "norm": _normal(seed, 1000, "norm", H, 0.01, 1.0), "layers": []}
        for i in range(cfg.L):
            L = {name: jobs[(i, name)].result() for name in shapes}
            L["bq"] = _normal(seed, i, "bq", cfg.NH * cfg.HD, 0.02)
            L["bk"] = _normal(seed, i, "bk", cfg.NKV * cfg.HD, 0.02)
            L["bv"] = _normal(seed, i, "bv", cfg.NKV * cfg.HD, 0.02)
            L["ln1"] = _normal(seed, i, "ln1", H, 0.01, 1.0)
            L["ln2"] = _normal(seed, i, "ln2", H, 0.01, 1.0)
            w["layers"].append(L)
    return w


def rope_tables(maxlen: int, hd: int = 128, theta: float = 1e6):
    """cos/sin fp32 [maxlen, hd/2] from float64 angles (scripts/qwen_gguf.py:108-113)."""
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.arange(maxlen, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


class Q4Mat:
    """A Q4_0 matrix resident in HBM in the library's tiled planes."""

    def __init__(self, b: np.ndarray, N: int, K: int, device):
        import torch
        qs, d = gguf.tile_q4_0(b, N, K)
        self.N, self.K = N, K
        self.qs = torch.from_numpy(qs.reshape(-1)).to(device)
        self.d = torch.from_numpy(d.reshape(-1).view(np.int16)).to(device)
        from .refcall import register
        register(self.qs, self)           # W / E pointers of reference-order launches resolve to this matrix

    @property
    def nbytes(self):
        return self.qs.numel() + 2 * self.d.numel()

    def data_ptr(self):
        """The matrix's handle in reference-order launches (its qs plane's address)."""
        return self.qs.data_ptr()


class Q6KMat:
    """A Q6_K matrix (the output head of llama.cpp's Qwen2.5 Q4_0 files) in the library's Q6_K planes."""

    def __init__(self, b: np.ndarray, N: int, K: int, device):
        import torch
        lo, hi, sc, d = gguf.tile_q6_k(b, N, K)
        self.N, self.K = N, K
        self.lo = torch.from_numpy(lo.reshape(-1)).to(device)
        self.hi = torch.from_numpy(hi.reshape(-1)).to(device)
        self.sc = torch.from_numpy(sc.reshape(-1).view(np.uint8)).to(device)
        self.d = torch.from_numpy(d.reshape(-1).view(np.int16)).to(device)
        from .refcall import register
        register(self.lo, self)           # the head pointer of reference-order launches resolves to this matrix

    @property
    def nbytes(self):
        return self.lo.numel() + self.hi.numel() + self.sc.numel() + 2 * self.d.numel()

    def data_ptr(self):
        return self.lo.data_ptr()


def weights_from_gguf(path) -> tuple:
    """A Qwen2 GGUF file (llama.cpp tensor names) -> (Config, weight dict) in the random_weights layout
    (scripts/qwen_gguf.py:63-121): Q4_0 matrices as GGUF bytes, norms and QKV biases fp32, the Q4_0 token
    embedding; output.weight (Q6_K in llama.cpp's Q4_0 files) becomes w["head_q6k"], else the head is tied.
    Every matrix of a layer must be Q4_0."""
    g = gguf.GGUF(path)
    m = g.meta
    H, nh, nkv = m["qwen2.embedding_length"], m["qwen2.attention.head_count"], m["qwen2.attention.head_count_kv"]
    emb_b, emb_t = g.raw("token_embd.weight")
    if emb_t.type != 2:
        raise ValueError(f"token_embd.weight is ggml type {emb_t.type}; this path needs Q4_0")
    cfg = Config(H=H, NH=nh, NKV=nkv, HD=H // nh, FFN=m["qwen2.feed_forward_length"], L=m["qwen2.block_count"],
                 V=emb_t.dims[1], eps=float(m["qwen2.attention.layer_norm_rms_epsilon"]),
                 theta=float(m.get("qwen2.rope.freq_base", 1e6)))

    def q4(name):
        b, t = g.raw(name)
        if t.type != 2:
            raise ValueError(f"{name} is ggml type {t.type}; this path needs Q4_0")
        return np.array(b, np.uint8).reshape(-1, 18)

    f32 = lambda name: np.array(g.f32(name), np.float32).reshape(-1)  # noqa: E731  (a writable copy)
    w = {"embed": q4("token_embd.weight"), "norm": f32("output_norm.weight"), "layers": []}
    for i in range(cfg.L):
        p = f"blk.{i}."
        w["layers"].append({
            "wq": q4(p + "attn_q.weight"), "wk": q4(p + "attn_k.weight"), "wv": q4(p + "attn_v.weight"),
            "bq": f32(p + "attn_q.bias"), "bk": f32(p + "attn_k.bias"), "bv": f32(p + "attn_v.bias"),
            "wo": q4(p + "attn_output.weight"), "wg": q4(p + "ffn_gate.weight"), "wu": q4(p + "ffn_up.weight"),
            "wd": q4(p + "ffn_down.weight"), "ln1": f32(p + "attn_norm.weight"), "ln2": f32(p + "ffn_norm.weight")})
    if "output.weight" in g.tensors:
        b, t = g.raw("output.weight")
        if t.type != 14:
            raise ValueError(f"output.weight is ggml type {t.type}; Q6_K or a tied head is supported")
        w["head_q6k"] = np.array(b, np.uint8).reshape(-1, 210)
    return cfg, w


class DeviceModel:
    """Weights of the whole model in HBM, in device row orders (QKV pair-interleaved for RoPE,
    gate/up interleaved for SwiGLU)."""

    def __init__(self, w: dict, cfg: Config = QWEN15, maxlen: int = 2048, device="cuda"):
        import torch
        self.cfg, self.maxlen, self.device = cfg, maxlen, device
        H, nqkv = cfg.H, cfg.nqkv
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)  # noqa: E731
        qkv_order = gguf.qkv_row_order(cfg.NH, cfg.NKV, cfg.HD)
        gu_order = gguf.gate_up_row_order(cfg.FFN)
        self.layers = []
        for L in w["layers"]:
            qkv = np.concatenate([L["wq"], L["wk"], L["wv"]])
            bias = np.concatenate([L["bq"], L["bk"], L["bv"]])[qkv_order]
            gu = np.concatenate([L["wg"], L["wu"]])
            self.layers.append({
                "ln1": f32(L["ln1"]), "ln2": f32(L["ln2"]), "qkv_b": f32(bias),
                "qkv": Q4Mat(gguf.take_rows_q4_0(qkv, H, qkv_order), nqkv, H, device),
                "o": Q4Mat(L["wo"], H, cfg.NH * cfg.HD, device),
                "gu": Q4Mat(gguf.take_rows_q4_0(gu, H, gu_order), 2 * cfg.FFN, H, device),
                "down": Q4Mat(L["wd"], H, cfg.FFN, device)})
        self.embed = Q4Mat(w["embed"], cfg.V, H, device)
        self.head_q6k = Q6KMat(w["head_q6k"], cfg.V, H, device) if "head_q6k" in w else None
        self.norm = f32(w["norm"])
        cos, sin = rope_tables(maxlen, cfg.HD, cfg.theta)
        self.cos, self.sin = f32(cos), f32(sin)

    def weight_bytes_per_token(self) -> int:
        per = sum(L[n].nbytes for L in self.layers for n in ("qkv", "o", "gu", "down"))
        return per + (self.head_q6k.nbytes if self.head_q6k is not None else self.embed.nbytes)


class Decoder:
    """Batch-T decode state (T <= 4 on the GEMV path) over a paged fp16 KV cache, and the step launch order.
    Mirrors FusedQwen (scripts/qwen_fused.py:55-145): buffers h, tok, pos, logits; step(); graph capture."""

    def __init__(self, m: DeviceModel, T: int = 1, max_ctx: int | None = None):
        import torch
        cfg = m.cfg
        self.m, self.cfg, self.T = m, cfg, T
        dev = m.device
        max_ctx = max_ctx or m.maxlen
        assert max_ctx <= m.maxlen
        self.max_chunks = -(-max_ctx // PAGE)
        n_pages = T * self.max_chunks
        self.kc = [torch.zeros(n_pages, cfg.NKV, PAGE, cfg.HD, dtype=torch.float16, device=dev) for _ in range(cfg.L)]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        # sequence j owns pages [j*max_chunks, (j+1)*max_chunks) (identity block table; paged layout)
        self.block_table = torch.arange(n_pages, dtype=torch.int32, device=dev).reshape(T, self.max_chunks)
        H = cfg.H
        self.h = torch.zeros(T, H, dtype=torch.int64, device=dev)       # fixed point, value * 2^48
        self.q = torch.zeros(T, cfg.NH * cfg.HD, dtype=torch.float16, device=dev)
        self.mlp = torch.zeros(T, cfg.FFN, dtype=torch.float32, device=dev)
        self.logits = torch.zeros(T, cfg.V, dtype=torch.float32, device=dev)
        self.nparts = call("q355_head_nparts", cfg.V)
        self.pmax = torch.zeros(T, self.nparts, dtype=torch.float32, device=dev)
        self.pidx = torch.zeros(T, self.nparts, dtype=torch.int32, device=dev)
        self.part = torch.zeros(T, cfg.NH, self.max_chunks, cfg.HD + 2, dtype=torch.float64, device=dev)
        self.tok = torch.zeros(T, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(T, dtype=torch.int32, device=dev)
        self.scale = 1.0 / math.sqrt(cfg.HD)

    # -- residual stream as fp32 (host-side views for tests and debugging) --
    def h_f64(self):
        import torch
        return self.h.to(torch.float64) / FIX_SCALE

    def h_f32(self):
        import torch
        return self.h_f64().to(torch.float32)

    def set_h(self, h):
        """Set the residual stream from fp32 values [T, H] (numpy or torch)."""
        import torch
        t = torch.as_tensor(np.asarray(h, np.float32)).to(self.h.device)
        self.h.copy_(torch.round(t.to(torch.float64) * FIX_SCALE).to(torch.int64))

    # -- per-layer ops (each is one library call) --
    def layer(self, i: int, embed: bool = False):
        """Layer i; with embed=True its QKV launch also takes the embedding of tok (q355_qkv_rope_kv_embed:
        the same h and q/k/v as embed() followed by layer(i), one launch fewer)."""
        m, c, T = self.m, self.cfg, self.T
        L = m.layers[i]
        qkv, o, gu, down = L["qkv"], L["o"], L["gu"], L["down"]
        if embed:
            e = m.embed
            call("q355_qkv_rope_kv_embed", ptr(qkv.qs), ptr(qkv.d), c.H, ptr(e.qs), ptr(e.d), e.N, ptr(self.tok),
                 ptr(self.h), ptr(L["ln1"]), c.eps, ptr(L["qkv_b"]), ptr(m.cos), ptr(m.sin), ptr(self.pos),
                 ptr(self.block_table), self.max_chunks, 1, ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.q), c.NH,
                 c.NKV, T)
        else:
            call("q355_qkv_rope_kv", ptr(qkv.qs), ptr(qkv.d), c.H, ptr(self.h), ptr(L["ln1"]), c.eps,
                 ptr(L["qkv_b"]), ptr(m.cos), ptr(m.sin), ptr(self.pos), ptr(self.block_table), self.max_chunks, 1,
                 ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.q), c.NH, c.NKV, T)
        call("q355_attn_decode", ptr(self.q), ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.pos), ptr(self.block_table),
             self.max_chunks, c.NH, c.NKV, self.max_chunks, self.scale, ptr(self.part), None, None, None, T, 0)
        call("q355_attn_o_resid", ptr(o.qs), ptr(o.d), o.N, ptr(self.part), self.max_chunks, ptr(self.pos), c.NH,
             ptr(self.h), T)
        call("q355_ffn_gate_up", ptr(gu.qs), ptr(gu.d), gu.N, gu.K, ptr(self.h), ptr(L["ln2"]), c.eps,
             ptr(self.mlp), T)
        call("q355_ffn_down", ptr(down.qs), ptr(down.d), down.N, down.K, ptr(self.mlp), ptr(self.h), T)

    def embed(self):
        e = self.m.embed
        call("q355_embed_q4_0", ptr(e.qs), ptr(e.d), e.N, e.K, ptr(self.tok), ptr(self.h), self.T)

    def head(self):
        e, q6 = self.m.embed, self.m.head_q6k
        if q6 is not None:     # llama.cpp's Q6_K output.weight
            call("q355_head_logits_q6k", ptr(q6.lo), ptr(q6.hi), ptr(q6.sc), ptr(q6.d), q6.N, q6.K, ptr(self.h),
                 ptr(self.m.norm), self.cfg.eps, ptr(self.logits), ptr(self.pmax), ptr(self.pidx), self.T)
        else:                  # tied Q4_0 head
            call("q355_head_logits", ptr(e.qs), ptr(e.d), e.N, e.K, ptr(self.h), ptr(self.m.norm), self.cfg.eps,
                 ptr(self.logits), ptr(self.pmax), ptr(self.pidx), self.T)
        call("q355_finish", ptr(self.pmax), ptr(self.pidx), self.nparts, ptr(self.tok), ptr(self.pos), self.T)

    def step(self):
        """One decode step for all T sequences: embed tok at pos (inside layer 0's QKV launch), 28 layers, head,
        tok <- argmax, pos += 1."""
        for i in range(self.cfg.L):
            self.layer(i, embed=(i == 0))
        self.head()

    # -- graph capture / replay (scripts/qwen_fused.py:148-180) --
    def capture(self):
        import torch
        pos0, tok0 = self.pos.clone(), self.tok.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()                     # warm-up outside capture
        torch.cuda.current_stream().wait_stream(side)
        self.pos.copy_(pos0)
        self.tok.copy_(tok0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.pos.copy_(pos0)
        self.tok.copy_(tok0)
        torch.cuda.synchronize()
        self.graph = g
        return g

    def prefill_tokens(self, ids):
        """Run the prompt token by token through step() (run_fused's prompt loop, scripts/qwen_fused.py:150-152);
        sequence j gets ids[j] (T == 1: ids is a flat list). Leaves tok = first generated token."""
        import torch
        ids = np.asarray(ids).reshape(self.T, -1) if self.T > 1 else np.asarray(ids).reshape(1, -1)
        for t in range(ids.shape[1]):
            self.tok.copy_(torch.from_numpy(ids[:, t].astype(np.int32)))
            self.step()

    def generate(self, n: int, use_graph: bool = True):
        """n greedy tokens (token 0 = current tok). Returns int array [T, n]."""
        import torch
        out = [self.tok.clone()]
        if use_graph and not hasattr(self, "graph"):
            self.capture()
        for _ in range(n - 1):
            if use_graph:
                self.graph.replay()
            else:
                self.step()
            out.append(self.tok.clone())
        return torch.stack(out, 1).cpu().numpy()
