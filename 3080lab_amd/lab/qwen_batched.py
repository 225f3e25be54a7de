"""Batched decode and prefill, with the reference's lab/qwen_batched.py names.

The reference's batched step (scripts/qwen_batched_decode.py:156-187) runs B sequences per step with
tensor-core GEMVs over bf16 activations (gemv_v2_source) and per-sequence contiguous bf16 KV caches.
Here B sequences share one step (BatchedDecoder). With act "f16" (the reference's gemv_v2 arithmetic):
  rmsnorm_fix_f16        RMSNorm of the fixed-point residual stream -> fp16 activations (per token)
  gemm_f16 (resid_fix)   QKV: fp16-dequantized Q4_0 x fp16 on v_mfma_f32_16x16x32_f16, K-sliced into int64
  qkv_finish             bias + RoPE + fp16 q + paged fp16 K/V write (clears the accumulator)
  attn_decode_f16        GQA attention on the matrix cores over 64-position pages + merge -> fp16
  gemm_f16 (resid_fix)   O projection into the residual stream
  rmsnorm_fix_f16, gemm_f16 (swiglu_f16)   gate_up + SwiGLU -> fp16
  gemm_f16 (resid_fix)   down projection into the residual stream
then rmsnorm_fix_q8_1 + mmq (logits) over the tied Q4_0 head + finish (argmax per sequence, pos += 1).
act "q8" (the default; BASELINE config 3 specifies int8 MMQ) runs the same step on Q8_1 activations and the
int8 MMQ kernels, with the matrix-core attention merged to Q8_1.
The KV cache is paged: a shared pool of 64-position pages, one block-table row per sequence.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .hip import call, ptr
from .qwen_kernels import KernelSpec
from .qwen_model import FIX_SCALE, PAGE, Config, DeviceModel


# reference generator names (lab/qwen_batched.py) -> the C-ABI entry points that replace them
def gemv_v2_source(WM=1, WK=1, MT=1, B=8, epi="store", PF=1, KS=1, ACC16=False) -> KernelSpec:
    """Batched decode GEMV (lab/qwen_batched.py:467-641) -> the fp16-weight products of the same arithmetic (fp16
    weight dequantization, fp16 MFMA, fp32 accumulation into the fixed-point residual). Launched with the
    reference's (W, S, X, Y, aux, N, K, ws, cnt) (lab/refcall.py:launch_gemv_v2): biasf on the qkv buffer ->
    q355_gemm_f16_qkv_rope at the ATTN launch; resid on the attention output -> the O product (split merge in
    its staging up to 16 tokens); swiglu -> q355_gemm_q4_0_f16 epi 8; resid -> epi 6. The tile shape (WM, WK,
    MT, KS, PF, ACC16) is the library's choice per shape and batch, so those arguments have no counterpart."""
    if epi not in ("store", "logits", "resid", "biasf", "swiglu"):
        raise ValueError(f"epilogue {epi!r}: store, logits, resid, biasf or swiglu")
    code = {"store": 0, "logits": 5, "resid": 6, "biasf": 6, "swiglu": 8}[epi]
    return KernelSpec("q355_gemm_q4_0_f16", {"epi": code, "epi_name": epi, "B": int(B)}, ref="gemv_v2")


def head_v2_source(WM=8, WK=1, MT=1, B=8, PF=1) -> KernelSpec:
    """Batched LM head (lab/qwen_batched.py:681-833), launched with (*head, x, logits, V, H): the final RMSNorm's
    Q8_1 times the head on int8 MFMA (the tied Q4_0 matrix, or llama.cpp's Q6_K output.weight) -> fp32 logits and
    argmax partials (lab/refcall.py:launch_head_v2)."""
    return KernelSpec("q355_mmq_q4_0_q8_1", {"B": int(B)}, ref="head_v2")


def batchify(spec: KernelSpec, lines: str = "") -> KernelSpec:
    """The reference's batchify (scripts/qwen_batched_decode.py:74-86) edits kernel source to offset each pointer by
    blockIdx.y; the library's entry points take the batch size, which Kern.launch reads from grid.y."""
    return KernelSpec(spec.symbol, {**spec.params, "batched": True}, spec.ref)


def gemm_q4i8_ms_source(WM=4, WN=2, MT=2, NT=4, epi="store", KB=4, NSTG=2, MINB=1, ABL=None) -> KernelSpec:
    """Prefill MMQ (lab/qwen_batched.py:1271-1561) -> the same int8 MFMA entry point (epi as above)."""
    e = epi.split(":")[0]
    code = {"store": 0, "resid": 6, "biasf": 6, "biasf_kv": 6, "swiglu": 7, "swiglu_q8": 7}[e]
    return KernelSpec("q355_mmq_q4_0_q8_1", {"epi": code})


gemm_q4i8_source = gemm_q4i8_ms_source
QUANT_Q8 = KernelSpec("q355_quant_q8_1")


def rmsnorm_q8_source(H: int) -> KernelSpec:
    """RMSNorm + Q8 quantizer (lab/qwen_batched.py:1044-1091) over the fixed-point residual stream."""
    return KernelSpec("q355_rmsnorm_fix_q8_1", {"H": H})


def pack_q6_mma(*head):
    """The reference repacks the Q6_K head into mma fragment order (lab/qwen_batched.py:439-466); the library's
    Q6_K planes (lab.gguf.tile_q6_k) already are its MFMA operand order, so this is the identity."""
    return head


def pack_q4_i8(W, S):
    """The reference repacks Q4_0 into mma fragment order (lab/qwen_batched.py:987-1013). The MI355X
    layout (16-row tiled planes, lab.gguf.tile_q4_0) already is the MFMA A-operand order, so this is the
    identity on (qs, d) planes."""
    return W, S


pack_q4_mma = pack_q4_i8


# up to this batch the attention merge runs inside the O product's staging (int8 and fp16 paths) (saves the merge
# launch: B = 8 step 1.391 -> 1.329 ms); above it the separate merge measured no slower
MERGE_IN_O_MAX_B = 16


class BatchedDecoder:
    """B sequences decoded together over a paged fp16 KV cache (scripts/qwen_batched_decode.py:86-187).

    ctx_pages: pages per sequence (max context / 64). Pages come from one pool and are assigned to the
    sequences in a seeded random order (the block table is a permutation), so the kernels are exercised
    on non-contiguous pages."""

    def __init__(self, m: DeviceModel, B: int, max_ctx: int, page_seed: int = 0, act: str = "q8",
                 keep_logits: bool = False):
        """act "q8" (default: Q4_0 x Q8_1 int8 MMQ on MFMA): Q8_1 activations on the int8
        MMQ kernels; "f16": fp16 activations and fp16-dequantized weights on the fp16 matrix cores, the
        reference's own batched decode arithmetic (gemv_v2_source, lab/qwen_batched.py:467-680).
        keep_logits: also write the fp32 logits [B][V] (19 MB at B = 32) to self.logits; the greedy token
        needs only the head's per-64-row argmax partials."""
        self.keep_logits = keep_logits
        import torch
        c = m.cfg
        if act not in ("f16", "q8"):
            raise ValueError(f"act={act!r}: 'f16' or 'q8'")
        self.m, self.cfg, self.B, self.act = m, c, B, act
        dev = m.device
        self.max_chunks = -(-max_ctx // PAGE)
        n_pages = B * self.max_chunks
        order = np.random.default_rng(page_seed).permutation(n_pages).astype(np.int32)
        self.block_table = torch.from_numpy(order.reshape(B, self.max_chunks)).to(dev)
        self.kc = [torch.zeros(n_pages, c.NKV, PAGE, c.HD, dtype=torch.float16, device=dev) for _ in range(c.L)]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        H = c.H
        self.h = torch.zeros(B, H, dtype=torch.int64, device=dev)
        self.xq = torch.zeros(B, max(H, c.FFN), dtype=torch.int8, device=dev)
        self.xds = torch.zeros(B, max(H, c.FFN) // 32, 2, dtype=torch.float16, device=dev)
        self.mq = torch.zeros(B, c.FFN, dtype=torch.int8, device=dev)
        self.mds = torch.zeros(B, c.FFN // 32, 2, dtype=torch.float16, device=dev)
        self.q = torch.zeros(B, c.NH * c.HD, dtype=torch.float16, device=dev)
        self.q64 = torch.zeros(B, c.NH * c.HD, dtype=torch.float64, device=dev)   # the int8 path's f64 queries
        self.part = torch.zeros(B, c.NH, self.max_chunks, c.HD + 2, dtype=torch.float64, device=dev)
        self.aq = torch.zeros(B, c.NH * c.HD, dtype=torch.int8, device=dev)
        self.xh = torch.zeros(B, max(H, c.NH * c.HD), dtype=torch.float16, device=dev)
        self.ah = torch.zeros(B, c.NH * c.HD, dtype=torch.float16, device=dev)
        self.mh = torch.zeros(B, c.FFN, dtype=torch.float16, device=dev)
        self.m32 = torch.zeros(B, c.FFN, dtype=torch.float32, device=dev)
        self.ads = torch.zeros(B, c.NH * c.HD // 32, 2, dtype=torch.float16, device=dev)
        self.logits = torch.zeros(B, c.V, dtype=torch.float32, device=dev)
        self.nparts = call("q355_mmq_nparts", c.V)
        self.pmax = torch.zeros(B, self.nparts, dtype=torch.float32, device=dev)
        self.pidx = torch.zeros(B, self.nparts, dtype=torch.int32, device=dev)
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.scale = 1.0 / math.sqrt(c.HD)
        # the step's live (token, KV head, split) items of the f64 attention, rebuilt by layer 0 of every step
        nb = call("q355_attn_f64_worklist_bytes", B, c.NKV, self.max_chunks)
        self.work = torch.zeros(nb // 4, dtype=torch.int32, device=dev) if B <= 64 else None

    def h_f32(self):
        import torch
        return (self.h.to(torch.float64) / FIX_SCALE).to(torch.float32)

    def _norm(self, w):
        c = self.cfg
        call("q355_rmsnorm_fix_q8_1", ptr(self.h), ptr(w), ptr(self.xq), ptr(self.xds), self.B, c.H, c.eps)

    def _mmq(self, W, xq, xds, epi, y=None, yfix=None, oq=None, ods=None, pmax=None, pidx=None):
        call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(xq), ptr(xds), self.B, epi,
             ptr(y), ptr(yfix), ptr(oq), ptr(ods), ptr(pmax), ptr(pidx))

    def _normh(self, w):
        c = self.cfg
        call("q355_rmsnorm_fix_f16", ptr(self.h), ptr(w), ptr(self.xh), self.B, c.H, c.eps)

    def _gemm(self, W, xh, epi, y=None, yfix=None, yh=None, pmax=None, pidx=None):
        call("q355_gemm_q4_0_f16", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(xh), self.B, epi, ptr(y), ptr(yfix), ptr(yh),
             ptr(pmax), ptr(pidx))

    def layer_f16(self, i: int):
        m, c, B = self.m, self.cfg, self.B
        L = m.layers[i]
        self._normh(L["ln1"])
        W = L["qkv"]                 # bias, RoPE and the K/V write in the product's epilogue
        call("q355_gemm_f16_qkv_rope", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xh), B, ptr(L["qkv_b"]), ptr(m.cos),
             ptr(m.sin), ptr(self.pos), ptr(self.block_table), self.max_chunks, 1, ptr(self.kc[i]), ptr(self.vc[i]),
             ptr(self.q), c.NH, c.NKV)
        if B <= MERGE_IN_O_MAX_B:
            # attention leaves split partials; the O product merges them per head while staging its activations
            call("q355_attn_decode_partials_f16", ptr(self.q), ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.pos),
                 ptr(self.block_table), self.max_chunks, c.NH, c.NKV, self.max_chunks, self.scale, ptr(self.part),
                 ptr(self.ah), B)
            W = L["o"]
            call("q355_gemm_f16_attn_o_resid", ptr(W.qs), ptr(W.d), W.N, ptr(self.part), self.max_chunks,
                 ptr(self.pos), c.NH, c.NKV, ptr(self.ah), ptr(self.h), B)
        else:
            call("q355_attn_decode_f16", ptr(self.q), ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.pos),
                 ptr(self.block_table), self.max_chunks, c.NH, c.NKV, self.max_chunks, self.scale, ptr(self.part),
                 ptr(self.ah), B)
            self._gemm(L["o"], self.ah, 6, yfix=self.h)
        self._normh(L["ln2"])
        self._gemm(L["gu"], self.xh, 8, yh=self.mh)
        self._gemm(L["down"], self.mh, 6, yfix=self.h)

    def layer(self, i: int):
        if self.act == "f16":
            return self.layer_f16(i)
        m, c, B = self.m, self.cfg, self.B
        L = m.layers[i]
        self._norm(L["ln1"])
        W = L["qkv"]                 # bias, RoPE and the K/V write in the product's epilogue; q also widened to f64
        call("q355_mmq_qkv_rope", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xq), ptr(self.xds), B, ptr(L["qkv_b"]),
             ptr(m.cos), ptr(m.sin), ptr(self.pos), ptr(self.block_table), self.max_chunks, 1, ptr(self.kc[i]),
             ptr(self.vc[i]), ptr(self.q), ptr(self.q64), c.NH, c.NKV)
        # f64 attention (the batch-1 arithmetic), split merge in f64 -> Q8_1
        args = (ptr(self.q64), ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.pos), ptr(self.block_table),
                self.max_chunks, c.NH, c.NKV, self.max_chunks, self.scale, ptr(self.part), ptr(self.aq),
                ptr(self.ads), None, B)
        if self.work is None:
            call("q355_attn_decode_f64", *args)
        else:
            if i == 0:                       # positions are fixed for the rest of the step
                call("q355_attn_f64_worklist", ptr(self.pos), ptr(self.block_table), self.max_chunks, c.NKV,
                     self.max_chunks, B, ptr(self.work))
            call("q355_attn_decode_f64_wl", *args, ptr(self.work))
        self._mmq(L["o"], self.aq, self.ads, 6, yfix=self.h)
        self._norm(L["ln2"])
        if B <= 16:
            # SwiGLU kept in fp32 and quantized to Q8_1 inside the down product (register-resident kernels;
            # faster up to 16 tokens, where the down kernel's fp32 activation reads stay small)
            self._mmq(L["gu"], self.xq, self.xds, 4, y=self.m32)
            W = L["down"]
            call("q355_mmq_q4_0_f32", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.m32), B, ptr(self.h))
        else:
            self._mmq(L["gu"], self.xq, self.xds, 7, oq=self.mq, ods=self.mds)
            self._mmq(L["down"], self.mq, self.mds, 6, yfix=self.h)

    def step(self):
        c, m = self.cfg, self.m
        e = m.embed
        call("q355_embed_q4_0", ptr(e.qs), ptr(e.d), e.N, e.K, ptr(self.tok), ptr(self.h), self.B)
        for i in range(c.L):
            self.layer(i)
        # the LM head runs on Q8_1 activations in both modes (the int8 LDS-tiled kernel reads its 131 MB once)
        self._norm(m.norm)
        if m.head_q6k is not None:           # llama.cpp's Q6_K output.weight, 32 tokens per launch
            q6 = m.head_q6k
            for j in range(0, self.B, 32):
                n = min(32, self.B - j)
                # the normalized activations are packed [B][H] (int8) and [B][H/32] (half2) from the buffer start
                call("q355_mmq_q6k_logits", ptr(q6.lo), ptr(q6.hi), ptr(q6.sc), ptr(q6.d), q6.N, q6.K,
                     ptr(self.xq) + j * c.H, ptr(self.xds) + j * (c.H // 32) * 4, n,
                     ptr(self.logits[j]) if self.keep_logits else None, ptr(self.pmax[j]), ptr(self.pidx[j]))
        else:
            self._mmq(e, self.xq, self.xds, 5, y=self.logits if self.keep_logits else None, pmax=self.pmax,
                      pidx=self.pidx)
        call("q355_finish", ptr(self.pmax), ptr(self.pidx), self.nparts, ptr(self.tok), ptr(self.pos), self.B)

    def capture(self):
        import torch
        pos0, tok0 = self.pos.clone(), self.tok.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()
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
        """ids int [B, P]: feed the prompts token by token through step() (scripts/qwen_batched_decode.py:205-208)."""
        import torch
        ids = np.asarray(ids)
        for t in range(ids.shape[1]):
            self.tok.copy_(torch.from_numpy(ids[:, t].astype(np.int32)))
            self.step()

    def fill_random_context(self, ctx_lens, seed: int = 0):
        """Synthetic contexts: positions 0..ctx-1 of every sequence and layer filled with
        N(0, 1) fp16 K/V; pos[b] = ctx_lens[b]. Generated on the GPU (torch, seeded)."""
        import torch
        g = torch.Generator(device=self.m.device).manual_seed(seed)
        for i in range(self.cfg.L):
            self.kc[i].normal_(generator=g)
            self.vc[i].normal_(generator=g)
        self.pos.copy_(torch.as_tensor(np.asarray(ctx_lens, np.int32)))

    def generate(self, n: int, use_graph: bool = True):
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


def flash_prefill_v3_source(maxlen: int = 4096, q8: bool = True) -> KernelSpec:
    """Causal prefill flash attention (lab/qwen_batched.py:1795-2037) -> q355_attn_prefill (fp16 MFMA,
    fp32 accumulation, fp32 output) or, with q8 (lab/qwen_batched.py:1811-1848), q355_attn_prefill_q8_1: the
    output quantized to Q8_1 for the O projection in the same launch."""
    return KernelSpec("q355_attn_prefill_q8_1" if q8 else "q355_attn_prefill")


# chunks of at least this many tokens run the QKV product on the LDS-tiled kernel with the finish in its
# epilogue (q355_mmq_qkv_rope); shorter ones keep the K-split product into the int64 accumulator plus
# q355_qkv_finish, which has parallelism enough at small P. From 512 tokens on every product of a chunk runs
# the LDS-tiled kernel, so chunking a prompt into pieces of >= 512 tokens gives the same results bit for bit.
QKV_FUSED_MIN_P = 512


class Prefill:
    """Chunked prefill of one sequence into a batch-1 Decoder's paged KV cache (scripts/qwen_prefill.py:196-246).

    chunk(ids, pos0) runs P prompt tokens at positions pos0 .. pos0 + P - 1 through all layers at once:
      embed -> per layer: rmsnorm_fix_q8_1, MMQ qkv with bias + RoPE + K/V write in its epilogue
      (P >= QKV_FUSED_MIN_P; else MMQ qkv into an int64 accumulator + qkv_finish),
      attn_prefill_q8_1 (causal, fp16 MFMA, Q8_1 output), MMQ o (+= h), rmsnorm_fix_q8_1, MMQ gate_up (SwiGLU -> Q8_1),
      MMQ down (+= h) -> final norm + head on the last token -> dec.tok = argmax, dec.pos = pos0 + P.
    The decoder then continues greedy decode from that state."""

    def __init__(self, dec, max_chunk: int = 2048):
        import torch
        m, c = dec.m, dec.cfg
        assert dec.T == 1, "prefill fills sequence 0 of a batch-1 decoder"
        self.dec, self.m, self.cfg, self.P_max = dec, m, c, max_chunk
        dev = m.device
        P, H = max_chunk, c.H
        self.h = torch.zeros(P, H, dtype=torch.int64, device=dev)
        self.xq = torch.zeros(P, max(H, c.FFN), dtype=torch.int8, device=dev)
        self.xds = torch.zeros(P, max(H, c.FFN) // 32, 2, dtype=torch.float16, device=dev)
        self.qkv_acc = torch.zeros(P, c.nqkv, dtype=torch.int64, device=dev)
        self.q = torch.zeros(P, c.NH * c.HD, dtype=torch.float16, device=dev)
        self.mq = torch.zeros(P, c.FFN, dtype=torch.int8, device=dev)
        self.mds = torch.zeros(P, c.FFN // 32, 2, dtype=torch.float16, device=dev)
        self.ids = torch.zeros(P, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(P, dtype=torch.int32, device=dev)
        self.fin_pos = torch.zeros(1, dtype=torch.int32, device=dev)
        # key-split workspace of the attention (zeroed once; its arrival counters reset themselves)
        nbytes = call("q355_attn_prefill_ws_bytes", P, dec.max_chunks * 64, c.NH, c.NKV)
        self.attn_ws = torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=dev)
        self.scale = 1.0 / math.sqrt(c.HD)

    def layer(self, i: int, P: int, pos0: int):
        m, c, d = self.m, self.cfg, self.dec
        L = m.layers[i]
        call("q355_rmsnorm_fix_q8_1", ptr(self.h), ptr(L["ln1"]), ptr(self.xq), ptr(self.xds), P, c.H, c.eps)
        W = L["qkv"]
        if P >= QKV_FUSED_MIN_P:
            # one writer per output: the finish (bias, RoPE, K/V write) runs in the GEMM epilogue
            call("q355_mmq_qkv_rope", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xq), ptr(self.xds), P, ptr(L["qkv_b"]),
                 ptr(m.cos), ptr(m.sin), ptr(self.pos), ptr(d.block_table), d.max_chunks, 0, ptr(d.kc[i]),
                 ptr(d.vc[i]), ptr(self.q), None, c.NH, c.NKV)
        else:
            call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xq), ptr(self.xds), P, 6,
                 None, ptr(self.qkv_acc), None, None, None, None)
            call("q355_qkv_finish", ptr(self.qkv_acc), ptr(L["qkv_b"]), ptr(m.cos), ptr(m.sin), ptr(self.pos),
                 ptr(d.block_table), d.max_chunks, 0, ptr(d.kc[i]), ptr(d.vc[i]), ptr(self.q), c.NH, c.NKV, P)
        call("q355_attn_prefill_q8_1", ptr(self.q), ptr(d.kc[i]), ptr(d.vc[i]), ptr(d.block_table), pos0, P, c.NH,
             c.NKV, self.scale, ptr(self.xq), ptr(self.xds), ptr(self.attn_ws), self.attn_ws.numel() * 4)
        W = L["o"]
        call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xq), ptr(self.xds), P, 6,
             None, ptr(self.h), None, None, None, None)
        call("q355_rmsnorm_fix_q8_1", ptr(self.h), ptr(L["ln2"]), ptr(self.xq), ptr(self.xds), P, c.H, c.eps)
        W = L["gu"]
        call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.xq), ptr(self.xds), P, 7,
             None, None, ptr(self.mq), ptr(self.mds), None, None)
        W = L["down"]
        call("q355_mmq_q4_0_q8_1", ptr(W.qs), ptr(W.d), W.N, W.K, ptr(self.mq), ptr(self.mds), P, 6,
             None, ptr(self.h), None, None, None, None)

    def chunk(self, ids, pos0: int = 0):
        """Prefill ids (int array, len P <= max_chunk) at positions pos0.. ; leaves dec.tok = the next token."""
        import torch
        ids = np.asarray(ids, np.int32).reshape(-1)
        P = len(ids)
        c, m, d = self.cfg, self.m, self.dec
        assert 1 <= P <= self.P_max and pos0 + P <= d.max_chunks * PAGE
        self.ids[:P].copy_(torch.from_numpy(ids))
        self.pos[:P].copy_(torch.arange(pos0, pos0 + P, dtype=torch.int32))
        self.enqueue(P, pos0)

    def enqueue(self, P: int, pos0: int):
        """The launches of chunk() on the current stream (ids/pos already set; capturable)."""
        c, m, d = self.cfg, self.m, self.dec
        e = m.embed
        call("q355_embed_q4_0", ptr(e.qs), ptr(e.d), e.N, e.K, ptr(self.ids), ptr(self.h), P)
        for i in range(c.L):
            self.layer(i, P, pos0)
        call("q355_head_logits", ptr(e.qs), ptr(e.d), e.N, e.K, ptr(self.h[P - 1:]), ptr(m.norm), c.eps,
             ptr(d.logits), ptr(d.pmax), ptr(d.pidx), 1)
        call("q355_finish", ptr(d.pmax), ptr(d.pidx), d.nparts, ptr(d.tok), ptr(self.fin_pos), 1)
        d.pos.fill_(pos0 + P)

    def hidden_f64(self, P: int):
        import torch
        return self.h[:P].to(torch.float64) / FIX_SCALE
