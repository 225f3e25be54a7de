"""Persistent whole-step decode (the reference's lab/qwen_mega.py entry points).

The reference's megakernel (mega_source, lab/qwen_mega.py:43-361) streams every layer's weights through
one persistent CUDA kernel per token with a software grid barrier; its own log records it as incorrect
(token 1 vs 89141, data/oct15_tiles_mega/megakernel_pos128.log). Here `mega_source` names the gfx950
persistent step q355_mega_decode: one launch per token (plus head and argmax launches for a Q6_K output matrix),
256 workgroups (one per CU), every phase's weight
loads issued before the phase waits for its inputs, dataflow flags between dependent phases and two full
barriers per layer; f64 arithmetic of the batch-1 GEMV path (same oracle, same tokens).
"""
from __future__ import annotations

import ctypes

from .hip import HipError, call, ptr
from .qwen_kernels import KernelSpec
from .qwen_model import Decoder, DeviceModel

_LAYER_FIELDS = ("qkv_qs", "qkv_d", "qkv_b", "ln1", "o_qs", "o_d", "ln2", "gu_qs", "gu_d", "down_qs", "down_d",
                 "kc", "vc")


class MegaLayer(ctypes.Structure):
    """Per-layer pointer table read by the persistent kernel (layout of MegaLayer in csrc/mega.hip)."""
    _fields_ = [(f, ctypes.c_void_p) for f in _LAYER_FIELDS]


def mega_source(nl: int = 28, maxlen: int = 2048, nw: int = 256, ch: int = 0, nch: int = 0, cap: int = 0) -> KernelSpec:
    """Persistent decode megakernel (lab/qwen_mega.py:43-361) -> q355_mega_decode. nw (workgroups) is fixed
    at 256 on gfx950 (one per CU); ch / nch / cap (the reference's stream chunking and capacity) have no
    counterpart: each phase's weights are addressed directly in the tiled Q4_0 planes."""
    if nw != 256:
        raise ValueError("the gfx950 persistent step runs exactly 256 workgroups (one per CU)")
    return KernelSpec("q355_mega_decode", {"L": nl, "maxlen": maxlen})


class MegaDecoder(Decoder):
    """Batch-1 decoder whose step() is one persistent-kernel launch (embed, 28 layers, head, argmax, pos += 1).
    Same buffers and interface as Decoder (prefill_tokens, capture, generate)."""

    SPIN_LIMIT_US = 200_000      # bounded waits: a stuck launch ends with the error word set

    def __init__(self, m: DeviceModel, max_ctx: int | None = None):
        import torch
        super().__init__(m, T=1, max_ctx=max_ctx)
        assert call("q355_mega_layer_bytes") == ctypes.sizeof(MegaLayer)
        # the kernel accepts any pos < max_chunks * 64: the RoPE tables must cover all of them
        assert m.maxlen >= self.max_chunks * 64, "DeviceModel maxlen must cover max_ctx rounded up to 64"
        c = m.cfg
        table = (MegaLayer * c.L)()
        for i, L in enumerate(m.layers):
            table[i] = MegaLayer(L["qkv"].qs.data_ptr(), L["qkv"].d.data_ptr(), L["qkv_b"].data_ptr(),
                                 L["ln1"].data_ptr(), L["o"].qs.data_ptr(), L["o"].d.data_ptr(), L["ln2"].data_ptr(),
                                 L["gu"].qs.data_ptr(), L["gu"].d.data_ptr(), L["down"].qs.data_ptr(),
                                 L["down"].d.data_ptr(), self.kc[i].data_ptr(), self.vc[i].data_ptr())
        raw = bytes(table)
        self.layer_table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(m.device)
        nbytes = call("q355_mega_ws_bytes", self.max_chunks, c.L)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=m.device)

    def step(self):
        m, c = self.m, self.cfg
        e = m.embed
        q6 = m.head_q6k
        # a Q6_K output matrix (llama.cpp's output.weight): the persistent launch stops after the layers and the
        # head + argmax run as two more launches
        call("q355_mega_decode", ptr(self.layer_table), c.L, ptr(e.qs), ptr(e.d), ptr(m.norm), c.V, ptr(m.cos),
             ptr(m.sin), ptr(self.block_table), self.max_chunks, c.eps, ptr(self.tok), ptr(self.pos), ptr(self.h),
             None if q6 is not None else ptr(self.logits), ptr(self.ws), self.SPIN_LIMIT_US)
        if q6 is not None:
            call("q355_head_logits_q6k", ptr(q6.lo), ptr(q6.hi), ptr(q6.sc), ptr(q6.d), q6.N, q6.K, ptr(self.h),
                 ptr(m.norm), c.eps, ptr(self.logits), ptr(self.pmax), ptr(self.pidx), 1)
            call("q355_finish", ptr(self.pmax), ptr(self.pidx), self.nparts, ptr(self.tok), ptr(self.pos), 1)
        import torch
        if not torch.cuda.is_current_stream_capturing():
            self.check()

    def check(self):
        """Raise HipError if the kernel's error word is set (a bounded wait expired, or a bad pos/tok): the tokens
        of that launch and every later one are invalid. Synchronises with the device."""
        e = self.error()
        if e:
            raise HipError(f"q355_mega_decode: error word {e:#x} (bounded wait expired or invalid pos/tok)")

    def generate(self, n: int, use_graph: bool = True):
        out = super().generate(n, use_graph)
        self.check()
        return out

    def error(self) -> int:
        """The kernel's error word (non-zero after a bounded wait expired or a bad pos/tok)."""
        import torch
        off = 256 * 16 * 4 + 32 * 16 * 4 + 16 * 4
        return int(self.ws[off:off + 4].view(torch.int32).item())
