"""Reference-order launches: Kern(spec).launch(grid, block, args) with the argument lists of the reference's kernels.

The reference's host step (scripts/qwen_fused.py:104-145) launches one generated kernel per operation, passing
raw device pointers in each kernel's own parameter order:

  EMBED / EMBED_F32          (E, tok, h, H)                                  lab/qwen_kernels.py:139-147, 284-290
  RMSNORM / RMSNORM_F32W_1P  (h, w, out, H, eps)                             :116-137, 683-705
  gemv_source(S, epi)        (W, S, X, Y, AUX, N, K)                         :14-113
  ATTN / ATTN2 / ATTN4       (qkv, cos, sin, pos, kc, vc, out, NH, NKV, scale[, prefetch args])  :149-220, 358-605
  FINISH / FINISH_MB         (logits, V, tok, pos[, partv, parti, cnt])      :222-282

The gfx950 library fuses neighbouring operations (RMSNorm into the consumer GEMV's prologue, RoPE and the K/V
write into the QKV epilogue, the attention merge into the O product's prologue, argmax partials into the head).
So the pointers a reference step passes are resolved to handles:

  Q4Mat (lab.qwen_model)  registered by its qs plane: W (and E for the tied embedding) resolve to the matrix
  NormedAct               the RMSNorm output `x`: RMSNORM records (h, w, eps); the consuming GEMV runs the
                          fused kernel (QKV, gate/up or the head) -- or, for a plain store/bias GEMV,
                          materialises Q8_1(x) first
  QKVOut                  the `qkv` buffer: gemv(bias) records (W, x, bias); ATTN runs q355_qkv_rope_kv
                          (RMSNorm + QKV + bias + RoPE + K/V write) then q355_attn_decode into an AttnOut
  AttnOut                 the `att` buffer: holds the attention partials; gemv(resid) on it runs
                          q355_attn_o_resid (merge + Q8_1 + O + residual)
  Logits                  the `logits` buffer: gemv(logits) runs q355_head_logits (its argmax partials);
                          FINISH runs q355_finish over them

Any other pointer is passed through unchanged (h int64 fixed point, tok/pos int32, the fp32 SwiGLU output m,
the RoPE tables, the paged caches). Every launch issues only library calls; nothing is computed on the host.
"""
from __future__ import annotations

import ctypes
import weakref

from .hip import HipError, call

_REG: "weakref.WeakValueDictionary[int, object]" = weakref.WeakValueDictionary()


def register(tensor, handle) -> None:
    """Make `tensor.data_ptr()` resolve to `handle` in reference-order launches."""
    _REG[tensor.data_ptr()] = handle


def resolve(a):
    """A launch argument -> the registered handle (by device pointer), or the plain value."""
    if hasattr(a, "data_ptr"):
        a = a.data_ptr()
    if isinstance(a, (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_double,
                      ctypes.c_void_p)):
        a = a.value
    if isinstance(a, int) and a in _REG:
        return _REG[a]
    return a


class NormedAct:
    """The reference's RMSNorm output buffer `x` [T, H] (bf16 there). Holds Q8_1 planes for a materialised copy."""

    def __init__(self, T: int, H: int, device="cuda"):
        import torch
        self.T, self.H = T, H
        self.xq = torch.zeros(T, H, dtype=torch.int8, device=device)
        self.xds = torch.zeros(T, H // 32, 2, dtype=torch.float16, device=device)
        self.src = None              # (h, w, eps) recorded by RMSNORM
        register(self.xq, self)

    def data_ptr(self):
        return self.xq.data_ptr()

    def norm(self):
        if self.src is None:
            raise HipError("RMSNorm output used before an RMSNORM launch wrote it")
        return self.src

    def materialise(self):
        h, w, eps = self.norm()
        call("q355_rmsnorm_fix_q8_1", h, w, self.xq.data_ptr(), self.xds.data_ptr(), self.T, self.H, eps)


class QKVOut:
    """The reference's `qkv` buffer. Holds the fp16 q the fused QKV epilogue writes; the paged cache's block table
    (one row of bt_stride pages per sequence) is given here because the reference's caches are contiguous."""

    def __init__(self, T: int, nh: int, hd: int, block_table, device="cuda"):
        import torch
        self.T, self.block_table = T, block_table
        self.bt_stride = block_table.shape[1]
        self.q = torch.zeros(T, nh * hd, dtype=torch.float16, device=device)
        self.pending = None          # (W, x, bias) recorded by gemv(bias)
        register(self.q, self)

    def data_ptr(self):
        return self.q.data_ptr()


class AttnOut:
    """The reference's attention output `att`: here the split-K partials f64 [T][nh][max_chunks][130]."""

    def __init__(self, T: int, nh: int, hd: int, max_chunks: int, device="cuda"):
        import torch
        self.T, self.nh, self.max_chunks = T, nh, max_chunks
        self.part = torch.zeros(T, nh, max_chunks, hd + 2, dtype=torch.float64, device=device)
        self.pos = None
        register(self.part, self)

    def data_ptr(self):
        return self.part.data_ptr()


class Logits:
    """The reference's `logits` [T, V] plus the head's per-workgroup argmax partials."""

    def __init__(self, T: int, V: int, device="cuda"):
        import torch
        self.T, self.V = T, V
        self.nparts = call("q355_head_nparts", V)
        self.logits = torch.zeros(T, V, dtype=torch.float32, device=device)
        self.pmax = torch.zeros(T, self.nparts, dtype=torch.float32, device=device)
        self.pidx = torch.zeros(T, self.nparts, dtype=torch.int32, device=device)
        register(self.logits, self)

    def data_ptr(self):
        return self.logits.data_ptr()


def _need(obj, cls, what):
    if not isinstance(obj, cls):
        raise HipError(f"{what}: expected a {cls.__name__} buffer, got {type(obj).__name__}")
    return obj


def _mat(W, what):
    from .qwen_model import Q4Mat
    return _need(W, Q4Mat, f"{what} weights")


def launch_embed(spec, args):
    E, tok, h, H = (resolve(a) for a in args[:4])
    e = _mat(E, "EMBED")
    T = spec.params.get("T", 1)
    return call("q355_embed_q4_0", e.qs.data_ptr(), e.d.data_ptr(), e.N, int(H), tok, h, T)


def launch_rmsnorm(spec, args):
    h, w, out, H, eps = (resolve(a) for a in args[:5])
    x = _need(out, NormedAct, "RMSNORM out")
    if int(H) != x.H:
        raise HipError(f"RMSNORM: H={H} but the output buffer holds {x.H}")
    x.src = (h, w, float(eps))       # runs inside the consumer's prologue
    return 0


def launch_gemv(spec, args):
    W, S, X, Y, AUX, N, K = (resolve(a) for a in args[:7])
    epi = spec.params.get("epi_name", "store")
    m = _mat(W, "gemv")
    N, K = int(N), int(K)
    if (m.N, m.K) != (N, K):
        raise HipError(f"gemv: N={N} K={K} but the matrix is {m.N} x {m.K}")
    if isinstance(Y, QKVOut):                                   # qkv: fused with RoPE + K/V write at ATTN
        Y.pending = (m, _need(X, NormedAct, "gemv(qkv) X"), AUX)
        return 0
    if isinstance(X, AttnOut):                                  # o: merge + Q8_1 + O + residual
        if epi != "resid":
            raise HipError(f"gemv on attention output: epilogue {epi!r} (only resid)")
        return call("q355_attn_o_resid", m.qs.data_ptr(), m.d.data_ptr(), N, X.part.data_ptr(), X.max_chunks,
                    X.pos, X.nh, Y, X.T)
    if epi == "swiglu":                                         # gate/up: RMSNorm prologue + SwiGLU
        h, w, eps = _need(X, NormedAct, "gemv(swiglu) X").norm()
        return call("q355_ffn_gate_up", m.qs.data_ptr(), m.d.data_ptr(), N, K, h, w, eps, Y, X.T)
    if epi == "logits" and isinstance(Y, Logits):               # head: RMSNorm prologue + argmax partials
        h, w, eps = _need(X, NormedAct, "gemv(logits) X").norm()
        return call("q355_head_logits", m.qs.data_ptr(), m.d.data_ptr(), N, K, h, w, eps, Y.logits.data_ptr(),
                    Y.pmax.data_ptr(), Y.pidx.data_ptr(), Y.T)
    if epi == "resid" and not isinstance(X, NormedAct):         # down: Q8_1 of the fp32 SwiGLU output + residual
        T = spec.params.get("T", 1)
        return call("q355_ffn_down", m.qs.data_ptr(), m.d.data_ptr(), N, K, X, Y, T)
    # plain store / bias / accumulate over a materialised Q8_1 activation
    x = _need(X, NormedAct, "gemv X")
    x.materialise()
    code = {"store": 0, "logits": 0, "resid": 1, "bias": 2, "biasf": 2}[epi]
    return call("q355_gemv_q4_0_q8_1", m.qs.data_ptr(), m.d.data_ptr(), N, K, x.xq.data_ptr(), x.xds.data_ptr(),
                x.T, Y.logits.data_ptr() if isinstance(Y, Logits) else Y, AUX if code == 2 else None, code)


def launch_attn(spec, args):
    qkv, cos, sin, pos, kc, vc, out, NH, NKV, scale = (resolve(a) for a in args[:10])
    q = _need(qkv, QKVOut, "ATTN qkv")
    att = _need(out, AttnOut, "ATTN out")
    if q.pending is None:
        raise HipError("ATTN before the QKV gemv")
    m, x, bias = q.pending
    h, w, eps = x.norm()
    call("q355_qkv_rope_kv", m.qs.data_ptr(), m.d.data_ptr(), m.K, h, w, eps, bias, cos, sin, pos,
         q.block_table.data_ptr(), q.bt_stride, 1, kc, vc, q.q.data_ptr(), int(NH), int(NKV), q.T)
    att.pos = pos
    return call("q355_attn_decode", q.q.data_ptr(), kc, vc, pos, q.block_table.data_ptr(), q.bt_stride, int(NH),
                int(NKV), att.max_chunks, float(scale), att.part.data_ptr(), None, None, None, q.T, 0)


def launch_finish(spec, args):
    logits, V, tok, pos = (resolve(a) for a in args[:4])
    lg = _need(logits, Logits, "FINISH logits")
    return call("q355_finish", lg.pmax.data_ptr(), lg.pidx.data_ptr(), lg.nparts, tok, pos, lg.T)


LAUNCHERS = {"embed": launch_embed, "rmsnorm": launch_rmsnorm, "gemv": launch_gemv, "attn": launch_attn,
             "finish": launch_finish}
