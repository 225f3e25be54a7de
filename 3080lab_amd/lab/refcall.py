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

The batched step (scripts/qwen_batched_decode.py:106-187: batchify'd EMBED_F32 / RMSNORM_F32W_1P / ATTN4 launched
over grid.y = B, gemv_v2_source GEMVs with (W, S, X, Y, aux, N, K, ws, cnt), head_v2_source with (*head, x,
logits, V, H)) runs the fp16 batched arithmetic of BatchedDecoder(act="f16") -- the reference's own gemv_v2
arithmetic -- over these handles:

  BatchAct                the batched `x` [B, H]: RMSNORM records (h, w, eps); a gemv_v2 consumer gets its fp16
                          form (q355_rmsnorm_fix_f16), the head its Q8_1 form (q355_rmsnorm_fix_q8_1)
  BatchQKV                the batched `qkv`: gemv_v2(biasf) records (W, x, bias); ATTN runs
                          q355_gemm_f16_qkv_rope then the batched attention into a BatchAttn
  BatchAttn               the batched `att`: the attention's split partials and fp16 output; gemv_v2(resid) on
                          it runs the O product (with the split merge in its staging up to 16 tokens)
  Logits                  head_v2 writes the fp32 logits (the reference takes the argmax with torch) and the
                          per-workgroup argmax partials

tok and pos are read as int32: the reference's torch.long tok/pos must be allocated as torch.int32 (a tensor of
another dtype passed to a launch is rejected with HipError; a bare data_ptr() integer cannot be checked).
Any other pointer is passed through unchanged (h int64 fixed point, the fp32 or fp16 SwiGLU output, the RoPE
tables, the paged caches). Every launch issues only library calls; nothing is computed on the host.
"""
from __future__ import annotations

import ctypes
import weakref

from .hip import HipError, call

_REG: "weakref.WeakValueDictionary[int, object]" = weakref.WeakValueDictionary()


def register(tensor, handle) -> None:
    """Make `tensor.data_ptr()` resolve to `handle` in reference-order launches."""
    _REG[tensor.data_ptr()] = handle


def int32_arg(a, what):
    """A tok/pos launch argument: a tensor must be int32 (the kernels read int32); returns the pointer."""
    dt = getattr(a, "dtype", None)
    if dt is not None:
        import torch
        if dt != torch.int32:
            raise HipError(f"{what}: {dt} buffer; the library reads int32 tok/pos (allocate them as torch.int32)")
    return resolve(a)


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
    """The reference's `logits` [T, V] plus the head's per-workgroup argmax partials (batched: the MFMA head's)."""

    def __init__(self, T: int, V: int, device="cuda", batched: bool = False):
        import torch
        self.T, self.V = T, V
        self.nparts = call("q355_mmq_nparts" if batched else "q355_head_nparts", V)
        self.logits = torch.zeros(T, V, dtype=torch.float32, device=device)
        self.pmax = torch.zeros(T, self.nparts, dtype=torch.float32, device=device)
        self.pidx = torch.zeros(T, self.nparts, dtype=torch.int32, device=device)
        register(self.logits, self)

    def data_ptr(self):
        return self.logits.data_ptr()


def _need(obj, cls, what):
    if not isinstance(obj, cls):
        names = " or ".join(c.__name__ for c in (cls if isinstance(cls, tuple) else (cls,)))
        raise HipError(f"{what}: expected a {names} buffer, got {type(obj).__name__}")
    return obj


def _mat(W, what):
    from .qwen_model import Q4Mat
    return _need(W, Q4Mat, f"{what} weights")


def launch_embed(spec, args, grid=None):
    E, h, H = resolve(args[0]), resolve(args[2]), resolve(args[3])
    tok = int32_arg(args[1], "EMBED tok")
    e = _mat(E, "EMBED")
    T = _grid_y(grid) if spec.params.get("batched") else spec.params.get("T", 1)
    return call("q355_embed_q4_0", e.qs.data_ptr(), e.d.data_ptr(), e.N, int(H), tok, h, T)


def _grid_y(grid):
    return grid[1] if isinstance(grid, (tuple, list)) and len(grid) > 1 else 1


def launch_rmsnorm(spec, args, grid=None):
    h, w, out, H, eps = (resolve(a) for a in args[:5])
    x = _need(out, (NormedAct, BatchAct), "RMSNORM out")
    if int(H) != x.H:
        raise HipError(f"RMSNORM: H={H} but the output buffer holds {x.H}")
    x.src = (h, w, float(eps))       # runs inside the consumer's prologue
    return 0


def launch_gemv(spec, args, grid=None):
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
        if not isinstance(X, int) or not isinstance(Y, int):
            raise HipError("gemv(resid) down: X (fp32 SwiGLU output) and Y (int64 residual) must be plain buffers")
        # plain pointers carry no row count: the reference's fused step (scripts/qwen_fused.py) is batch 1
        if spec.params.get("T", 1) != 1:
            raise HipError("gemv(resid) down over plain buffers: batch 1 only (the buffers carry no row count)")
        return call("q355_ffn_down", m.qs.data_ptr(), m.d.data_ptr(), N, K, X, Y, 1)
    # plain store / bias / accumulate over a materialised Q8_1 activation (fp32 Y)
    x = _need(X, NormedAct, "gemv X")
    if not isinstance(Y, (int, Logits)):
        raise HipError(f"gemv({epi}): Y must be an fp32 buffer, got {type(Y).__name__}")
    x.materialise()
    code = {"store": 0, "logits": 0, "resid": 1, "bias": 2, "biasf": 2}[epi]
    return call("q355_gemv_q4_0_q8_1", m.qs.data_ptr(), m.d.data_ptr(), N, K, x.xq.data_ptr(), x.xds.data_ptr(),
                x.T, Y.logits.data_ptr() if isinstance(Y, Logits) else Y, AUX if code == 2 else None, code)


def launch_attn(spec, args, grid=None):
    qkv, cos, sin, kc, vc, out, NH, NKV, scale = (resolve(a) for a in (args[:3] + args[4:10]))
    pos = int32_arg(args[3], "ATTN pos")
    if isinstance(qkv, BatchQKV):
        return _attn_batched(qkv, cos, sin, pos, kc, vc, out, int(NH), int(NKV), float(scale))
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


def launch_finish(spec, args, grid=None):
    logits, V = resolve(args[0]), resolve(args[1])
    tok, pos = int32_arg(args[2], "FINISH tok"), int32_arg(args[3], "FINISH pos")
    lg = _need(logits, Logits, "FINISH logits")
    return call("q355_finish", lg.pmax.data_ptr(), lg.pidx.data_ptr(), lg.nparts, tok, pos, lg.T)


# ------------------------------------------------------------------------------------------------------------
# the batched step (fp16 batched arithmetic)

class BatchAct:
    """The batched `x` [B, H] (bf16 in the reference): its fp16 form for the layer products and Q8_1 planes for
    the LM head, both written from the recorded RMSNorm source when a consumer needs them."""

    def __init__(self, B: int, H: int, device="cuda"):
        import torch
        self.T, self.H = B, H
        self.xh = torch.zeros(B, H, dtype=torch.float16, device=device)
        self.xq = torch.zeros(B, H, dtype=torch.int8, device=device)
        self.xds = torch.zeros(B, H // 32, 2, dtype=torch.float16, device=device)
        self.src = None
        register(self.xh, self)

    def data_ptr(self):
        return self.xh.data_ptr()

    def norm(self):
        if self.src is None:
            raise HipError("RMSNorm output used before an RMSNORM launch wrote it")
        return self.src

    def f16(self) -> int:
        h, w, eps = self.norm()
        call("q355_rmsnorm_fix_f16", h, w, self.xh.data_ptr(), self.T, self.H, eps)
        return self.xh.data_ptr()

    def q8(self):
        h, w, eps = self.norm()
        call("q355_rmsnorm_fix_q8_1", h, w, self.xq.data_ptr(), self.xds.data_ptr(), self.T, self.H, eps)


class BatchQKV:
    """The batched `qkv` [B, (nh + 2 nkv) hd]: the fp16 q the fused QKV epilogue writes; the paged cache's block
    table (one row per sequence) is given here (the reference's caches are contiguous per sequence)."""

    def __init__(self, B: int, nh: int, hd: int, block_table, device="cuda"):
        import torch
        self.T, self.block_table = B, block_table
        self.bt_stride = block_table.shape[1]
        self.q = torch.zeros(B, nh * hd, dtype=torch.float16, device=device)
        self.pending = None
        register(self.q, self)

    def data_ptr(self):
        return self.q.data_ptr()


class BatchAttn:
    """The batched `att` [B, nh hd]: split partials f64 [B][nh][max_chunks][130] and the fp16 output (tokens the
    attention finished itself, or all tokens when the merge runs in its own launch)."""

    def __init__(self, B: int, nh: int, nkv: int, hd: int, max_chunks: int, device="cuda"):
        import torch
        self.T, self.nh, self.nkv, self.max_chunks = B, nh, nkv, max_chunks
        self.part = torch.zeros(B, nh, max_chunks, hd + 2, dtype=torch.float64, device=device)
        self.oh = torch.zeros(B, nh * hd, dtype=torch.float16, device=device)
        self.pos, self.merged = None, True
        register(self.oh, self)

    def data_ptr(self):
        return self.oh.data_ptr()


def _attn_batched(q, cos, sin, pos, kc, vc, out, NH, NKV, scale):
    from .qwen_batched import MERGE_IN_O_MAX_B
    att = _need(out, BatchAttn, "ATTN out")
    if q.pending is None:
        raise HipError("ATTN before the QKV gemv")
    m, x, bias = q.pending
    B = q.T
    bt = q.block_table.data_ptr()
    call("q355_gemm_f16_qkv_rope", m.qs.data_ptr(), m.d.data_ptr(), m.N, m.K, x.f16(), B, bias, cos, sin, pos, bt,
         q.bt_stride, 1, kc, vc, q.q.data_ptr(), NH, NKV)
    att.pos, att.merged = pos, B > MERGE_IN_O_MAX_B
    name = "q355_attn_decode_f16" if att.merged else "q355_attn_decode_partials_f16"
    return call(name, q.q.data_ptr(), kc, vc, pos, bt, q.bt_stride, NH, NKV, att.max_chunks, scale,
                att.part.data_ptr(), att.oh.data_ptr(), B)


def launch_gemv_v2(spec, args, grid=None):
    """gemv_v2_source's (W, S, X, Y, aux, N, K, ws, cnt): the fp16-weight product of the epilogue's entry point
    (ws and cnt, the reference's split-K scratch, are not needed: every entry point finishes in-kernel)."""
    W, S, X, Y, AUX, N, K = (resolve(a) for a in args[:7])
    epi = spec.params["epi_name"]
    B = spec.params["B"]
    m = _mat(W, "gemv_v2")
    N, K = int(N), int(K)
    if (m.N, m.K) != (N, K):
        raise HipError(f"gemv_v2: N={N} K={K} but the matrix is {m.N} x {m.K}")
    if epi == "biasf":                                          # qkv: bias, RoPE and the K/V write at ATTN
        _need(Y, BatchQKV, "gemv_v2(biasf) Y").pending = (m, _need(X, BatchAct, "gemv_v2(qkv) X"), AUX)
        return 0
    if isinstance(X, BatchAttn):                                # o: (merge +) fp16 product + residual
        if epi != "resid":
            raise HipError(f"gemv_v2 on attention output: epilogue {epi!r} (only resid)")
        if not isinstance(Y, int):
            raise HipError("gemv_v2(o): Y must be the int64 residual buffer")
        if X.merged:
            return call("q355_gemm_q4_0_f16", m.qs.data_ptr(), m.d.data_ptr(), N, K, X.oh.data_ptr(), B, 6, None, Y,
                        None, None, None)
        return call("q355_gemm_f16_attn_o_resid", m.qs.data_ptr(), m.d.data_ptr(), N, X.part.data_ptr(),
                    X.max_chunks, X.pos, X.nh, X.nkv, X.oh.data_ptr(), Y, B)
    if epi == "swiglu":                                         # gate/up -> fp16 SwiGLU
        return call("q355_gemm_q4_0_f16", m.qs.data_ptr(), m.d.data_ptr(), N, K,
                    _need(X, BatchAct, "gemv_v2(swiglu) X").f16(), B, 8, None, None, Y, None, None)
    if epi == "resid":                                          # down: fp16 SwiGLU output -> residual
        if not isinstance(X, int) or not isinstance(Y, int):
            raise HipError("gemv_v2(resid): X (fp16 activations) and Y (int64 residual) must be plain buffers")
        return call("q355_gemm_q4_0_f16", m.qs.data_ptr(), m.d.data_ptr(), N, K, X, B, 6, None, Y, None, None, None)
    raise HipError(f"gemv_v2: epilogue {epi!r} (biasf, resid, swiglu)")


def launch_head_v2(spec, args, grid=None):
    """head_v2_source's (*head, x, logits, V, H): the head's weights as pack_q6_mma returns them (here: the
    tied Q4_0 matrix, or the Q6_K planes of llama.cpp's output.weight), on the final RMSNorm's Q8_1."""
    from .qwen_model import Q6KMat
    *wts, X, Y, V, H = (resolve(a) for a in args)
    x = _need(X, BatchAct, "head_v2 x")
    lg = _need(Y, Logits, "head_v2 logits")
    V, H, B = int(V), int(H), x.T
    x.q8()
    w = wts[0]
    if isinstance(w, Q6KMat):
        for j in range(0, B, 32):
            n = min(32, B - j)
            call("q355_mmq_q6k_logits", w.lo.data_ptr(), w.hi.data_ptr(), w.sc.data_ptr(), w.d.data_ptr(), V, H,
                 x.xq.data_ptr() + j * H, x.xds.data_ptr() + j * (H // 32) * 4, n, lg.logits[j].data_ptr(),
                 lg.pmax[j].data_ptr(), lg.pidx[j].data_ptr())
        return 0
    e = _mat(w, "head_v2")
    return call("q355_mmq_q4_0_q8_1", e.qs.data_ptr(), e.d.data_ptr(), V, H, x.xq.data_ptr(), x.xds.data_ptr(), B,
                5, lg.logits.data_ptr(), None, None, None, lg.pmax.data_ptr(), lg.pidx.data_ptr())


LAUNCHERS = {"embed": launch_embed, "rmsnorm": launch_rmsnorm, "gemv": launch_gemv, "attn": launch_attn,
             "finish": launch_finish, "gemv_v2": launch_gemv_v2, "head_v2": launch_head_v2}
