"""GGUF reader, ggml block decoders and the device repack of Q4_0 (numpy).

Same API and block semantics as the reference's lab/gguf.py (GGUF, q4_0_blocks, q6_k_blocks,
q6_k_parts; lab/gguf.py:1-123):
  Q4_0 block, 18 B: fp16 d + 16 B qs; weight i = (qs[i] & 15) - 8, weight i+16 = (qs[i] >> 4) - 8.
  Q6_K block, 210 B: ql[128], qh[64], int8 scales[16], fp16 d.
Added for this build:
  quantize_q4_0   the BASELINE Q4_0 rule (llama.cpp quantize_row_q4_0_ref semantics) -> GGUF bytes
  tile_q4_0       GGUF Q4_0 bytes of W [N, K] -> the library's 16-row tiled planes (qs, d)
  permute_rows_rope / interleave_rows   the QKV and gate/up row orders the fused epilogues expect
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

# ------------------------------------------------------------------------------------------------
# GGUF container (format as published with ggml: little-endian header "GGUF", u32 version, u64 tensor
# count, u64 key/value count; key/value pairs; tensor infos; padding to general.alignment; tensor data).
# The whole file is memory-mapped once and parsed with a byte cursor.

# tensor element types this build decodes: type id -> (element count per block, bytes per block)
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 14: (256, 210)}
_TYPE_NAME = {0: "F32", 1: "F16", 2: "Q4_0", 14: "Q6_K"}
# metadata value types with a fixed width: id -> numpy dtype
_META_SCALAR = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
                6: np.float32, 7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}
_META_STRING, _META_ARRAY = 8, 9


@dataclass
class Tensor:
    """One entry of the tensor directory. dims are in GGUF order: dims[0] varies fastest (the K axis of a
    row-major [N, K] matrix); offset is relative to the start of the data section."""
    name: str
    dims: tuple
    type: int
    offset: int


class _Cursor:
    """Sequential little-endian decoding over a uint8 buffer."""

    def __init__(self, buf: np.ndarray):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> np.ndarray:
        if self.pos + n > self.buf.size:
            raise ValueError("GGUF: truncated file")
        out = self.buf[self.pos:self.pos + n]
        self.pos += n
        return out

    def scalar(self, dtype):
        dt = np.dtype(dtype).newbyteorder("<")
        v = self.take(dt.itemsize).view(dt)[0]
        return v.item()

    def u32(self) -> int:
        return self.scalar(np.uint32)

    def u64(self) -> int:
        return self.scalar(np.uint64)

    def text(self) -> str:
        return bytes(self.take(self.u64())).decode("utf-8", "replace")

    def meta_value(self, kind: int):
        if kind == _META_STRING:
            return self.text()
        if kind == _META_ARRAY:
            elem, count = self.u32(), self.u64()
            if elem in _META_SCALAR:                # fixed-width arrays decode in one step
                dt = np.dtype(_META_SCALAR[elem]).newbyteorder("<")
                return self.take(count * dt.itemsize).view(dt).tolist()
            return [self.meta_value(elem) for _ in range(count)]
        if kind not in _META_SCALAR:
            raise ValueError(f"GGUF: unknown metadata value type {kind}")
        return self.scalar(_META_SCALAR[kind])


class GGUF:
    """A GGUF (v2/v3) file: `meta` (key -> value), `tensors` (name -> Tensor), tensor bytes by `raw`."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        cur = _Cursor(self.mm)
        if bytes(cur.take(4)) != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        self.version = cur.u32()
        n_tensors, n_meta = cur.u64(), cur.u64()
        self.meta = {}
        for _ in range(n_meta):
            key = cur.text()
            self.meta[key] = cur.meta_value(cur.u32())
        self.tensors = {}
        for _ in range(n_tensors):
            name = cur.text()
            dims = tuple(cur.u64() for _ in range(cur.u32()))
            kind, offset = cur.u32(), cur.u64()
            self.tensors[name] = Tensor(name, dims, kind, offset)
        align = int(self.meta.get("general.alignment", 32))
        self.data_start = (cur.pos + align - 1) // align * align

    def raw(self, name: str):
        """-> (uint8 bytes of the tensor, Tensor)."""
        t = self.tensors[name]
        if t.type not in _BLOCK:
            raise NotImplementedError(f"{name}: ggml type {t.type}")
        per, nbytes = _BLOCK[t.type]
        count = 1
        for d in t.dims:
            count *= d
        begin = self.data_start + t.offset
        return np.asarray(self.mm[begin:begin + count // per * nbytes]), t

    def f32(self, name: str) -> np.ndarray:
        """The tensor decoded to float32, shaped row-major (reverse of the GGUF dims)."""
        b, t = self.raw(name)
        return _DECODE[_TYPE_NAME[t.type]](b).reshape(t.dims[::-1])


def _decode_q4_0(b):
    d, q = q4_0_blocks(b)
    return (q.astype(np.float32) - 8) * d[:, None]


def _decode_q6_k(b):
    q, s = q6_k_blocks(b)
    return q.reshape(-1, 16, 16).astype(np.float32) * s[:, :, None]


_DECODE = {"F32": lambda b: b.view(np.float32), "F16": lambda b: b.view(np.float16).astype(np.float32),
           "Q4_0": _decode_q4_0, "Q6_K": _decode_q6_k}


def q4_0_blocks(b: np.ndarray):
    """-> d float32 [nblk], q uint8 [nblk, 32] in weight order (low nibbles 0..15, high nibbles 16..31)."""
    blk = np.asarray(b, np.uint8).reshape(-1, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    lo, hi = blk[:, 2:] & 15, blk[:, 2:] >> 4
    return d, np.concatenate([lo, hi], axis=1)


def q6_k_blocks(b: np.ndarray):
    """Q6_K super-blocks (210 bytes each) decoded: the 256 signed 6-bit values of every block, and one float32
    factor per 16 of them, the super-block scale times that group's int8 scale."""
    q, sc, d = _q6_k_fields(b)
    return q, d.astype(np.float32)[:, None] * sc.astype(np.float32)


def q6_k_parts(b: np.ndarray):
    """The same values, with the scales left as stored: 16 int8 group scales and the fp16 super-block scale."""
    return _q6_k_fields(b)


def _q6_k_fields(b: np.ndarray):
    blk = np.asarray(b, np.uint8).reshape(-1, 210)
    ql = blk[:, :128].astype(np.int16)
    qh = blk[:, 128:192].astype(np.int16)
    sc = blk[:, 192:208].copy().view(np.int8)
    d = blk[:, 208:210].copy().view(np.float16).reshape(-1)
    q = np.empty((blk.shape[0], 256), np.int16)
    # each 128-weight half: 64 ql bytes (low nibbles then high nibbles) and 32 qh bytes (four 2-bit fields)
    for half in range(2):
        L = ql[:, 64 * half:64 * half + 64]
        Hh = qh[:, 32 * half:32 * half + 32]
        base = 128 * half
        for quarter in range(4):
            low = (L[:, :32] if quarter % 2 == 0 else L[:, 32:])
            low = low & 15 if quarter < 2 else low >> 4
            high = (Hh >> (2 * quarter)) & 3
            q[:, base + 32 * quarter: base + 32 * quarter + 32] = (low | (high << 4)) - 32
    return q.astype(np.int8), sc, d


# ------------------------------------------------------------------------------------------------
# Q4_0 quantizer (BASELINE rule) and the device repack


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """fp32 [..., K] (K % 32 == 0) -> GGUF Q4_0 bytes uint8 [n_blocks, 18].
    Per 32-block: m = signed value of max |x| (first on ties), d = m / -8 (fp32, stored fp16),
    q = clamp(round(x / d) + 8, 0, 15) rounding halves away from zero; q = 8 if d == 0.
    All in float32: rint is exact, and a half is detected exactly as |r - trunc(r)| == 0.5."""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    n = xb.shape[0]
    d = xb[np.arange(n), np.abs(xb).argmax(axis=1)] / np.float32(-8.0)
    zero = d == 0
    r = xb / np.where(zero, np.float32(1.0), d)[:, None]
    t = np.trunc(r)
    q = np.where(np.abs(r - t) == np.float32(0.5), t + np.sign(r), np.rint(r))
    q += 8
    np.clip(q, 0, 15, out=q)
    q[zero] = 8
    q = q.astype(np.uint8)
    out = np.empty((n, 18), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out


def tile_q4_0(b: np.ndarray, N: int, K: int):
    """GGUF Q4_0 bytes of W [N, K] -> (qs uint8 [N/16, K/32, 16, 16], d fp16 [N/16, K/32, 16]).
    Row n, block j lands at qs[n // 16, j, n % 16] (bytes unchanged), d[n // 16, j, n % 16]."""
    assert N % 16 == 0 and K % 32 == 0
    blk = np.asarray(b, np.uint8).reshape(N // 16, 16, K // 32, 18)
    qs = np.ascontiguousarray(blk[..., 2:].transpose(0, 2, 1, 3))
    d = np.ascontiguousarray(blk[..., :2].transpose(0, 2, 1, 3)).view(np.float16).reshape(N // 16, K // 32, 16)
    return qs, d


def untile_q4_0(qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Inverse of tile_q4_0 -> GGUF bytes [N*K/32, 18]."""
    nt, nb = qs.shape[:2]
    out = np.empty((nt, 16, nb, 18), np.uint8)
    out[..., 2:] = qs.transpose(0, 2, 1, 3)
    out[..., :2] = np.ascontiguousarray(d.transpose(0, 2, 1)).view(np.uint8).reshape(nt, 16, nb, 2)
    return out.reshape(-1, 18)


def tile_q6_k(b: np.ndarray, N: int, K: int):
    """GGUF Q6_K bytes of W [N, K] (K % 256 == 0) -> the library's Q6_K planes, 6.5625 bits per weight as
    in the file (weights in natural order, v = q + 32 in 0..63):
      lo uint8 [N/16, K/32, 16, 16]: byte i = (v_i & 15) | (v_{i+16} & 15) << 4 of each 32-weight block
      hi uint8 [N/16, K/32, 16, 8]:  byte b = sum_j (v_{b+8j} >> 4) << 2j, j = 0..3
      sc int8  [N/16, K/32, 16, 2]:  the two 16-weight sub-block scales of the block
      d  fp16  [N/16, K/256, 16]:    the super-block scale
    so weight i of a block is d * sc[i // 16] * (v_i - 32)."""
    assert N % 16 == 0 and K % 256 == 0
    q, sc, d = q6_k_parts(b)
    v = (q.astype(np.int16) + 32).astype(np.uint8).reshape(N, K // 32, 32)
    lo = (v[..., :16] & 15) | ((v[..., 16:] & 15) << 4)
    hv = v >> 4
    hi = hv[..., 0:8] | (hv[..., 8:16] << 2) | (hv[..., 16:24] << 4) | (hv[..., 24:32] << 6)
    sc2 = sc.reshape(N, K // 32, 2)
    dd = d.reshape(N, K // 256)
    t = lambda a: np.ascontiguousarray(a.reshape(N // 16, 16, *a.shape[1:]).swapaxes(1, 2))  # noqa: E731
    return t(lo.astype(np.uint8)), t(hi.astype(np.uint8)), t(sc2), t(dd)


def rope_row_order(n_heads: int, hd: int = 128) -> np.ndarray:
    """Row permutation that interleaves the RoPE pairs of every head: new row 2i <- dim i,
    new row 2i+1 <- dim i + hd/2 (so one 16-row tile holds 8 complete pairs)."""
    half = hd // 2
    within = np.stack([np.arange(half), np.arange(half) + half], 1).reshape(-1)
    return (np.arange(n_heads)[:, None] * hd + within[None]).reshape(-1)


def qkv_row_order(nh: int, nkv: int, hd: int = 128) -> np.ndarray:
    """Device row order of the concatenated [q; k; v] projection: q and k heads pair-interleaved, v as is
    (reference concat: scripts/qwen_gguf.py:77-78, 82)."""
    q = rope_row_order(nh, hd)
    k = nh * hd + rope_row_order(nkv, hd)
    v = (nh + nkv) * hd + np.arange(nkv * hd)
    return np.concatenate([q, k, v])


def gate_up_row_order(ffn: int) -> np.ndarray:
    """Rows g0, u0, g1, u1, ... of [gate; up] (reference interleave: scripts/qwen_gguf.py:79-81)."""
    return np.stack([np.arange(ffn), ffn + np.arange(ffn)], 1).reshape(-1)


def take_rows_q4_0(b: np.ndarray, K: int, order: np.ndarray) -> np.ndarray:
    """Reorder the rows of a GGUF Q4_0 matrix (bytes [N*K/32, 18]) -> bytes in `order`."""
    rows = np.asarray(b, np.uint8).reshape(-1, K // 32 * 18)
    return np.ascontiguousarray(rows[order]).reshape(-1, 18)
