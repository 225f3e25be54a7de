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

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

# ggml type id -> (name, block size in elements, bytes per block)
GGML = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 14: ("Q6_K", 256, 210)}
# GGUF metadata scalar type id -> struct format
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_T_STRING, _T_ARRAY = 8, 9


@dataclass
class Tensor:
    name: str
    dims: tuple      # ggml order: dims[0] is the contiguous (K) axis
    type: int
    offset: int


class _Reader:
    def __init__(self, f):
        self.f = f

    def unpack(self, fmt):
        return struct.unpack(fmt, self.f.read(struct.calcsize(fmt)))

    def string(self):
        (n,) = self.unpack("<Q")
        return self.f.read(n).decode("utf-8", "replace")

    def value(self, typ):
        if typ == _T_STRING:
            return self.string()
        if typ == _T_ARRAY:
            sub, n = self.unpack("<IQ")
            return [self.value(sub) for _ in range(n)]
        return self.unpack(_FMT[typ])[0]


class GGUF:
    """GGUF v2/v3 file: metadata dict, tensor directory, memory-mapped data."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self.meta, self.tensors = {}, {}
        with open(self.path, "rb") as f:
            r = _Reader(f)
            magic, self.version, n_tensors, n_kv = r.unpack("<4sIQQ")
            if magic != b"GGUF":
                raise ValueError(f"{path}: not a GGUF file (magic {magic!r})")
            for _ in range(n_kv):
                key = r.string()
                (typ,) = r.unpack("<I")
                self.meta[key] = r.value(typ)
            for _ in range(n_tensors):
                name = r.string()
                (nd,) = r.unpack("<I")
                dims = r.unpack(f"<{nd}Q")
                typ, off = r.unpack("<IQ")
                self.tensors[name] = Tensor(name, tuple(dims), typ, off)
            align = int(self.meta.get("general.alignment", 32))
            self.data_start = -(-f.tell() // align) * align
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")

    def raw(self, name: str):
        """-> (uint8 bytes of the tensor, Tensor)."""
        t = self.tensors[name]
        _, blk, bsz = GGML[t.type]
        n = int(np.prod(t.dims))
        start = self.data_start + t.offset
        return np.asarray(self.mm[start:start + n // blk * bsz]), t

    def f32(self, name: str) -> np.ndarray:
        """Decoded float32 array, shape reversed from ggml dims (row-major [N, K])."""
        b, t = self.raw(name)
        kind = GGML[t.type][0]
        if kind == "F32":
            a = b.view(np.float32)
        elif kind == "F16":
            a = b.view(np.float16).astype(np.float32)
        elif kind == "Q4_0":
            d, q = q4_0_blocks(b)
            a = (d[:, None] * (q.astype(np.float32) - 8)).reshape(-1)
        elif kind == "Q6_K":
            q, s = q6_k_blocks(b)
            a = (q.astype(np.float32) * np.repeat(s, 16, axis=1)).reshape(-1)
        else:
            raise NotImplementedError(kind)
        return a.reshape(tuple(reversed(t.dims)))


def q4_0_blocks(b: np.ndarray):
    """-> d float32 [nblk], q uint8 [nblk, 32] in weight order (low nibbles 0..15, high nibbles 16..31)."""
    blk = np.asarray(b, np.uint8).reshape(-1, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    lo, hi = blk[:, 2:] & 15, blk[:, 2:] >> 4
    return d, np.concatenate([lo, hi], axis=1)


def q6_k_blocks(b: np.ndarray):
    """-> q int8 [nblk, 256] in [-32, 31], s float32 [nblk, 16] (= d * scale of each 16 weights)."""
    q, sc, d = _q6_k_fields(b)
    return q, d.astype(np.float32)[:, None] * sc.astype(np.float32)


def q6_k_parts(b: np.ndarray):
    """-> q int8 [nblk, 256] in [-32, 31], sc int8 [nblk, 16], d fp16 [nblk] (Q6_K's raw fields)."""
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
