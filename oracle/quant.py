"""Oracle: Q4_0 / Q8_1 formats and the Q4_0 x Q8_1 GEMV (numpy). TEST INFRASTRUCTURE ONLY.

Restates:
  * the GGUF Q4_0 block (lab/gguf.py:3-5, 88-94): 18 B = fp16 d + 16 B qs; weight i is
    (qs[i] & 15) - 8 and weight i+16 is (qs[i] >> 4) - 8, value = d * weight;
  * the Q4_0 quantizer of BASELINE config 0 (llama.cpp quantize_row_q4_0_ref semantics, not in
    the reference tree): m = the signed value of max |x| (first on ties), d = m / -8 in fp32,
    stored fp16, q = clamp(round(x / d) + 8, 0, 15) with round = half away from zero, q = 8 when d = 0;
  * the Q8_1 activation quantizer: the rule is the reference's QUANT_Q8 (lab/qwen_batched.py:1032-1033):
    d = amax / 127 and r = x / d, both IEEE fp32 divisions, q = r rounded half to even (__float2int_rn),
    q = 0 when d = 0. The block is stored as BASELINE config 0 and llama.cpp's block_q8_1 store it
    (quantize_row_q8_1): d as fp16 (the scale every product uses), s = fp16(d * sum(q)) with the fp32 d;
  * the per-block int32 dot and the Q4_0 offset correction of the reference's int8 MMQ
    (lab/qwen_batched.py:1099-1101, 1237-1243): per 32-block b,
    dot_b = sum_i q_w,i (0..15) * q_x,i (exact int32), y += d_w * d_x * (dot_b - 8 * sum_i q_x,i).
"""
from __future__ import annotations

import numpy as np

QK = 32                 # weights per Q4_0 / Q8_1 block
Q4_0_BYTES = 18         # fp16 d + 16 B nibbles


def round_half_away(v: np.ndarray) -> np.ndarray:
    """C roundf(): nearest integer, halves away from zero. Evaluated in float64 so that
    v + 0.5 is exact for every float32 v of magnitude < 2^24 (no double rounding).
    pinned by: tests/test_oracle.py::test_round_half_away (hand cases incl. 0.49999997, 2.5, -2.5)."""
    v64 = np.asarray(v, dtype=np.float64)
    return np.trunc(v64 + np.copysign(0.5, v64))


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """fp32 [..., K] (K % 32 == 0) -> GGUF Q4_0 bytes uint8 [n_blocks, 18] in row-major block order.
    pinned by: hand-computed known-answer block, invariants (extreme element -> q = 0 exactly, |x - deq| <= |d|/2
    away from the clamp), round trip through the independent decoder q4_0_blocks()."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    idx = np.argmax(np.abs(x), axis=1)                      # first maximum, as llama.cpp's strict '<' scan
    m = x[np.arange(x.shape[0]), idx]
    d = (m / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d[:, None] != 0, x / d[:, None], np.float32(0.0)).astype(np.float32)
    q = np.clip(round_half_away(r) + 8, 0, 15).astype(np.uint8)
    out = np.empty((x.shape[0], Q4_0_BYTES), np.uint8)
    out[:, :2] = d.astype(np.float16).reshape(-1, 1).view(np.uint8)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out


def q4_0_blocks(b: np.ndarray):
    """GGUF Q4_0 bytes -> (d float32 [nblk], q uint8 [nblk, 32] stored 0..15) exactly as lab/gguf.py:88-94.
    pinned by: hand-written bytes with known nibbles (tests/test_oracle.py)."""
    blk = np.asarray(b, np.uint8).reshape(-1, Q4_0_BYTES)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    qs = blk[:, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    return d, q


def dequant_q4_0(b: np.ndarray, shape) -> np.ndarray:
    """GGUF Q4_0 bytes -> float32 values, reshaped (lab/gguf.py:77-79)."""
    d, q = q4_0_blocks(b)
    return (d[:, None] * (q.astype(np.float32) - 8)).reshape(shape)


def round_half_even(v: np.ndarray) -> np.ndarray:
    """CUDA __float2int_rn / rintf: nearest integer, halves to the even neighbour (numpy rint).
    pinned by: tests/test_oracle.py::test_round_half_even (hand cases 0.5, 1.5, 2.5, -0.5, -2.5)."""
    return np.rint(np.asarray(v, dtype=np.float32))


def quantize_q8_1(x: np.ndarray):
    """fp32 [T, K] -> (qs int8 [T, K], d fp16 [T, K/32], s fp16 [T, K/32]) by the rule above
    (lab/qwen_batched.py:1032-1033 for d and q; llama.cpp block_q8_1 for the stored d and s).
    pinned by: hand blocks where the rules differ (a half-integer x / d rounds to even; a value whose fp32
    quotient x / d and x / fp16(d) round to different codes), the amax element -> +-127, an all-zero block
    -> q = 0, d = 0, the bound |x - d q| <= d/2, and per-element brute-force loops in Python floats
    (tests/test_oracle.py)."""
    x = np.asarray(x, dtype=np.float32)
    T, K = x.shape
    xb = x.reshape(T, K // QK, QK)
    amax = np.abs(xb).max(axis=2)
    d32 = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d32[..., None] != 0, xb / d32[..., None], np.float32(0.0)).astype(np.float32)
    q = round_half_even(r).astype(np.int8)
    sq = q.astype(np.int32).sum(axis=2)
    s = (d32 * sq.astype(np.float32)).astype(np.float16)
    return q.reshape(T, K), d32.astype(np.float16), s


def dequant_q8_1(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    T, K = q.shape
    return (q.reshape(T, K // QK, QK).astype(np.float32) * d.astype(np.float32)[..., None]).reshape(T, K)


def block_dots(qw: np.ndarray, qx: np.ndarray) -> np.ndarray:
    """Unsigned-nibble x int8 per-block dots: qw uint8 [N, K] (0..15), qx int8 [T, K] -> int32 [T, N, K/32].
    Exact integer arithmetic (the values the GPU's v_dot4 / MFMA i8 chains must reproduce bit for bit).
    pinned by: brute-force triple loop on tiny shapes (tests)."""
    N, K = qw.shape
    T = qx.shape[0]
    a = qw.reshape(N, K // QK, QK).astype(np.int32)
    b = qx.reshape(T, K // QK, QK).astype(np.int32)
    return np.einsum("nbi,tbi->tnb", a, b, optimize=True).astype(np.int32)


def gemv_q4_0_q8_1(wbytes: np.ndarray, N: int, K: int, qx: np.ndarray, dx: np.ndarray,
                   out_dtype=np.float32) -> np.ndarray:
    """Y[T, N] = sum_b d_w[n,b] d_x[t,b] (dot_b - 8 sum(q_x,b)), accumulated in float64 (each term is exact),
    returned as out_dtype (fp32 by default).
    wbytes: GGUF Q4_0 bytes of W [N, K] (row-major); qx int8 [T, K], dx fp16 [T, K/32].
    pinned by: equality (to fp64 rounding) with the dequantize-then-matmul form
    (d_w (q_w - 8)) @ (d_x q_x)^T, which has no int32 dot and no -8 sum(q) correction term."""
    dw, qw = q4_0_blocks(wbytes)
    dw = dw.reshape(N, K // QK).astype(np.float64)
    qw = qw.reshape(N, K)
    T = qx.shape[0]
    dots = block_dots(qw, qx).astype(np.int64)                       # [T, N, nb]
    sq = qx.reshape(T, K // QK, QK).astype(np.int64).sum(axis=2)    # [T, nb]
    sumi = dots - 8 * sq[:, None, :]
    y = np.einsum("tnb,nb,tb->tn", sumi.astype(np.float64), dw, dx.astype(np.float64), optimize=True)
    return y.astype(out_dtype)


Q6_K_BYTES = 210        # ql[128] + qh[64] + int8 scales[16] + fp16 d, 256 weights


def dequant_q6_k(b: np.ndarray, shape) -> np.ndarray:
    """GGUF Q6_K bytes -> float64 values (llama.cpp block_q6_K; the reference reads it in lab/gguf.py:97-123).
    Per 256-weight block and 128-weight half n, for l < 32 (v = 6-bit value, scale index is):
      y[128n + l]      = d sc[8n + l/16]     (((ql[64n + l]      & 15) | ((qh[32n + l]      & 3) << 4)) - 32)
      y[128n + l + 32] = d sc[8n + l/16 + 2] (((ql[64n + l + 32] & 15) | ((qh[32n + l] >> 2 & 3) << 4)) - 32)
      y[128n + l + 64] = d sc[8n + l/16 + 4] (((ql[64n + l]      >> 4) | ((qh[32n + l] >> 4 & 3) << 4)) - 32)
      y[128n + l + 96] = d sc[8n + l/16 + 6] (((ql[64n + l + 32] >> 4) | ((qh[32n + l] >> 6 & 3) << 4)) - 32)
    pinned by: an element-by-element loop over the same formula on hand-set bytes (tests/test_oracle.py)."""
    blk = np.asarray(b, np.uint8).reshape(-1, Q6_K_BYTES)
    ql = blk[:, :128].astype(np.int64)
    qh = blk[:, 128:192].astype(np.int64)
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float64).reshape(-1)
    y = np.empty((blk.shape[0], 256), np.float64)
    l = np.arange(32)
    for n in range(2):
        a, c, h = ql[:, 64 * n + l], ql[:, 64 * n + 32 + l], qh[:, 32 * n + l]
        vals = [(a & 15) | ((h & 3) << 4), (c & 15) | (((h >> 2) & 3) << 4),
                (a >> 4) | (((h >> 4) & 3) << 4), (c >> 4) | (((h >> 6) & 3) << 4)]
        for k, v in enumerate(vals):
            s_idx = 8 * n + l // 16 + 2 * k
            y[:, 128 * n + 32 * k + l] = d[:, None] * sc[:, s_idx] * (v - 32)
    return y.reshape(shape)


def gemv_q6_k_q8_1(wbytes: np.ndarray, N: int, K: int, qx: np.ndarray, dx: np.ndarray) -> np.ndarray:
    """Y[T, N] = dequant(W_q6k) @ dequant(Q8_1 x)^T in float64 (every product is exact in f64: the sum is
    the only rounding)."""
    w = dequant_q6_k(wbytes, (N, K))
    x = dequant_q8_1(qx, dx).astype(np.float64)
    return x @ w.T


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32: the 16 bits are the top half of the float32 (bfloat16 definition).
    pinned by: hand values (0x3F80 = 1.0, 0xC040 = -3.0, 0x0000 = 0)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def gemv_q4_0_bf16(wbytes: np.ndarray, N: int, K: int, xbits: np.ndarray) -> np.ndarray:
    """Reference-parity GEMV (lab/qwen_kernels.py:14-113 semantics): Y[T, N] = dequant(W) @ x^T with x in bf16,
    evaluated in float64 (the GPU's fp32 accumulation agrees to ~1e-6 relative)."""
    w = dequant_q4_0(wbytes, (N, K)).astype(np.float64)
    return bf16_to_f32(xbits).astype(np.float64) @ w.T


def dequant_q4_0_f16(b: np.ndarray, shape) -> np.ndarray:
    """GGUF Q4_0 bytes -> fp16 values d (q - 8), rounded once (the batched-decode weight dequantization of
    gemv_v2_source, lab/qwen_batched.py:486-491: (q | 0x6400) as fp16 = 1024 + q, minus 1032, times d).
    The float32 product d (q - 8) is exact (11 x 4 significant bits), so one float32 -> float16 rounding
    gives the single rounding of the fp16 multiply.
    pinned by: the same value computed in numpy float16 arithmetic step by step (tests/test_oracle.py)."""
    d, q = q4_0_blocks(b)
    return (d.astype(np.float32)[:, None] * (q.astype(np.float32) - 8)).astype(np.float16).reshape(shape)


def gemv_q4_0_f16(wbytes: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    """Batched-decode product (gemv_v2_source semantics): fp16-dequantized W [N, K] times fp16 activations
    x [T, K] (rounded to fp16 here if given wider), evaluated in float64 (the GPU's fp32 MFMA accumulation
    agrees to ~1e-6 relative)."""
    w = dequant_q4_0_f16(wbytes, (N, K)).astype(np.float64)
    return np.asarray(x).astype(np.float16).astype(np.float64) @ w.T


def gemv_dequant_f64(wbytes: np.ndarray, N: int, K: int, qx: np.ndarray, dx: np.ndarray) -> np.ndarray:
    """Independent form of gemv_q4_0_q8_1 (dequantize both operands, float64 matmul); pins it."""
    w = dequant_q4_0(wbytes, (N, K)).astype(np.float64)
    x = dequant_q8_1(qx, dx).astype(np.float64)
    return (x @ w.T).astype(np.float32)
