"""CPU checks that pin the numpy oracle (oracle/) independently of the code under test.

The reference repository holds no golden vectors for this path (its checks are float64 recomputations
inside benchmark scripts), so each oracle function is pinned here by a hand-computed known answer, a
closed form, an invariant, or an independently written second form, chosen so that a plausible
mistake (a dropped -8 term, a wrong nibble order, a transposed operand, a wrong RoPE pairing) fails.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
from scipy.special import expit, softmax

from oracle import model as OM
from oracle import quant as OQ


# ------------------------------------------------------------------------------------------------
# rounding and quantizers

def test_round_half_away():
    v = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997, 1.4999999, 7.5, -7.5, 0.0], np.float32)
    assert OQ.round_half_away(v).tolist() == [1, -1, 2, 3, -3, 0, -0, 1, 8, -8, 0]


def _fp16_bytes(x):
    return np.array([x], np.float16).view(np.uint8).tolist()


def test_q4_0_known_block():
    """x_i = i - 16: max |x| is x_0 = -16 -> d = 2, q_i = round((i - 16) / 2) + 8 (halves away from zero)."""
    x = np.arange(32, dtype=np.float32) - 16
    b = OQ.quantize_q4_0(x)
    assert b.shape == (1, 18)
    assert b[0, :2].tolist() == _fp16_bytes(2.0)
    expect = []
    for i in range(32):
        r = Fraction(i - 16, 2)
        q = math.floor(r + Fraction(1, 2)) if r >= 0 else -math.floor(-r + Fraction(1, 2))
        expect.append(min(15, max(0, q + 8)))
    qs = b[0, 2:]
    assert [int(v) for v in (qs & 15)] == expect[:16]
    assert [int(v) for v in (qs >> 4)] == expect[16:]
    assert expect[0] == 0 and expect[31] == 15          # -16 -> 0; 15 / 2 = 7.5 -> 8 -> 16 clamped to 15


def test_q4_0_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 32)).astype(np.float32) * 0.02
    x[0] = 0.0                                             # all-zero block
    x[1] = 0.0
    x[1, 5] = -3.0                                         # single non-zero element
    b = OQ.quantize_q4_0(x)
    d, q = OQ.q4_0_blocks(b)
    assert d[0] == 0 and (q[0] == 8).all()
    assert q[1, 5] == 0 and d[1] == np.float32(np.float16(-3.0 / -8))
    i = np.abs(x).argmax(axis=1)
    live = d != 0
    assert (q[np.arange(len(q)), i][live] == 0).all()      # the extreme element maps to q = 0 exactly
    d32 = (x[np.arange(len(x)), i] / np.float32(-8)).astype(np.float32)
    r = x / np.where(d32 == 0, 1, d32)[:, None]
    unclamped = r < 7.5                                     # q = 15 clamps only where x/d rounds past 7
    err = np.abs(r - (q.astype(np.float64) - 8))
    assert (err[unclamped] <= 0.5 + 1e-6).all()


def test_q4_0_decoder_known_bytes():
    """lab/gguf.py:88-94 layout: weight i is the low nibble of qs[i], weight i + 16 the high nibble."""
    b = np.zeros((1, 18), np.uint8)
    b[0, :2] = _fp16_bytes(0.5)
    b[0, 2:] = np.arange(16) | ((15 - np.arange(16)) << 4)
    d, q = OQ.q4_0_blocks(b)
    assert d.tolist() == [0.5]
    assert q[0].tolist() == list(range(16)) + list(range(15, -1, -1))
    assert OQ.dequant_q4_0(b, (32,)).tolist() == [0.5 * (v - 8) for v in q[0].tolist()]


def test_round_half_even():
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, 126.5, -124.5], np.float32)
    assert OQ.round_half_even(v).tolist() == [0, 2, 2, -0, -2, -2, 0, 126, -124]


def _rn32(fr: Fraction) -> Fraction:
    """Exact rational -> the nearest float32 (ties to even significand), decided by exact comparisons."""
    f = np.float32(float(fr))
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr), int(np.array(c).view(np.uint32)) & 1))
    return Fraction(float(best))


def _q8_expect(block):
    """Q8_1 of one 32-value block from its definition (lab/qwen_batched.py:1032-1033): d = RN32(amax / 127),
    q = round-half-even(RN32(x / d)), 0 when d = 0; computed with exact rationals."""
    amax = max(abs(Fraction(float(v))) for v in block)
    d = _rn32(amax / 127)
    if d == 0:
        return [0] * 32, d
    return [round(_rn32(Fraction(float(v)) / d)) for v in block], d   # round() on a Fraction: half to even


def test_q8_1_known_blocks():
    x = np.zeros((1, 160), np.float32)
    x[0, :32] = np.linspace(-1.0, 2.0, 32, dtype=np.float32)    # amax 2 at the last element
    x[0, 64:96] = -1e-9                                           # d underflows to fp16 zero (fp32 d does not)
    x[0, 96:128] = np.float32(127.0)                              # d = 1 exactly: half-integers round to even
    x[0, 96:105] = [2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -3.5, 4.5, 0.0]
    x[0, 128:160] = np.float32(1.0)                               # d = fp32(1/127): fp16(d) differs from it
    x[0, 128] = np.float32(-0.9803)
    q, d, s = OQ.quantize_q8_1(x)
    assert q[0, 31] == 127 and d[0, 0] == np.float16(np.float32(2.0) / np.float32(127))
    assert d[0, 1] == 0 and (q[0, 32:64] == 0).all() and s[0, 1] == 0
    assert d[0, 2] == 0 and (q[0, 64:96] == -127).all()        # the rule divides by the fp32 d (nonzero)
    assert q[0, 96:105].tolist() == [2, -2, 0, 0, 2, 126, -4, 4, 0]   # half away from zero would give 3, -3, 1, ...
    # x / fp32 d = -124.498 -> -124; x / fp16 d = -124.506 would give -125: the divisor is the fp32 d
    assert q[0, 128] == -124
    for b in range(5):
        want, d32 = _q8_expect(x[0, 32 * b:32 * b + 32])
        assert q[0, 32 * b:32 * b + 32].tolist() == want
        assert d[0, b] == np.float16(float(d32))
        # llama.cpp block_q8_1: s = fp16(d * sum q) with the fp32 d
        assert s[0, b] == np.float16(np.float32(float(d32)) * np.float32(sum(want)))


def test_q8_1_fp16_subnormal_scale():
    """A block of small values (amax 1e-4): d = amax / 127 = 7.9e-7 is an fp16 subnormal. The codes follow the
    reference's QUANT_Q8 (divisor = the fp32 d, so the amax element is +-127); the stored scale is BASELINE's fp16
    d, here a subnormal whose relative error (~1e-2) exceeds fp16's 2^-11 -- where this build's products differ
    from the reference's (which keeps the fp32 d). The GPU quantizer writes the same bytes (test_gpu_kernels)."""
    x = (np.linspace(-1.0, 1.0, 32, dtype=np.float32) * np.float32(1e-4))[None]
    q, d, _ = OQ.quantize_q8_1(x)
    want, d32 = _q8_expect(x[0])
    assert q[0].tolist() == want and abs(q[0]).max() == 127
    assert 0 < float(d[0, 0]) < 6.1e-5                              # fp16 subnormal
    assert abs(float(d[0, 0]) - float(d32)) > float(d32) * 2.0 ** -11


def test_q8_1_bruteforce_random():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 96)) * rng.choice([1e-3, 1.0, 40.0], (3, 1))).astype(np.float32)
    q, d, _ = OQ.quantize_q8_1(x)
    for t in range(3):
        for b in range(3):
            want, d32 = _q8_expect(x[t, 32 * b:32 * b + 32])
            assert q[t, 32 * b:32 * b + 32].tolist() == want
            assert d[t, b] == np.float16(float(d32))


def test_q8_1_error_bound():
    x = np.random.default_rng(1).standard_normal((8, 1536)).astype(np.float32)
    q, d, _ = OQ.quantize_q8_1(x)
    d32 = np.abs(x.reshape(8, -1, 32)).max(axis=2).astype(np.float64) / 127    # the divisor (fp32 d, ~1 ulp)
    back = q.astype(np.float64) * np.repeat(d32, 32, axis=1)
    assert (np.abs(back - x) <= 0.5 * np.repeat(d32, 32, axis=1) * (1 + 1e-5)).all()
    assert (np.abs(d.astype(np.float64) - d32) <= d32 * 2.0 ** -11).all()        # stored d = fp16 of it
    assert np.abs(q).max() == 127


# ------------------------------------------------------------------------------------------------
# int dots and the GEMV

def test_block_dots_bruteforce():
    rng = np.random.default_rng(2)
    N, K, T = 5, 64, 3
    qw = rng.integers(0, 16, (N, K), dtype=np.uint8)
    qx = rng.integers(-127, 128, (T, K), dtype=np.int8)
    got = OQ.block_dots(qw, qx)
    for t in range(T):
        for n in range(N):
            for b in range(K // 32):
                want = sum(int(qw[n, 32 * b + i]) * int(qx[t, 32 * b + i]) for i in range(32))
                assert got[t, n, b] == want


@pytest.mark.parametrize("N,K,T", [(64, 1536, 1), (48, 256, 3)])
def test_gemv_int_form_equals_dequant_form(N, K, T):
    rng = np.random.default_rng(N + K)
    b = OQ.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    q, d, _ = OQ.quantize_q8_1(rng.standard_normal((T, K)).astype(np.float32))
    y_int = OQ.gemv_q4_0_q8_1(b, N, K, q, d)
    y_deq = OQ.gemv_dequant_f64(b, N, K, q, d)
    assert np.allclose(y_int, y_deq, rtol=1e-6, atol=1e-7)
    # the -8 offset matters: dropping it changes the result by far more than the tolerance
    dw, qw = OQ.q4_0_blocks(b)
    wrong = (np.repeat(dw.reshape(N, -1), 32, 1) * qw.reshape(N, K)).astype(np.float64) @ OQ.dequant_q8_1(q, d).T
    assert np.abs(wrong.T - y_int).max() > 1e-2


def test_linear_modes_agree():
    rng = np.random.default_rng(3)
    N, K = 96, 512
    b = OQ.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    x = rng.standard_normal((2, K)).astype(np.float32)
    a = OM.Linear(b, N, K, "int")(x)
    f = OM.Linear(b, N, K, "f64")(x)
    assert np.allclose(a, f, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------------------------------------
# elementwise ops

def test_rope_tables_closed_form():
    cos, sin = OM.rope_tables(4, 128, 1e6)
    assert (cos[0] == 1).all() and (sin[0] == 0).all()
    for i in (0, 1, 31, 63):
        inv = 1e6 ** (-2 * i / 128)
        assert cos[1, i] == np.float32(math.cos(inv)) and sin[3, i] == np.float32(math.sin(3 * inv))


def test_rope_is_complex_rotation():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(128)
    cos, sin = OM.rope_tables(300, 128, 1e6)
    p = 257
    out = OM.rope(x, cos[p], sin[p])
    z = (x[:64] + 1j * x[64:]) * (cos[p].astype(np.float64) + 1j * sin[p].astype(np.float64))
    assert np.allclose(out[:64], z.real) and np.allclose(out[64:], z.imag)
    assert np.isclose(np.linalg.norm(out), np.linalg.norm(x), rtol=1e-6)
    assert np.array_equal(OM.rope(x, cos[0], sin[0]), x)


def test_rmsnorm_closed_form():
    w = np.linspace(0.5, 1.5, 64)
    h = np.full((1, 64), 3.0)
    assert np.allclose(OM.rmsnorm(h, w, 1e-6), 3.0 / math.sqrt(9.0 + 1e-6) * w)
    g = np.random.default_rng(5).standard_normal((2, 64))
    assert np.allclose(OM.rmsnorm(g * 7.0, w, 0.0), OM.rmsnorm(g, w, 0.0))


def test_silu_mul():
    g = np.linspace(-20, 20, 101)
    u = np.linspace(1, 2, 101)
    assert np.allclose(OM.silu_mul(g, u), g * expit(g) * u)
    assert OM.silu_mul(np.array([0.0]), np.array([5.0]))[0] == 0


def test_argmax_lowest_index():
    assert OM.argmax_lowest(np.array([1.0, 3.0, 3.0, 2.0])) == 1
    assert OM.argmax_lowest(np.array([-1.0, -1.0])) == 0


# ------------------------------------------------------------------------------------------------
# attention

def test_attn_decode_special_cases():
    rng = np.random.default_rng(6)
    nh, nkv, hd, n = 4, 2, 16, 10
    V = rng.standard_normal((nkv, n, hd)).astype(np.float16)
    K = np.zeros((nkv, n, hd), np.float16)                    # uniform scores -> mean of V
    q = rng.standard_normal((nh, hd)).astype(np.float16)
    out = OM.attn_decode(q, K, V, n, nh, nkv).reshape(nh, hd)
    for h in range(nh):
        assert np.allclose(out[h], V[h // 2].astype(np.float64).mean(0), atol=1e-6)
    K2 = np.zeros((nkv, n, hd), np.float16)
    K2[:, 3] = 60.0                                            # one dominant key per KV head
    q2 = np.ones((nh, hd), np.float16)
    out2 = OM.attn_decode(q2, K2, V, n, nh, nkv).reshape(nh, hd)
    for h in range(nh):
        assert np.allclose(out2[h], V[h // 2, 3].astype(np.float64), atol=1e-5)


def test_attn_prefill_matches_decode_and_softmax():
    rng = np.random.default_rng(7)
    nh, nkv, hd, pos0, P = 6, 2, 32, 5, 4
    n = pos0 + P
    K = rng.standard_normal((nkv, n, hd)).astype(np.float16)
    V = rng.standard_normal((nkv, n, hd)).astype(np.float16)
    q = rng.standard_normal((P, nh, hd)).astype(np.float16)
    out = OM.attn_prefill(q, K, V, pos0, nh, nkv).reshape(P, nh, hd)
    for t in range(P):
        dec = OM.attn_decode(q[t], K, V, pos0 + t + 1, nh, nkv).reshape(nh, hd)
        assert np.allclose(out[t], dec, atol=1e-6)
        for h in range(nh):                                   # scipy softmax, written out per row
            s = K[h // 3, :pos0 + t + 1].astype(np.float64) @ q[t, h].astype(np.float64) / math.sqrt(hd)
            want = softmax(s) @ V[h // 3, :pos0 + t + 1].astype(np.float64)
            assert np.allclose(out[t, h], want, atol=1e-6)


# ------------------------------------------------------------------------------------------------
# whole model: prefill of a prompt equals token-by-token decode of it

def test_model_prefill_equals_decode():
    from lab import qwen_model as QM      # the weight generator (input data), not code under test here
    cfg = QM.Config(L=2, V=512, FFN=256, H=256, NH=4, NKV=2, HD=64)
    w = QM.random_weights(cfg, seed=3)
    ocfg = OM.Config(H=256, NH=4, NKV=2, HD=64, FFN=256, L=2, V=512)
    m = OM.Model(ocfg, w, maxlen=64)
    toks = [5, 17, 300, 2, 99]
    c1 = m.new_cache()
    h1 = m.forward(toks, 0, c1)
    c2 = m.new_cache()
    hs = [m.forward([t], i, c2)[0] for i, t in enumerate(toks)]
    assert np.allclose(h1, np.stack(hs), rtol=1e-4, atol=1e-4)
    assert np.allclose(c1["K"][:, :, :5].astype(np.float32), c2["K"][:, :, :5].astype(np.float32), atol=2e-3)
    assert np.allclose(c1["V"][:, :, :5].astype(np.float32), c2["V"][:, :, :5].astype(np.float32), atol=2e-3)


def test_model_decode_batch_equals_per_sequence():
    """decode_batch (the S rows' GEMVs as one product) equals Model.forward run for each sequence alone, for
    sequences at different positions; a mixed-up row/cache pairing (two caches swapped) fails it."""
    from lab import qwen_model as QM      # the weight generator (input data), not code under test here
    cfg = QM.Config(L=2, V=512, FFN=256, H=256, NH=4, NKV=2, HD=64)
    w = QM.random_weights(cfg, seed=5)
    ocfg = OM.Config(H=256, NH=4, NKV=2, HD=64, FFN=256, L=2, V=512)
    m = OM.Model(ocfg, w, maxlen=64)
    prompts = [[5, 17, 300], [2, 99, 7, 44, 1], [8]]
    def setup():
        caches = [m.new_cache() for _ in prompts]
        for p, c in zip(prompts, caches):
            m.forward(p, 0, c)
        return caches
    toks, pos = [11, 23, 400], [len(p) for p in prompts]
    ca, cb = setup(), setup()
    hb = m.decode_batch(toks, pos, ca)
    for r in range(3):
        hs = m.forward([toks[r]], pos[r], cb[r])[0]
        assert np.allclose(hb[r], hs, rtol=1e-12, atol=1e-12)
        assert np.array_equal(ca[r]["K"], cb[r]["K"]) and np.array_equal(ca[r]["V"], cb[r]["V"])
    cc = setup()
    hx = m.decode_batch(toks, pos, [cc[1], cc[0], cc[2]])
    assert not np.allclose(hx[0], hb[0], rtol=1e-3)


def test_q6_k_decode_matches_encoded_values():
    """Q6_K: chosen 6-bit values and scales, scattered into ql/qh bytes by an encoder written from the block
    definition, decode back exactly (and the three independent decoders agree)."""
    rng = np.random.default_rng(12)
    v = rng.integers(0, 64, (3, 256))
    sc = rng.integers(-128, 128, (3, 16))
    blk = np.zeros((3, 210), np.uint8)
    for b in range(3):
        for n in range(256):
            half, r = divmod(n, 128)
            quarter, l = divmod(r, 32)
            qi = 64 * half + l + (32 if quarter % 2 else 0)
            blk[b, qi] |= (v[b, n] & 15) << (4 if quarter >= 2 else 0)
            blk[b, 128 + 32 * half + l] |= (v[b, n] >> 4) << (2 * quarter)
        blk[b, 192:208] = sc[b].astype(np.int8).view(np.uint8)
        blk[b, 208:210] = np.array([0.125], np.float16).view(np.uint8)
    y = OQ.dequant_q6_k(blk, (3, 256))
    assert np.array_equal(y, 0.125 * np.repeat(sc, 16, axis=1) * (v - 32))


def test_bf16_decode_and_rounding():
    assert OQ.bf16_to_f32(np.array([0x3F80, 0xC040, 0x0000], np.uint16)).tolist() == [1.0, -3.0, 0.0]
    # 1 + 2^-8 is a bf16 midpoint between 1 and 1 + 2^-7: ties to even (1.0); 1 + 3 * 2^-8 rounds up
    x = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -2.5], np.float32)
    assert OQ.bf16_to_f32(OQ.f32_to_bf16(x)).tolist() == [1.0, 1.0, 1 + 2 ** -6, -2.5]


def test_q4_0_f16_dequant_matches_fp16_arithmetic():
    """d (q - 8) rounded once to fp16 equals the reference's fp16 steps: (1024 + q) - 1032, times d, each
    step in float16 arithmetic (lab/qwen_batched.py:486-491)."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 256)) * rng.choice([1e-3, 0.02, 3.0], (64, 1))).astype(np.float32)
    b = OQ.quantize_q4_0(w)
    d, q = OQ.q4_0_blocks(b)
    step = ((np.float16(1024) + q.astype(np.float16)) - np.float16(1032)) * d.astype(np.float16)[:, None]
    assert step.dtype == np.float16
    got = OQ.dequant_q4_0_f16(b, (64, 256))
    assert np.array_equal(got.reshape(-1, 32).view(np.uint16), step.view(np.uint16))
    # and it is the fp32 dequantization rounded to fp16
    assert np.array_equal(got, OQ.dequant_q4_0(b, (64, 256)).astype(np.float16))
