"""CPU tests of the host side: GGUF reader and block decoders, the product Q4_0 quantizer (against the
oracle), the device repack and row orders, the synthetic weight generator, and the C-ABI library
(loads and exports every symbol declared in include/qwen355.h; no GPU calls)."""
import re
from pathlib import Path

import numpy as np
import pytest

from ggufio import random_q6_k, write_gguf, write_qwen_gguf
from lab import gguf, hip, qwen_kernels
from lab import qwen_model as QM
from oracle import quant as OQ

ROOT = Path(__file__).resolve().parents[1]


def test_product_quantizer_matches_oracle():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2048, 32)).astype(np.float32) * 0.02
    x[0] = 0
    x[1] = np.float32(0.5) * (np.arange(32) - 16)          # exact halves at x / d
    x[2] = -x[2] * 1e-30
    assert np.array_equal(gguf.quantize_q4_0(x), OQ.quantize_q4_0(x))


def test_tile_roundtrip_and_layout():
    rng = np.random.default_rng(1)
    N, K = 48, 96
    b = OQ.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
    qs, d = gguf.tile_q4_0(b, N, K)
    assert qs.shape == (N // 16, K // 32, 16, 16) and d.shape == (N // 16, K // 32, 16)
    blk = b.reshape(N, K // 32, 18)
    assert np.array_equal(qs[1, 2, 5], blk[16 + 5, 2, 2:])
    assert d[2, 1, 3].view(np.uint16) == blk[32 + 3, 1, :2].view(np.uint16)[0]
    assert np.array_equal(gguf.untile_q4_0(qs, d), b)


def test_row_orders():
    order = gguf.qkv_row_order(12, 2, 128)
    assert sorted(order.tolist()) == list(range(2048))
    assert order[:4].tolist() == [0, 64, 1, 65] and order[128:130].tolist() == [128, 192]
    assert order[1536:1538].tolist() == [1536, 1600]                   # k heads pair-interleaved
    assert order[1792:1795].tolist() == [1792, 1793, 1794]             # v in order
    gu = gguf.gate_up_row_order(8960)
    assert gu[:4].tolist() == [0, 8960, 1, 8961] and sorted(gu.tolist()) == list(range(17920))
    b = np.arange(4 * 2 * 18, dtype=np.uint8).reshape(8, 18)           # 4 rows x 2 blocks, K = 64
    t = gguf.take_rows_q4_0(b, 64, np.array([2, 0, 3, 1]))
    assert np.array_equal(t.reshape(4, 36)[0], b.reshape(4, 36)[2])


def _q6k_ref(block):
    """Q6_K decode written per element from the ggml block definition (ql[128], qh[64], scales[16], d)."""
    ql, qh = block[:128], block[128:192]
    sc = block[192:208].view(np.int8)
    d = float(block[208:210].view(np.float16)[0])
    out = np.zeros(256)
    for n in range(256):
        half, r = divmod(n, 128)
        quarter, l = divmod(r, 32)
        lo = ql[64 * half + l + (32 if quarter in (1, 3) else 0)]
        lo = lo & 15 if quarter < 2 else lo >> 4
        hi = (qh[32 * half + l] >> (2 * quarter)) & 3
        out[n] = d * sc[n // 16] * ((int(lo) | (int(hi) << 4)) - 32)
    return out


def test_gguf_reader_and_decoders(tmp_path):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((4, 64)).astype(np.float32)
    q4 = OQ.quantize_q4_0(w)
    q6 = rng.integers(0, 256, (2, 210), dtype=np.uint8)
    q6[:, 208:210] = np.array([0.01], np.float16).view(np.uint8)
    f16 = rng.standard_normal(8).astype(np.float16)
    tensors = {"a.weight": (2, (64, 4), q4.tobytes()), "b": (0, (4, 64), w.tobytes()),
               "c": (1, (8,), f16.tobytes()), "h": (14, (256, 2), q6.tobytes())}
    p = tmp_path / "t.gguf"
    write_gguf(p, tensors, {"qwen2.block_count": 28, "general.architecture": "qwen2",
                            "tokenizer.ggml.tokens": ["a", "bc", ""], "tokenizer.ggml.token_type": [1, -2, 3],
                            "qwen2.rope.freq_base": 1e6})
    g = gguf.GGUF(p)
    assert g.meta["qwen2.block_count"] == 28 and g.meta["general.architecture"] == "qwen2"
    assert g.meta["tokenizer.ggml.tokens"] == ["a", "bc", ""] and g.meta["tokenizer.ggml.token_type"] == [1, -2, 3]
    assert g.meta["qwen2.rope.freq_base"] == 1e6 and g.version == 3
    assert g.tensors["h"].dims == (256, 2) and g.tensors["h"].type == 14
    assert g.f32("a.weight").shape == (4, 64)
    assert np.array_equal(g.f32("a.weight"), OQ.dequant_q4_0(q4, (4, 64)))
    assert np.array_equal(g.f32("b").reshape(-1), w.reshape(-1).view(np.float32))
    assert np.array_equal(g.f32("c"), f16.astype(np.float32))
    dec = g.f32("h").reshape(2, 256)
    for i in range(2):
        assert np.allclose(dec[i], _q6k_ref(q6[i]), rtol=1e-6, atol=1e-7)
    q, sc, d = gguf.q6_k_parts(q6)
    assert q.dtype == np.int8 and sc.shape == (2, 16) and d.shape == (2,)


def test_random_weights_deterministic():
    cfg = QM.Config(L=1, V=256, FFN=128, H=128, NH=2, NKV=1, HD=64)
    a = QM.random_weights(cfg, seed=9)
    b = QM.random_weights(cfg, seed=9)
    c = QM.random_weights(cfg, seed=10)
    assert np.array_equal(a["embed"], b["embed"]) and np.array_equal(a["layers"][0]["wd"], b["layers"][0]["wd"])
    assert not np.array_equal(a["embed"], c["embed"])
    assert a["layers"][0]["wq"].shape == (2 * 64 * 128 // 32, 18)
    assert abs(float(a["layers"][0]["ln1"].mean()) - 1.0) < 0.01


def test_rope_tables_match_oracle():
    from oracle import model as OM
    a = QM.rope_tables(100)
    b = OM.rope_tables(100)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_library_exports_header_symbols():
    header = (ROOT / "include" / "qwen355.h").read_text()
    declared = sorted(set(re.findall(r"\b(q355_[a-z0-9_]+)\s*\(", header)))
    L = hip.lib()
    for name in declared:
        assert hasattr(L, name), name
    assert set(declared) == set(hip.exported_symbols())
    assert L.q355_version().startswith(b"qwen355")


def test_kernel_specs_name_exported_symbols():
    names = set(hip.exported_symbols())
    specs = [qwen_kernels.gemv_source(2, e) for e in ("store", "resid", "biasf", "swiglu", "biasf_kv")]
    specs += [qwen_kernels.RMSNORM_F32W_1P, qwen_kernels.ATTN4, qwen_kernels.FINISH_MB, qwen_kernels.EMBED_F32,
              qwen_kernels.QUANT_Q8, qwen_kernels.gemv_head_source()]
    for sp in specs:
        assert sp.symbol in names
    with pytest.raises(ValueError):
        qwen_kernels.gemv_source(1, "store", quant="g128f32")
    assert qwen_kernels.gemv_source(1, "resid", quant="bf16").symbol == "q355_gemv_q4_0_bf16"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(hip, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(hip, "_lib", None)
    with pytest.raises(hip.HipError, match="not built"):
        hip.lib()


def test_q6_k_planes_decode_to_the_oracle_values():
    """lab.gguf.tile_q6_k: decoding the planes with their documented bit layout gives the oracle's Q6_K values."""
    rng = np.random.default_rng(9)
    N, K = 32, 512
    b = random_q6_k(N * K // 256, rng, d=0.01)
    lo, hi, sc, d = gguf.tile_q6_k(b, N, K)
    ref = OQ.dequant_q6_k(b, (N, K))
    n = np.arange(N)
    for k in range(K):
        blk, i = divmod(k, 32)
        lo_b = lo[n // 16, blk, n % 16, i % 16].astype(np.int64)
        v = (lo_b & 15) if i < 16 else (lo_b >> 4)
        hb = hi[n // 16, blk, n % 16, i % 8].astype(np.int64)
        v = v | (((hb >> (2 * (i // 8))) & 3) << 4)
        s = sc[n // 16, blk, n % 16, i // 16].astype(np.float64)
        dd = d[n // 16, k // 256, n % 16].astype(np.float64)
        assert np.array_equal(dd * s * (v - 32), ref[:, k])


def test_weights_from_gguf_roundtrip(tmp_path):
    """A Qwen2 GGUF written from random weights (Q6_K head) is read back into the same weight dict."""
    cfg = QM.Config(L=2, V=512, FFN=256, H=256, NH=2, NKV=1, HD=128)
    w = QM.random_weights(cfg, seed=3)
    w["head_q6k"] = random_q6_k(cfg.V * cfg.H // 256, np.random.default_rng(4))
    p = tmp_path / "qwen.gguf"
    write_qwen_gguf(p, cfg, w)
    cfg2, w2 = QM.weights_from_gguf(p)
    assert (cfg2.H, cfg2.NH, cfg2.NKV, cfg2.HD, cfg2.FFN, cfg2.L, cfg2.V) == (256, 2, 1, 128, 256, 2, 512)
    assert abs(cfg2.eps - 1e-6) < 1e-12 and cfg2.theta == 1e6
    assert np.array_equal(w2["embed"], w["embed"]) and np.array_equal(w2["head_q6k"], w["head_q6k"])
    for a, b in zip(w["layers"], w2["layers"]):
        for k in a:
            assert np.array_equal(np.asarray(a[k]).reshape(-1), np.asarray(b[k]).reshape(-1)), k
