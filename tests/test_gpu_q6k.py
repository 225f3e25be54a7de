"""GPU parity of the Q6_K head path (llama.cpp's output.weight) and of a model loaded from a GGUF file."""
import numpy as np
import pytest

from ggufio import random_q6_k, write_qwen_gguf
from lab import qwen_model as QM
from lab.hip import call, ptr
from oracle import model as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
NEAR_TIE = 1e-2


def relerr(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("N,K,T", [(4096, 1536, 1), (2048, 1536, 3), (512, 256, 4)])
def test_gemv_q6_k(cuda, N, K, T):
    """Q6_K x Q8_1: f64 accumulation of exact per-sub-block int32 terms -> agrees with the f64 dequantized
    product to ~1e-12 (reported against a 1e-9 bound)."""
    import torch
    rng = np.random.default_rng(N + T)
    b = random_q6_k(N * K // 256, rng, d=0.003)
    W = QM.Q6KMat(b, N, K, "cuda")
    x = rng.standard_normal((T, K), dtype=np.float32)
    q, d, s = OQ.quantize_q8_1(x)
    xq = torch.from_numpy(q).cuda()
    xds = torch.from_numpy(np.stack([d, s], -1)).cuda()
    y = torch.zeros(T, N, device=cuda)
    call("q355_gemv_q6_k_q8_1", ptr(W.lo), ptr(W.hi), ptr(W.sc), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(y))
    torch.cuda.synchronize()
    ref = OQ.gemv_q6_k_q8_1(b, N, K, q, d)
    assert relerr(y.cpu().numpy(), ref) < 1e-6          # fp32 output of an f64 sum


def test_gemv_q6_k_rejects_bad_k(cuda):
    from lab.hip import HipError
    with pytest.raises(HipError, match="multiple of 256"):
        call("q355_gemv_q6_k_q8_1", 1, 1, 1, 1, 64, 96, 1, 1, 1, 1)


def test_gguf_model_with_q6k_head_greedy(cuda, tmp_path):
    """Random weights written as a llama.cpp-style Qwen2 GGUF (Q4_0 layers and embedding, Q6_K output.weight),
    loaded back, decoded greedily on the GPU: tokens match the oracle up to its first near-tie."""
    cfg = QM.Config(L=2, V=4096)
    w = QM.random_weights(cfg, seed=31)
    w["head_q6k"] = random_q6_k(cfg.V * cfg.H // 256, np.random.default_rng(32), d=0.0005)
    p = tmp_path / "m.gguf"
    write_qwen_gguf(p, cfg, w)
    cfg2, w2 = QM.weights_from_gguf(p)
    dm = QM.DeviceModel(w2, cfg2, maxlen=256)
    assert dm.head_q6k is not None
    dec = QM.Decoder(dm, T=1, max_ctx=256)
    prompt = [int(t) for t in np.random.default_rng(33).integers(0, cfg.V, 12)]
    dec.prefill_tokens(prompt)
    got = dec.generate(12)[0]
    om = OM.Model(OM.Config(L=2, V=4096), w2, maxlen=256)
    ref, margins = om.greedy(prompt, 12)
    for i, (a, b) in enumerate(zip(got, ref)):
        if margins[i] < NEAR_TIE:
            break
        assert a == b, f"token {i}: {a} vs {b} (margin {margins[i]:.3g})"
