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


@pytest.mark.parametrize("N,K,T", [(8192, 1536, 8), (151936, 1536, 32), (4096, 1536, 5), (1024, 256, 17)])
def test_mmq_q6k_logits(cuda, N, K, T):
    """The batched Q6_K head on int8 MFMA (exact int32 sub-block dots, fp32 accumulation) against the oracle's
    f64 dequantized product (oracle.quant.gemv_q6_k_q8_1, the arithmetic of oracle.model.LinearQ6K): logits
    within 1e-5 relative, argmax partials of every 64 rows consistent with the logits."""
    import torch
    rng = np.random.default_rng(N + T)
    b = random_q6_k(N * K // 256, rng, d=0.0005)
    W = QM.Q6KMat(b, N, K, "cuda")
    x = rng.standard_normal((T, K), dtype=np.float32)
    q, d, s = OQ.quantize_q8_1(x)
    xq = torch.from_numpy(q).cuda()
    xds = torch.from_numpy(np.stack([d, s], -1)).cuda()
    y = torch.full((T, N), float("nan"), device=cuda)
    pmax = torch.zeros(T, N // 64, device=cuda)
    pidx = torch.zeros(T, N // 64, dtype=torch.int32, device=cuda)
    call("q355_mmq_q6k_logits", ptr(W.lo), ptr(W.hi), ptr(W.sc), ptr(W.d), N, K, ptr(xq), ptr(xds), T, ptr(y),
         ptr(pmax), ptr(pidx))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = OQ.gemv_q6_k_q8_1(b, N, K, q, d)
    assert relerr(got, ref) < 1e-5
    parts = got.reshape(T, N // 64, 64)
    assert np.array_equal(pmax.cpu().numpy(), parts.max(axis=2))
    assert np.array_equal(pidx.cpu().numpy(), parts.argmax(axis=2) + 64 * np.arange(N // 64)[None])


@pytest.mark.parametrize("B", [8, 32])
def test_batched_decode_with_q6k_head(cuda, B):
    """BatchedDecoder with llama.cpp's Q6_K output.weight (int8 MMQ layers, Q6_K MFMA head), teacher-forced
    against the oracle (oracle.model.LinearQ6K head): logits within the batched int8 mode's bound (1e-3 of the
    largest |logit|), argmax equal wherever the oracle's margin is at least NEAR_TIE."""
    import torch
    from lab import qwen_batched as QB
    cfg = QM.Config(L=2, V=4096)
    w = QM.random_weights(cfg, seed=31)
    # d = 2e-5: weights of std ~0.02 like the Q4_0 layers (logits of the magnitude of the tied Q4_0 head's)
    w["head_q6k"] = random_q6_k(cfg.V * cfg.H // 256, np.random.default_rng(32), d=0.00002)
    dm = QM.DeviceModel(w, cfg, maxlen=256)
    om = OM.Model(OM.Config(L=2, V=4096), w, maxlen=256)
    rng = np.random.default_rng(B + 40)
    prompts = rng.integers(0, cfg.V, (B, 5))
    bd = QB.BatchedDecoder(dm, B=B, max_ctx=128, page_seed=B, keep_logits=True)
    bd.prefill_tokens(prompts)
    seqs = [0, B // 2, B - 1]
    caches, lgs = {}, {}
    for s_ in seqs:
        caches[s_] = om.new_cache()
        lgs[s_] = om.logits(om.forward(list(prompts[s_]), 0, caches[s_])[-1:])[0]
    for t in range(4):
        got = bd.logits.cpu().numpy()
        toks = got.argmax(axis=1).astype(np.int32)
        for s_ in seqs:
            lg = lgs[s_]
            dev = float(np.abs(got[s_] - lg).max())
            assert dev <= 1e-3 * float(np.abs(lg).max()), f"B={B} seq {s_} step {t}: logits off by {dev:.3g}"
            top2 = np.partition(lg, -2)[-2:]
            if top2[1] - top2[0] >= NEAR_TIE:
                assert int(toks[s_]) == int(np.argmax(lg))
            toks[s_] = int(np.argmax(lg))
            lgs[s_] = om.logits(om.forward([int(toks[s_])], 5 + t, caches[s_]))[0]
        bd.tok.copy_(torch.from_numpy(toks))
        bd.step()
