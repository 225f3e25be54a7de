"""GPU runs against the committed golden fixtures (tests/golden/, written by make_golden.py from the oracle).

Covers BASELINE config 0 (the 8960 x 1536 GEMV: per-block int32 dots bit-exact, y within 1e-3) and
config 2 (the full 28-layer model, 128-token prompt, 256 greedy tokens). Greedy parity is checked
free-running over all 256 steps (the reference's check), and teacher-forced: at every step the GPU is fed the
oracle's token, and its argmax must equal the oracle's wherever the oracle's top-2 logit margin is not a
near-tie (< NEAR_TIE).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from lab import gguf
from lab import qwen_model as QM
from lab.hip import call, ptr

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLD / "golden.json").read_text())
NEAR_TIE = 1e-2
FREE_TIE = 1e-6


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_quant_vectors(cuda):
    import torch
    f = np.load(GOLD / "quant_vectors.npz")
    x = torch.from_numpy(f["q8_x"]).cuda()
    T, K = x.shape
    q = torch.zeros(T, K, dtype=torch.int8, device=cuda)
    ds = torch.zeros(T, K // 32, 2, dtype=torch.float16, device=cuda)
    call("q355_quant_q8_1", ptr(x), ptr(q), ptr(ds), T, K)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), f["q8_q"])
    assert np.array_equal(ds.cpu().numpy()[..., 0].view(np.uint16), f["q8_d"].view(np.uint16))
    assert np.array_equal(ds.cpu().numpy()[..., 1].view(np.uint16), f["q8_s"].view(np.uint16))
    assert np.array_equal(gguf.quantize_q4_0(f["q4_x"]), f["q4_bytes"])


def test_config0_gemv(cuda):
    """BASELINE config 0 on the GPU: every per-block int32 dot bit-exact, y within 1e-3 of the oracle."""
    import torch
    f = np.load(GOLD / "config0_gemv.npz")
    rng = np.random.default_rng(0)
    w = rng.standard_normal((8960, 1536), dtype=np.float32) * np.float32(0.02)
    x = rng.standard_normal((1, 1536), dtype=np.float32)
    wb = gguf.quantize_q4_0(w)
    assert sha(wb) == META["config0"]["w_q4_0_sha256"]
    W = QM.Q4Mat(wb, 8960, 1536, "cuda")
    xt = torch.from_numpy(x).cuda()
    xq = torch.zeros(1, 1536, dtype=torch.int8, device=cuda)
    xds = torch.zeros(1, 48, 2, dtype=torch.float16, device=cuda)
    call("q355_quant_q8_1", ptr(xt), ptr(xq), ptr(xds), 1, 1536)
    y = torch.zeros(1, 8960, device=cuda)
    call("q355_gemv_q4_0_q8_1", ptr(W.qs), ptr(W.d), 8960, 1536, ptr(xq), ptr(xds), 1, ptr(y), None, 0)
    dots = torch.zeros(1, 8960, 48, dtype=torch.int32, device=cuda)
    call("q355_gemv_blockdots", ptr(W.qs), 8960, 1536, ptr(xq), 1, ptr(dots))
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), f["qx"])
    d = dots.cpu().numpy()
    assert sha(d) == META["config0"]["dots_sha256"]
    assert np.array_equal(d[0, 0], f["dots_row0"]) and int(d.astype(np.int64).sum()) == int(f["dots_sum"][0])
    ref = f["y"]
    assert float(np.abs(y.cpu().numpy() - ref).max() / np.abs(ref).max()) < 1e-3


def _teacher_forced(dec, first_tok, ref_tokens):
    """Replay the decode graph with the reference token fed at every step; return the GPU's argmax per step."""
    import torch
    dec.tok.fill_(int(first_tok))
    g = dec.capture()
    got = []
    for t in range(len(ref_tokens)):
        g.replay()
        got.append(int(dec.tok.item()))
        dec.tok.fill_(int(ref_tokens[t]))
    return got


def _check(got, ref, margins, what):
    bad = [i for i, (x, y) in enumerate(zip(got, ref)) if x != y and margins[i] >= NEAR_TIE]
    assert not bad, f"{what}: steps {bad[:10]} differ at non-tie margins {[margins[i] for i in bad[:10]]}"


def test_small_model_golden(cuda):
    m = META["small_model"]
    cfg = QM.Config(L=m["cfg"]["L"], V=m["cfg"]["V"])
    w = QM.random_weights(cfg, seed=m["seed"])
    assert sha(w["embed"]) == m["embed_sha256"]
    dm = QM.DeviceModel(w, cfg, maxlen=512)
    dec = QM.Decoder(dm, T=1, max_ctx=512)
    dec.prefill_tokens(m["prompt"][:-1])
    # the prompt's last token is fed by the forced loop; step t then predicts token t
    forced = _teacher_forced(dec, m["prompt"][-1], m["tokens"])
    _check(forced, m["tokens"], m["margins"], "small model")


@pytest.mark.skipif("config2" not in META, reason="config-2 fixture not generated")
def test_config2_greedy_256(cuda):
    """28 layers, tied Q4_0 head, 128-token prompt, 256 greedy steps (teacher-forced)."""
    m = META["config2"]
    w = QM.random_weights(QM.QWEN15, seed=m["seed"])
    assert sha(w["embed"]) == m["embed_sha256"] and sha(w["layers"][0]["wq"]) == m["layer0_wq_sha256"]
    dm = QM.DeviceModel(w, QM.QWEN15, maxlen=512)
    dec = QM.Decoder(dm, T=1, max_ctx=512)
    dec.prefill_tokens(m["prompt"][:-1])
    pos0 = dec.pos.clone()
    forced = _teacher_forced(dec, m["prompt"][-1], m["tokens"])
    _check(forced, m["tokens"], m["margins"], "config 2")
    # free running from the same state (the reference's own check, scripts/qwen_e2e.py:240-243): the batch-1
    # path reproduces the oracle's f64 logits to ~1e-12, so every one of the 256 tokens must agree unless the
    # oracle's top-2 margin at the first difference is below FREE_TIE (far above that error, far below any
    # margin of this run, whose smallest is ~4e-4)
    dec.pos.copy_(pos0)
    dec.tok.fill_(int(m["prompt"][-1]))
    dec.graph.replay()
    free = dec.generate(256)[0].tolist()
    agree = next((i for i, (x, y) in enumerate(zip(free, m["tokens"])) if x != y), 256)
    print(f"config 2: free-running agreement {agree}/256 (smallest oracle margin {min(m['margins']):.3g})")
    assert agree == 256 or m["margins"][agree] < FREE_TIE, \
        f"config 2 free-running: step {agree} differs at oracle margin {m['margins'][agree]:.3g}"
