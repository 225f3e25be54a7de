"""Free-running greedy decode of BASELINE config 3's int8 batched path against the oracle: B = 8 sequences,
contexts uniform in [256, 2048] (seed 3, as bench.py), 2 layers at full width (H 1536, FFN 8960, 12/2 heads),
256 greedy steps with no teacher forcing (the reference's own check is greedy agreement, scripts/qwen_e2e.py:
240-243). The batched path has the oracle's arithmetic (f64 accumulation, f64 attention, fixed-point
residual); its logits differ only by the LM head's fp32 accumulation (~1e-7 relative), so every token must
agree until the first step whose oracle top-2 margin is below NEAR_TIE_EXACT (1e-5, a hundred times that
error); from there the two sequences may legitimately part. The run reports how many steps were checked."""
import numpy as np
import pytest

from lab import qwen_batched as QB
from lab import qwen_model as QM
from oracle import model as OM

pytestmark = pytest.mark.gpu
CFG = QM.Config(L=2, V=4096)
B, STEPS = 8, 256
NEAR_TIE_EXACT = 1e-5


def test_batched_free_running_256(cuda):
    import torch
    w = QM.random_weights(CFG, seed=3)
    maxlen = 2048 + STEPS + 64
    dm = QM.DeviceModel(w, CFG, maxlen=maxlen)
    om = OM.Model(OM.Config(L=2, V=CFG.V), w, maxlen=maxlen)
    rng = np.random.default_rng(3)
    ctx = rng.integers(256, 2049, B)
    tok0 = rng.integers(0, CFG.V, B).astype(np.int32)
    bd = QB.BatchedDecoder(dm, B=B, max_ctx=2048 + STEPS + 16, page_seed=B)
    bd.fill_random_context(ctx, seed=B)
    caches = []
    for b in range(B):                                   # the oracle's contiguous caches, from the GPU's pages
        cache = om.new_cache()
        bt = bd.block_table[b].cpu().numpy()
        for i in range(CFG.L):
            for name, src in (("K", bd.kc[i]), ("V", bd.vc[i])):
                full = src[bt].cpu().numpy().transpose(1, 0, 2, 3).reshape(CFG.NKV, -1, CFG.HD)
                cache[name][i, :, :ctx[b]] = full[:, :ctx[b]]
        caches.append(cache)
    bd.tok.copy_(torch.from_numpy(tok0))
    got = bd.generate(STEPS + 1)                         # [B, STEPS + 1]: column 0 is tok0
    toks = tok0.copy()
    margins = np.zeros((B, STEPS))
    ref = np.zeros((B, STEPS), np.int64)
    for t in range(STEPS):
        lg = om.logits(om.decode_batch(list(toks), list(ctx + t), caches))
        top2 = np.partition(lg, -2, axis=1)[:, -2:]
        margins[:, t] = top2[:, 1] - top2[:, 0]
        ref[:, t] = lg.argmax(axis=1)
        toks = ref[:, t].astype(np.int32)
    checked = 0
    for b in range(B):
        for t in range(STEPS):
            if margins[b, t] < NEAR_TIE_EXACT:
                break
            assert got[b, t + 1] == ref[b, t], (f"seq {b} step {t}: {got[b, t + 1]} vs {ref[b, t]} "
                                                f"(oracle margin {margins[b, t]:.3g})")
            checked += 1
    print(f"free-running: {checked} of {B * STEPS} tokens checked, smallest oracle margin {margins.min():.3g}")
    assert checked >= B * STEPS // 2
