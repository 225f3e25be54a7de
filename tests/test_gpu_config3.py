"""BASELINE config 3 at its context range: batched decode of B = 8 and B = 32 sequences whose contexts are drawn
uniform in [256, 2048] (seed 3, as bench.py), on a paged fp16 KV cache with scattered pages, checked step by step
against the oracle in the matching arithmetic. Contexts of more than 256 positions make the attention split its
pages (up to 8 splits of 4 pages), so the split merge -- inside the O product's staging up to B = 16, in its own
launch above -- runs inside a real batched step. 2 layers at full width (H 1536, FFN 8960, 12/2 heads)."""
import numpy as np
import pytest

from lab import qwen_batched as QB
from lab import qwen_model as QM
from oracle import model as OM

pytestmark = pytest.mark.gpu
CFG = QM.Config(L=2, V=4096)
from test_gpu_mmq import logit_tol, token_margin   # the batched modes' bounds (q8: 1e-3 of max |logit|)
STEPS = 4


@pytest.fixture(scope="module")
def model(cuda):
    w = QM.random_weights(CFG, seed=33)
    return w, QM.DeviceModel(w, CFG, maxlen=2048 + 64)


def _oracle_cache(om, bd, b, ctx):
    """The oracle's contiguous cache for sequence b, filled from the GPU's pages (positions 0..ctx-1)."""
    cache = om.new_cache()
    bt = bd.block_table[b].cpu().numpy()
    for i in range(CFG.L):
        for name, src in (("K", bd.kc[i]), ("V", bd.vc[i])):
            pages = src[bt].cpu().numpy()                                  # [chunks, nkv, 64, hd]
            full = pages.transpose(1, 0, 2, 3).reshape(CFG.NKV, -1, CFG.HD)
            cache[name][i, :, :ctx] = full[:, :ctx]
    return cache


@pytest.mark.parametrize("act", ["q8", "f16"])
@pytest.mark.parametrize("B", [8, 32])
def test_config3_context_range(model, B, act):
    import torch
    w, dm = model
    om = OM.Model(OM.Config(L=2, V=CFG.V), w, maxlen=2048 + 16, act=act)
    rng = np.random.default_rng(3)
    ctx = rng.integers(256, 2049, B)
    toks = rng.integers(0, CFG.V, B).astype(np.int32)
    bd = QB.BatchedDecoder(dm, B=B, max_ctx=2048 + 16, page_seed=B, act=act, keep_logits=True)
    bd.fill_random_context(ctx, seed=B)
    seqs = sorted({int(np.argmax(ctx)), int(np.argmin(ctx)), 1, B - 1})
    caches = {s: _oracle_cache(om, bd, s, int(ctx[s])) for s in seqs}
    assert int(ctx.max()) > 1024 and int(ctx.min()) < 512          # several splits and short ones in one batch
    for t in range(STEPS):
        bd.tok.copy_(torch.from_numpy(toks))
        bd.step()
        got = bd.logits.cpu().numpy()
        for s in seqs:
            h = om.forward([int(toks[s])], int(ctx[s]) + t, caches[s])
            ref = om.logits(h)[0]
            dev = float(np.abs(got[s] - ref).max())
            assert dev <= logit_tol(act, ref), f"B={B} {act} seq {s} (ctx {ctx[s]}) step {t}: logits off by {dev:.3g}"
            top2 = np.partition(ref, -2)[-2:]
            if top2[1] - top2[0] >= token_margin(act):
                assert int(got[s].argmax()) == int(ref.argmax()), f"B={B} {act} seq {s} step {t}"
            toks[s] = int(ref.argmax())                                  # teacher forcing
        assert (bd.pos.cpu().numpy() == ctx + t + 1).all()
