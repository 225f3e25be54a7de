"""Full-size (BASELINE config 3 and 4 shapes, the 28-layer Qwen2.5-1.5B-shape model) checks through properties
that do not need an oracle run at that size:
- prefill of 2048 tokens in one chunk equals two chunks of 1024 (the second at pos0 = 1024) bit for bit: K/V
  cache of every layer, logits and next token;
- batched decode at B = 8 isolates its sequences: a slot's tokens and logits are bit-equal whatever its
  batch-mates hold.
(The fp32 batched and prefill paths are compared with the f64 batch-1 path at the small configuration, where
the oracle runs: over 28 layers of random weights their Q8_1 roundings diverge by more than a near-tie.)
"""
import numpy as np
import pytest

from lab import qwen_batched as QB
from lab import qwen_model as QM

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full(cuda):
    cfg = QM.QWEN15
    w = QM.random_weights(cfg, seed=0)
    return cfg, QM.DeviceModel(w, cfg, maxlen=2048 + 64)


def caches(dec, L, n):
    """K and V of positions 0 .. n - 1 of sequence 0 in logical order, per layer."""
    pages = dec.block_table[0, : (n + 63) // 64].cpu().numpy()
    out = []
    for i in range(L):
        k = dec.kc[i][pages].permute(1, 0, 2, 3).reshape(dec.kc[i].shape[1], -1, 128)[:, :n]
        v = dec.vc[i][pages].permute(1, 0, 2, 3).reshape(dec.vc[i].shape[1], -1, 128)[:, :n]
        out.append((k.float().cpu().numpy(), v.float().cpu().numpy()))
    return out


def test_config4_prefill_one_chunk_equals_two(full):
    import torch
    cfg, dm = full
    ids = np.random.default_rng(4).integers(0, cfg.V, 2048)
    a = QM.Decoder(dm, T=1, max_ctx=2048 + 64)
    QB.Prefill(a, max_chunk=2048).chunk(ids, 0)
    b = QM.Decoder(dm, T=1, max_ctx=2048 + 64)
    pb = QB.Prefill(b, max_chunk=1024)
    pb.chunk(ids[:1024], 0)
    pb.chunk(ids[1024:], 1024)
    torch.cuda.synchronize()
    assert int(a.pos.item()) == int(b.pos.item()) == 2048
    # every product of a >= 512-token chunk runs the LDS-tiled kernel and attention reads the cache: bit-equal
    for i, ((ka, va), (kb, vb)) in enumerate(zip(caches(a, cfg.L, 2048), caches(b, cfg.L, 2048))):
        assert np.array_equal(kb, ka) and np.array_equal(vb, va), f"layer {i}"
    assert int(a.tok.item()) == int(b.tok.item())
    assert np.array_equal(a.logits[0].cpu().numpy(), b.logits[0].cpu().numpy())


@pytest.mark.parametrize("act", ["q8", "f16"])
def test_config3_batch_isolation(full, act):
    """A sequence's tokens and logits do not depend on its batch-mates: two B = 8 batches that share the prompts
    of slots 0 and 5 (every other slot differs, and so do the random context lengths' neighbours) give those
    two slots the same 12 greedy tokens and bit-equal final logits."""
    cfg, dm = full
    B, steps = 8, 12
    rng = np.random.default_rng(6)
    p1 = rng.integers(0, cfg.V, (B, 16))
    p2 = rng.integers(0, cfg.V, (B, 16))
    p2[[0, 5]] = p1[[0, 5]]
    out = []
    for prompts in (p1, p2):
        bd = QB.BatchedDecoder(dm, B=B, max_ctx=128, page_seed=B, act=act, keep_logits=True)
        bd.prefill_tokens(prompts)
        toks = bd.generate(steps)
        out.append((toks, bd.logits.cpu().numpy()))
    for s_ in (0, 5):
        assert np.array_equal(out[0][0][s_], out[1][0][s_]), f"slot {s_}"
        assert np.array_equal(out[0][1][s_], out[1][1][s_]), f"slot {s_} logits"
