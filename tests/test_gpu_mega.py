"""GPU checks of the persistent whole-step decode (q355_mega_decode) against the graph-of-kernels decoder
and the oracle."""
import numpy as np
import pytest

from lab import qwen_mega as QG
from lab import qwen_model as QM
from oracle import model as OM

pytestmark = pytest.mark.gpu
NEAR_TIE = 1e-2
CFG_S = QM.Config(L=2, V=4096)


@pytest.fixture(scope="module")
def small(cuda):
    w = QM.random_weights(CFG_S, seed=21)
    return w, QM.DeviceModel(w, CFG_S, maxlen=1024), OM.Model(OM.Config(L=2, V=4096), w, maxlen=512)


def test_mega_step_matches_graph_step(small):
    """Same prompt through both decoders: logits agree to f64 rounding (~1e-9) at every step, tokens equal."""
    w, dm, om = small
    prompt = [int(t) for t in np.random.default_rng(22).integers(0, CFG_S.V, 8)]
    a = QM.Decoder(dm, T=1, max_ctx=256)
    b = QG.MegaDecoder(dm, max_ctx=256)
    for t in prompt:
        a.tok.fill_(t)
        b.tok.fill_(t)
        a.step()
        b.step()
        la, lb = a.logits[0].cpu().numpy(), b.logits[0].cpu().numpy()
        assert b.error() == 0
        assert np.abs(la - lb).max() <= 1e-6 * np.abs(la).max()
        assert int(a.tok.item()) == int(b.tok.item())
        assert int(a.pos.item()) == int(b.pos.item())
    assert np.abs(a.h_f64().cpu().numpy() - b.h_f64().cpu().numpy()).max() < 1e-9


@pytest.mark.parametrize("pos", [300, 700])
def test_mega_matches_graph_over_many_pages(small, pos):
    """Contexts of several pages (5 and 11 at the first step: the short and the general partial merge): caches
    filled with the same N(0, 1) rows, then 4 steps of both decoders; logits to f64 rounding, tokens equal."""
    import torch
    w, dm, om = small
    a = QM.Decoder(dm, T=1, max_ctx=1024)
    b = QG.MegaDecoder(dm, max_ctx=1024)
    g = torch.Generator(device="cuda").manual_seed(pos)
    for i in range(CFG_S.L):
        a.kc[i].normal_(generator=g)
        a.vc[i].normal_(generator=g)
        b.kc[i].copy_(a.kc[i])
        b.vc[i].copy_(a.vc[i])
    for d in (a, b):
        d.pos.fill_(pos)
        d.tok.fill_(77)
    for _ in range(4):
        a.step()
        b.step()
        la, lb = a.logits[0].cpu().numpy(), b.logits[0].cpu().numpy()
        assert b.error() == 0
        assert np.abs(la - lb).max() <= 1e-6 * np.abs(la).max()
        assert int(a.tok.item()) == int(b.tok.item()) and int(a.pos.item()) == int(b.pos.item())
    assert np.abs(a.h_f64().cpu().numpy() - b.h_f64().cpu().numpy()).max() < 1e-9


def test_mega_greedy_matches_oracle(small):
    """Greedy decode through graph replays of the persistent step, 70-token prompt (two KV pages)."""
    w, dm, om = small
    prompt = list(np.random.default_rng(23).integers(0, CFG_S.V, 70))
    dec = QG.MegaDecoder(dm, max_ctx=256)
    dec.prefill_tokens(prompt)
    got = dec.generate(16)[0]
    assert dec.error() == 0
    ref, margins = om.greedy(prompt, 16)
    for i, (x, y) in enumerate(zip(got, ref)):
        if margins[i] < NEAR_TIE:
            break
        assert x == y, f"token {i}: {x} vs {y} (margin {margins[i]:.3g})"


def test_mega_with_q6k_head_matches_graph(small):
    """llama.cpp's Q6_K output.weight: the persistent launch runs the layers, the Q6_K head and the argmax follow
    as two launches; logits and tokens equal the graph decoder's, also under graph capture (generate)."""
    from ggufio import random_q6_k
    w, _, _ = small
    w = dict(w)
    w["head_q6k"] = random_q6_k(CFG_S.V * CFG_S.H // 256, np.random.default_rng(24), d=0.0005)
    dm = QM.DeviceModel(w, CFG_S, maxlen=512)
    prompt = [int(t) for t in np.random.default_rng(25).integers(0, CFG_S.V, 6)]
    a = QM.Decoder(dm, T=1, max_ctx=256)
    b = QG.MegaDecoder(dm, max_ctx=256)
    for t in prompt:
        a.tok.fill_(t)
        b.tok.fill_(t)
        a.step()
        b.step()
        la, lb = a.logits[0].cpu().numpy(), b.logits[0].cpu().numpy()
        assert np.abs(la - lb).max() <= 1e-6 * np.abs(la).max()
        assert int(a.tok.item()) == int(b.tok.item()) and int(a.pos.item()) == int(b.pos.item())
    assert (a.generate(8) == b.generate(8)).all()


def test_mega_rejects_position_past_cache(small):
    """pos beyond the cache: the launch returns at once with the error word set (no out-of-range access), and
    step() raises."""
    from lab.hip import HipError
    w, dm, om = small
    dec = QG.MegaDecoder(dm, max_ctx=128)
    dec.pos.fill_(128)
    with pytest.raises(HipError, match="error word"):
        dec.step()
    assert dec.error() != 0
    assert int(dec.pos.item()) == 128


def test_mega_source_spec():
    assert QG.mega_source(28, 2048).symbol == "q355_mega_decode"
    with pytest.raises(ValueError):
        QG.mega_source(28, 2048, nw=64)
