"""The paired harness's in-process arms on a small model: every arm returns a positive throughput and the
graph and persistent arms leave the decoders on the same tokens."""
import numpy as np
import pytest

from lab import paired as PA
from lab import qwen_model as QM

pytestmark = pytest.mark.gpu


def test_decode_arms_two_rounds(cuda):
    cfg = QM.Config(L=2, V=4096)        # the persistent step needs V >= 4096
    dm = QM.DeviceModel(QM.random_weights(cfg, seed=3), cfg, maxlen=256)
    prompt = np.random.default_rng(2).integers(0, cfg.V, 20)
    arms = PA.decode_arms(dm, prompt, steps=8, batch=0)
    raw = PA.collect(arms, 2)
    res, table = PA.summarize(raw, PA.DECODE_PAIRS)
    assert set(res) == {"A/A: graph_dup / graph", "mega / graph"}
    for rec in raw["rounds"]:
        assert all(rec[a]["tg_b1"] > 0 for a in ("graph", "graph_dup", "mega"))
