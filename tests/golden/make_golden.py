"""Write the golden fixtures under tests/golden/ from the numpy oracle (run on the CPU, once).

The reference repository ships no golden vectors for this path, so these fixtures are the oracle's own
outputs on seeded BASELINE-config inputs; tests/test_oracle.py pins the oracle functions they come from.
Large operands are not stored: they are regenerated from their seeds and checked by checksum.

  python tests/golden/make_golden.py            # small fixtures (seconds)
  python tests/golden/make_golden.py --config2  # + 256 greedy tokens of the full config-2 model (minutes)
"""
from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "3080lab_amd"))

from lab import qwen_model as QM  # noqa: E402  (seeded weight generator = the inputs)
from oracle import model as OM  # noqa: E402
from oracle import quant as OQ  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config0_inputs():
    """W [8960, 1536] N(0, 0.02) and x [1536] N(0, 1) from seed 0."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((8960, 1536), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal((1, 1536), dtype=np.float32)
    return w, x


def small():
    out = {}
    # quantizer vectors (inputs included: small)
    rng = np.random.default_rng(11)
    xq = rng.standard_normal((4, 256), dtype=np.float32) * np.float32(3.0)
    xq[0, :32] = 0
    xq[1, 32:64] = np.float32(0.25) * np.arange(32)
    q, d, s = OQ.quantize_q8_1(xq)
    xw = rng.standard_normal((16, 64), dtype=np.float32) * np.float32(0.02)
    np.savez_compressed(HERE / "quant_vectors.npz", q8_x=xq, q8_q=q, q8_d=d, q8_s=s,
                        q4_x=xw, q4_bytes=OQ.quantize_q4_0(xw))
    # config 0 GEMV: outputs + checksums of the regenerated operands
    w, x = config0_inputs()
    wb = OQ.quantize_q4_0(w)
    qx, dx, sx = OQ.quantize_q8_1(x)
    y = OQ.gemv_q4_0_q8_1(wb, 8960, 1536, qx, dx)
    dots = OQ.block_dots(OQ.q4_0_blocks(wb)[1].reshape(8960, 1536), qx)
    np.savez_compressed(HERE / "config0_gemv.npz", y=y, qx=qx, dx=dx, sx=sx, dots_row0=dots[0, 0],
                        dots_sum=np.array([int(dots.astype(np.int64).sum())]))
    out["config0"] = {"w_q4_0_sha256": sha(wb), "dots_sha256": sha(dots)}
    # small 2-layer model greedy decode (the GPU test regenerates the weights from the seed)
    cfg = QM.Config(L=2, V=4096)
    wts = QM.random_weights(cfg, seed=21)
    m = OM.Model(OM.Config(L=2, V=4096), wts, maxlen=512)
    prompt = [int(t) for t in np.random.default_rng(22).integers(0, 4096, 8)]
    toks, margins = m.greedy(prompt, 24)
    out["small_model"] = {"cfg": {"L": 2, "V": 4096}, "seed": 21, "prompt": prompt, "tokens": toks,
                          "margins": margins, "embed_sha256": sha(wts["embed"])}
    return out


def config2(n_gen: int = 256):
    """full 28-layer model (seed 0), 128 uniform prompt ids (seed 1), 256 greedy tokens."""
    t0 = time.time()
    w = QM.random_weights(QM.QWEN15, seed=0)
    m = OM.Model(OM.Config(), w, maxlen=128 + n_gen + 8, mode="f64")
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, 151936, 128)]
    toks, margins = m.greedy(prompt, n_gen)
    return {"seed": 0, "prompt_seed": 1, "prompt": prompt, "tokens": toks, "margins": margins,
            "embed_sha256": sha(w["embed"]), "layer0_wq_sha256": sha(w["layers"][0]["wq"]),
            "seconds": round(time.time() - t0, 1)}


if __name__ == "__main__":
    meta_path = HERE / "golden.json"
    meta = json.loads(meta_path.read_text()) if meta_path.exists() else {}
    meta.update(small())
    if "--config2" in sys.argv:
        meta["config2"] = config2()
    meta_path.write_text(json.dumps(meta, indent=1))
    print("wrote", meta_path)
