"""The int8 batched path's f64 attention (q355_attn_decode_f64) against the oracle's float64 attention
(oracle/model.py:attn_decode, the semantics of ATTN4, lab/qwen_kernels.py:517-605).

f64 scores, softmax and P.V of the fp16 q/K/V: the fp32 output is the oracle's float64 result rounded once,
so it may differ from it by at most one fp32 ulp (2^-23 relative: the two f64 values, equal to ~1e-15, can
straddle an fp32 rounding boundary; written below as 1.2e-7 of the row's largest value), and the Q8_1 bytes equal the oracle's quantization of its own fp32 result
except where that rounding crosses a code boundary. Covered: GQA groups 4/6/8, contexts of 1 position to
64 pages (1 to 32 two-page splits, so the merge kernel's batches of 20 splits both single and double), pages
scattered through the pool, tokens of one launch with contexts that need and do not need the merge."""
import math

import numpy as np
import pytest

from lab.hip import call, ptr
from oracle import model as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu


def _run(cuda, nh, nkv, pos, mc, seed):
    import torch
    rng = np.random.default_rng(seed)
    T = len(pos)
    kc = rng.standard_normal((T * mc, nkv, 64, 128)).astype(np.float16)
    vc = rng.standard_normal((T * mc, nkv, 64, 128)).astype(np.float16)
    bt = rng.permutation(T * mc).astype(np.int32).reshape(T, mc)
    q = (rng.standard_normal((T, nh * 128)) * 2).astype(np.float16)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    part = torch.zeros(T, nh, mc, 130, dtype=torch.float64, device=cuda)
    oq = torch.zeros(T, nh * 128, dtype=torch.int8, device=cuda)
    ods = torch.zeros(T, nh * 4, 2, dtype=torch.float16, device=cuda)
    o32 = torch.zeros(T, nh * 128, device=cuda)
    keep = [d(q.astype(np.float64)), d(kc), d(vc), d(np.asarray(pos, np.int32)), d(bt)]   # alive until the sync
    call("q355_attn_decode_f64", *[ptr(t) for t in keep], mc, nh, nkv, mc, 1 / math.sqrt(128), ptr(part), ptr(oq),
         ptr(ods), ptr(o32), T)
    torch.cuda.synchronize()
    got, gq, gds = o32.cpu().numpy(), oq.cpu().numpy(), ods.cpu().numpy()
    # the same launch over the live-item list: bit-identical
    nsp = (mc + 1) // 2
    work = torch.zeros(call("q355_attn_f64_worklist_bytes", T, nkv, mc) // 4, dtype=torch.int32, device=cuda)
    assert work.numel() == nkv * nsp * T * 4 + T * nkv          # the items, then the arrival counters
    work[:nkv * nsp * T * 4] = -7                               # every item slot is rewritten
    call("q355_attn_f64_worklist", ptr(keep[3]), ptr(keep[4]), mc, nkv, mc, T, ptr(work))
    for t in (part, oq, ods, o32):
        t.zero_()
    for rep in range(2):                # up to 16 tokens the merge by the last split: its counters reset themselves
        call("q355_attn_decode_f64_wl", *[ptr(t) for t in keep], mc, nh, nkv, mc, 1 / math.sqrt(128), ptr(part),
             ptr(oq), ptr(ods), ptr(o32), T, ptr(work))
        torch.cuda.synchronize()
        assert np.array_equal(o32.cpu().numpy().view(np.uint32), got.view(np.uint32)), rep
        assert np.array_equal(oq.cpu().numpy(), gq), rep
        assert np.array_equal(ods.cpu().numpy().view(np.uint16), gds.view(np.uint16)), rep
        assert int(work[nkv * nsp * T * 4:].abs().sum()) == 0
        o32.zero_()
    w = work[:nkv * nsp * T * 4].cpu().numpy().reshape(-1, 4)
    live = [(j, k, sp) for sp in range(nsp) for j in range(T) for k in range(nkv) if sp <= int(pos[j]) // 128]
    assert len(w) == nkv * nsp * T and (w[len(live):, 0] == -1).all()
    assert [(x & 0xffff, (x >> 16) & 0xff, x >> 24) for x in w[:len(live), 0]] == live
    assert all(w[i, 1] == pos[j] and w[i, 2] == bt[j, min(2 * sp, mc - 1)] and w[i, 3] == bt[j, min(2 * sp + 1, mc - 1)]
               for i, (j, _, sp) in enumerate(live))
    for j in range(T):
        K = np.concatenate([kc[bt[j, p]] for p in range(mc)], axis=1)
        V = np.concatenate([vc[bt[j, p]] for p in range(mc)], axis=1)
        ref = OM.attn_decode(q[j].reshape(nh, 128), K, V, int(pos[j]) + 1, nh, nkv)
        err = np.abs(got[j] - ref).max() / np.abs(ref).max()
        assert err <= 1.2e-7, (nh, nkv, j, int(pos[j]), err)
        rq, rd, _ = OQ.quantize_q8_1(ref[None])
        assert (gq[j] == rq.reshape(-1)).mean() >= 0.999, j
        assert (gds[j][:, 0] == rd.reshape(-1)).mean() >= 0.99, j


def test_attn_f64_merge_launch_above_16_tokens(cuda):
    """20 tokens: the work-list launch merges in a separate launch (bit-identical all the same)."""
    _run(cuda, 12, 2, [(37 * j) % 900 for j in range(20)], 16, 77)


@pytest.mark.parametrize("nh,nkv", [(12, 2), (8, 2), (16, 2), (12, 3)])
def test_attn_f64_groups_and_splits(cuda, nh, nkv):
    """GQA 6 (the model), 4 and 8; contexts of 1, 64, 65 positions (one split: finished in the attention
    kernel), 129 and 1000 (2 and 8 splits, merged)."""
    _run(cuda, nh, nkv, [0, 63, 64, 128, 999], 16, nh * 10 + nkv)


def test_attn_f64_longest_context(cuda):
    """64 pages (4096 positions, 32 splits: two merge batches) beside a 1-position token."""
    _run(cuda, 12, 2, [64 * 64 - 1, 0, 20 * 128 + 5], 64, 64)


def test_attn_f64_batch_of_32(cuda):
    """BASELINE config 3's shape: 32 tokens, contexts uniform in [256, 2048]."""
    pos = np.random.default_rng(3).integers(256, 2049, 32)
    _run(cuda, 12, 2, list(pos), 33, 5)
