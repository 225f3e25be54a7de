"""q355_attn_decode_noalloc (split partials in the library's fixed device array) against q355_attn_decode with
fp32 = 1 and a caller-allocated partials buffer: bit-equal Q8_1 codes, scales and fp32 outputs, on two calls in a
row, the second with fewer tokens and a shorter context, and a rejected oversize call."""
import math

import numpy as np
import pytest

from lab.hip import HipError, call, ptr

pytestmark = pytest.mark.gpu


def _outs(torch, cuda, T, nh):
    return (torch.zeros(T, nh * 128, dtype=torch.int8, device=cuda),
            torch.zeros(T, nh * 4, 2, dtype=torch.float16, device=cuda),
            torch.zeros(T, nh * 128, device=cuda))


def test_attn_decode_noalloc_matches_allocating_entry(cuda):
    import torch
    nh, nkv, mc = 12, 2, 32
    rng = np.random.default_rng(41)
    Tmax = 32
    kc = torch.from_numpy(rng.standard_normal((Tmax * mc, nkv, 64, 128)).astype(np.float16)).to(cuda)
    vc = torch.from_numpy(rng.standard_normal((Tmax * mc, nkv, 64, 128)).astype(np.float16)).to(cuda)
    bt = torch.from_numpy(rng.permutation(Tmax * mc).astype(np.int32).reshape(Tmax, mc)).to(cuda)
    q = torch.from_numpy(rng.standard_normal((Tmax, nh * 128)).astype(np.float16)).to(cuda)
    part = torch.empty(Tmax, nh, mc, 130, dtype=torch.float64, device=cuda)
    scale = 1 / math.sqrt(128)
    assert call("q355_attn_decode_noalloc_max_bytes") == 4 << 20
    # first call: 32 tokens with contexts up to the 2048 of BASELINE config 3 (8 splits); second: 5 tokens, 12 pages
    for T, m, positions in [(32, mc, rng.integers(0, 64 * mc, 32)), (5, 12, [0, 63, 64, 700, 767])]:
        pos = torch.tensor(np.asarray(positions, np.int32), device=cuda)
        oq_a, ods_a, o32_a = _outs(torch, cuda, T, nh)
        oq_b, ods_b, o32_b = _outs(torch, cuda, T, nh)
        call("q355_attn_decode", ptr(q), ptr(kc), ptr(vc), ptr(pos), ptr(bt), mc, nh, nkv, m, scale, ptr(part),
             ptr(oq_a), ptr(ods_a), ptr(o32_a), T, 1)
        call("q355_attn_decode_noalloc", ptr(q), ptr(kc), ptr(vc), ptr(pos), ptr(bt), mc, nh, nkv, m, scale,
             ptr(oq_b), ptr(ods_b), ptr(o32_b), T)
        torch.cuda.synchronize()
        assert torch.equal(oq_a, oq_b), T
        assert torch.equal(ods_a.view(torch.int16), ods_b.view(torch.int16)), T
        assert torch.equal(o32_a.view(torch.int32), o32_b.view(torch.int32)), T
    # beyond the fixed scratch: rejected before any launch
    # (100 tokens x 12 heads x 8 splits x 520 B = 4.99 MB > 4 MiB; the size check precedes every launch)
    # (its own buffers sized for 100 tokens, so the call stays in bounds whatever order the checks run in)
    T = 100
    qT = torch.zeros(T, nh * 128, dtype=torch.float16, device=cuda)
    posT = torch.zeros(T, dtype=torch.int32, device=cuda)
    btT = torch.zeros(T, mc, dtype=torch.int32, device=cuda)
    oq_c, ods_c, o32_c = _outs(torch, cuda, T, nh)
    with pytest.raises(HipError, match="scratch"):
        call("q355_attn_decode_noalloc", ptr(qT), ptr(kc), ptr(vc), ptr(posT), ptr(btT), mc, nh, nkv, mc, scale,
             ptr(oq_c), ptr(ods_c), ptr(o32_c), T)
