"""Benchmark of the MI355X Qwen2.5 Q4_0 hot path (BASELINE.json metric:
"decode tok/s at batch 1/8/32 (Qwen2.5-1.5B-shape Q4_0); GEMV HBM GB/s").

  python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--no-cpu] [--quick] [--prefill-only]

Workload: the full 28-layer Qwen2.5-1.5B-shape model with random weights
(seeded, fp32 N(0, 0.02) quantized to Q4_0; tied Q4_0 embedding/head), a 128-token prompt of
uniform random ids, then greedy decode at batch 1 as one hipGraph-captured step per token. A step
is one decode token; `value` = tokens / second over the K timed steps (positions 128..128+K-1),
weights and KV cache resident in HBM.

Printed on one JSON line, besides the contract fields:
  roofline      the dominant kernel (gate_up GEMV with fused RMSNorm and SwiGLU; 35 % of the
                reference's decode time), algorithmic bytes / its average duration measured with
                HIP events on the launch stream, cycling the 28 layers' distinct weights (434 MB > MALL)
  gemv          BASELINE config 0: the 8960 x 1536 Q4_0 x Q8_1 GEMV, cold (64 distinct weight copies,
                495 MB) and hot-MALL, GB/s of algorithmic bytes (7,779,008 B per call)
  batched       BASELINE config 3 at B = 8 and 32 on the config's int8 MMQ (Q4_0 x Q8_1), tok/s
  batched_f16   the same batches in the reference's own batched arithmetic (fp16-dequantized Q4_0 x fp16)
  prefill       BASELINE config 4: one 2048-token prompt, tok/s
  cpu_baseline  the numpy oracle (exact int32 block-dot form, one core) timed on this host for a few
                decode steps of the same model, tok/s
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "3080lab_amd"))

HBM_PEAK_GBS = 8000.0
GEMV0_BYTES = 6_881_280 + 860_160 + 1_728 + 35_840     # config 0: nibbles + scales + Q8_1 x + fp32 y
# HBM bytes per launch of the roofline kernel come from the committed rocprofv3 PMC summary (counters cannot be
# read from inside this process): FETCH_SIZE and WRITE_SIZE KiB per dispatch, each scaled by what the same counter
# reads for a 64 MiB device-to-device copy (see the command lines at the top of that file).
TRAFFIC_PROFILE = ROOT / "profiles" / "decode_gemv_hbm_traffic_pmc.txt"
ROOFLINE_KERNEL = "k_gemv<1, 5, 4, 3, 1, 4, 0>"       # q355_ffn_gate_up


def traffic_from_profile(kernel: str = ROOFLINE_KERNEL, path: Path = TRAFFIC_PROFILE):
    """HBM bytes per dispatch of `kernel` from the PMC summary: FETCH_SIZE * (64 MiB / copy FETCH_SIZE) +
    WRITE_SIZE * (64 MiB / copy WRITE_SIZE). None if the summary does not hold the kernel."""
    if not path.exists():
        return None
    vals, section = {}, None
    for line in path.read_text().splitlines():
        if line.startswith("pmc_"):
            section = line.split("/")[0]                 # pmc_dec_FETCH_SIZE, pmc_copy_WRITE_SIZE, ...
            continue
        parts = line.split()
        if section and len(parts) >= 6 and parts[0] in ("FETCH_SIZE", "WRITE_SIZE") and "mean" in parts:
            kib = float(parts[parts.index("mean") + 1])
            name = line.split("KiB", 1)[1].strip()
            if section.startswith("pmc_copy") and "copyBuffer" in name:
                vals[(section, "copy")] = kib
            elif section.startswith("pmc_dec") and kernel in name:
                vals[(section, "kernel")] = kib
    need = [("pmc_dec_FETCH_SIZE", "kernel"), ("pmc_dec_WRITE_SIZE", "kernel"),
            ("pmc_copy_FETCH_SIZE", "copy"), ("pmc_copy_WRITE_SIZE", "copy")]
    if any(k not in vals for k in need):
        return None
    mib64 = 64.0 * 1024
    fetch = vals[need[0]] * mib64 / vals[need[2]]
    write = vals[need[1]] * mib64 / vals[need[3]]
    return int(round((fetch + write) * 1024))


KSTATS_PROFILE = ROOT / "profiles" / "bench_kernel_stats_rocprofv3.txt"


def profile_avg_us(kernel: str = ROOFLINE_KERNEL, path: Path = KSTATS_PROFILE):
    """Average duration (us) of `kernel` in the committed rocprofv3 --kernel-trace --stats summary of this
    command, or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 6 and not line.startswith("#") and kernel in line:
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_launches(fn, n: int, reps: int = 20) -> float:
    """Average ms per launch of fn(0..n-1), captured back to back in one hipGraph and replayed `reps` times,
    timed with HIP events on the launch stream (the same per-launch duration rocprofv3 reports, plus the
    graph's inter-node gap)."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (reps * n)


def gate_up_roofline(dm, dec) -> dict:
    from lab.hip import call, ptr
    c = dm.cfg
    gu0 = dm.layers[0]["gu"]
    algo = gu0.nbytes + c.H * 8 + c.H * 4 + c.FFN * 4     # weights + h (int64) + ln2 + m (fp32)

    def run(i):
        L = dm.layers[i % c.L]
        g = L["gu"]
        call("q355_ffn_gate_up", ptr(g.qs), ptr(g.d), g.N, g.K, ptr(dec.h), ptr(L["ln2"]), c.eps,
             ptr(dec.mlp), 1)
    ms = time_launches(run, c.L)
    ach = algo / (ms * 1e-3) / 1e9
    # the same kernel's average in the committed rocprofv3 summary of this command (traced: each dispatch
    # carries the profiler's per-dispatch work, so it reads longer than the live HIP-event figure)
    pus = profile_avg_us()
    # the practical ceiling for a stream of this size launched this way: a pure streaming read of the same
    # bytes from 28 distinct buffers (435 MB: more than the 256 MB Infinity Cache), one graph of 28 launches
    import torch
    bufs = [torch.ones(algo // 16 * 4, dtype=torch.int32, device="cuda") for _ in range(c.L)]
    sms = time_launches(lambda i: call("q355_stream_read", ptr(bufs[i]), bufs[i].numel() * 4), c.L)
    ceil = bufs[0].numel() * 4 / (sms * 1e-3) / 1e9
    del bufs
    torch.cuda.empty_cache()
    return {"kernel": "q355_ffn_gate_up (k_gemv<1,5,4,3,PRO_RMS,EPI_SWIGLU>)", "bound": "hbm",
            "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profile(), "traffic_source": str(TRAFFIC_PROFILE.relative_to(ROOT)),
            "algorithmic_bytes": int(algo), "avg_us": round(ms * 1e3, 3),
            "profile_avg_us": pus, "profile_source": str(KSTATS_PROFILE.relative_to(ROOT)),
            "frac_profile": round(algo / (pus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if pus else None,
            "same_size_stream": {"us": round(sms * 1e3, 3), "GBps": round(ceil, 1),
                                 "frac_of_peak": round(ceil / HBM_PEAK_GBS, 4), "achieved_over_it": round(ach / ceil, 4)}}


def gemv_config0(copies: int = 64) -> dict:
    import torch
    from lab import gguf
    from lab import qwen_model as QM
    from lab.hip import call, ptr
    N, K = 8960, 1536
    rng = np.random.default_rng(0)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    W0 = QM.Q4Mat(gguf.quantize_q4_0(w), N, K, "cuda")
    # distinct copies (same bytes, different addresses) defeat the 256 MB Infinity Cache
    qs = [W0.qs.clone() for _ in range(copies)]
    ds = [W0.d.clone() for _ in range(copies)]
    x = rng.standard_normal((1, K), dtype=np.float32)
    xt = torch.from_numpy(x).cuda()
    xq = torch.zeros(1, K, dtype=torch.int8, device="cuda")
    xds = torch.zeros(1, K // 32, 2, dtype=torch.float16, device="cuda")
    call("q355_quant_q8_1", ptr(xt), ptr(xq), ptr(xds), 1, K)
    y = torch.zeros(1, N, device="cuda")

    def run(i):
        j = i % copies
        call("q355_gemv_q4_0_q8_1", ptr(qs[j]), ptr(ds[j]), N, K, ptr(xq), ptr(xds), 1, ptr(y), None, 0)

    def run_hot(i):
        call("q355_gemv_q4_0_q8_1", ptr(qs[0]), ptr(ds[0]), N, K, ptr(xq), ptr(xds), 1, ptr(y), None, 0)
    cold = time_launches(run, copies)
    hot = time_launches(run_hot, copies)
    return {"shape": "8960x1536 Q4_0 x Q8_1, batch 1", "algorithmic_bytes": GEMV0_BYTES,
            "cold_us": round(cold * 1e3, 3), "cold_GBps": round(GEMV0_BYTES / (cold * 1e-3) / 1e9, 1),
            "hot_mall_us": round(hot * 1e3, 3), "hot_mall_GBps": round(GEMV0_BYTES / (hot * 1e-3) / 1e9, 1),
            "weight_copies": copies}


def batched_decode(dm, B: int, steps: int = 32, warmup: int = 2, act: str = "q8") -> dict:
    """B sequences with contexts uniform in [256, 2048] (seed 3), paged fp16 KV filled
    with N(0, 1), one hipGraph per step. act "q8": the config's Q4_0 x Q8_1 int8 MMQ on MFMA; act "f16":
    the reference's own batched arithmetic (fp16-dequantized Q4_0 x fp16 activations on the fp16 matrix
    cores, gemv_v2_source). tok/s = B * steps / time."""
    import torch
    from lab import qwen_batched as QB
    rng = np.random.default_rng(3)
    ctx = rng.integers(256, 2049, B)
    bd = QB.BatchedDecoder(dm, B=B, max_ctx=2048 + warmup + steps + 1, page_seed=B, act=act)
    bd.fill_random_context(ctx, seed=B)
    bd.tok.copy_(torch.from_numpy(rng.integers(0, dm.cfg.V, B).astype(np.int32)))
    pos0, tok0 = bd.pos.clone(), bd.tok.clone()
    g = bd.capture()
    for _ in range(warmup):
        g.replay()
    bd.pos.copy_(pos0)
    bd.tok.copy_(tok0)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    kv = int(28_672 * (ctx.sum() + B * steps / 2))          # mean K+V bytes read per step
    wbytes = dm.weight_bytes_per_token()
    out = {"B": B, "act": act, "tok_per_s": round(B * 1e3 / ms, 1), "ms_per_step": round(ms, 4),
           "ctx_mean": float(ctx.mean()), "bytes_per_step": wbytes + kv,
           "hbm_GBps": round((wbytes + kv) / (ms * 1e-3) / 1e9, 1)}
    del bd
    torch.cuda.empty_cache()
    return out


def prefill(dm, P: int = 2048, reps: int = 3) -> dict:
    """one 2048-token prompt (uniform ids, seed 4) through the chunked prefill path
    (int8 MFMA MMQ GEMMs at M = P, causal fp16-MFMA flash attention), one chunk; tok/s = P / time."""
    import torch
    from lab import qwen_batched as QB
    from lab import qwen_model as QM
    c = dm.cfg
    dec = QM.Decoder(dm, T=1, max_ctx=P + 64)
    pf = QB.Prefill(dec, max_chunk=P)
    ids = np.random.default_rng(4).integers(0, c.V, P)
    pf.chunk(ids, 0)                                   # warm-up (also sets ids / positions)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        pf.enqueue(P, 0)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    gemm_ops = 2 * P * (c.nqkv * c.H + c.H * c.NH * c.HD + 2 * c.FFN * c.H + c.H * c.FFN) * c.L
    attn_flop = 4 * c.NH * c.HD * (P * (P + 1) // 2) * c.L
    out = {"P": P, "tok_per_s": round(P * 1e3 / ms, 1), "ms": round(ms, 3), "gemm_ops": gemm_ops,
           "attn_flop": attn_flop, "effective_TOPS": round((gemm_ops + attn_flop) / (ms * 1e-3) / 1e12, 1)}
    del pf, dec
    torch.cuda.empty_cache()
    return out


def cpu_baseline(w, cfg, prompt, n_steps: int = 4) -> dict:
    """The oracle (oracle/model.py, exact int32 block-dot mode, numpy, one core) on the same workload as the GPU
    line: the 128-token prompt is run through the oracle's float64 form (untimed; it fills the same K/V cache),
    then n_steps greedy decode steps at positions 128.. are timed in int32 block-dot mode; tok/s =
    n_steps / wall time. Also times BASELINE config 0 (one 8960 x 1536 GEMV) and config 1 (one decoder layer
    at 512 past positions) in the same mode, median of 3 after one warm-up."""
    sys.path.insert(0, str(ROOT))
    from oracle import model as OM
    from oracle import quant as OQ
    ocfg = OM.Config(**{k: getattr(cfg, k) for k in ("H", "NH", "NKV", "HD", "FFN", "L", "V", "eps", "theta")})
    P = len(prompt)
    m64 = OM.Model(ocfg, w, maxlen=P + n_steps + 8, mode="f64")
    cache = m64.new_cache()
    h = m64.forward([int(t) for t in prompt], 0, cache)
    tok = int(np.argmax(m64.logits(h[-1:])[0]))
    del m64
    m = OM.Model(ocfg, w, maxlen=P + n_steps + 8, mode="int")
    t0 = time.perf_counter()
    for s in range(n_steps):
        h = m.forward([tok], P + s, cache)
        tok = int(np.argmax(m.logits(h)[0]))
    dt = time.perf_counter() - t0

    def med(fn, n=3):
        fn()
        ts = []
        for _ in range(n):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return float(np.median(ts))
    # config 0: one GEMV, int32 block-dot form
    rng = np.random.default_rng(0)
    w0 = rng.standard_normal((8960, 1536), dtype=np.float32) * np.float32(0.02)
    wb0 = OQ.quantize_q4_0(w0)
    qx, dx, _ = OQ.quantize_q8_1(rng.standard_normal((1, 1536), dtype=np.float32))
    t_gemv = med(lambda: OQ.gemv_q4_0_q8_1(wb0, 8960, 1536, qx, dx))
    # config 1: one layer at 512 past positions (K/V filled with N(0, 1))
    m1 = OM.Model(OM.Config(L=1, V=cfg.V), {"embed": w["embed"], "norm": w["norm"], "layers": w["layers"][:1]},
                  maxlen=520, mode="int")
    c1 = m1.new_cache()
    kv = np.random.default_rng(5).standard_normal((2, 1, cfg.NKV, 512, cfg.HD)).astype(np.float16)
    c1["K"][:, :, :512], c1["V"][:, :, :512] = kv[0], kv[1]
    h1 = np.random.default_rng(6).standard_normal((1, cfg.H))
    t_layer = med(lambda: m1.layer(0, h1, 512, c1))
    return {"value": round(n_steps / dt, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n_steps} greedy decode steps of the config-2 model (28 layers + tied head) at positions "
                      f"{P}..{P + n_steps - 1} after the same {P}-token prompt, oracle/model.py in int32 block-dot "
                      f"mode, single-threaded numpy, {dt:.1f} s; host os.cpu_count()={os.cpu_count()}",
            "config0_gemv": {"us": round(t_gemv * 1e6, 1),
                             "GBps": round(GEMV0_BYTES / t_gemv / 1e9, 3), "cores": 1},
            "config1_layer": {"us": round(t_layer * 1e6, 1), "past_positions": 512, "cores": 1}}


def paired(args):
    """Paired A/B rounds (scripts/decode_paired.py protocol) over the config-2 model: arms graph, graph_dup
    (A/A control), mega and batched (B = 8), `args.steps` tokens each per round."""
    from lab import paired as PA
    from lab import qwen_model as QM
    cfg = QM.QWEN15
    w = QM.random_weights(cfg, seed=0)
    dm = QM.DeviceModel(w, cfg, maxlen=2048 + 64)
    prompt = np.random.default_rng(1).integers(0, cfg.V, 128)
    arms = PA.decode_arms(dm, prompt, steps=args.steps)
    if args.llama_bench:
        arms["llama"] = PA.llama_bench_arm(*args.llama_bench)
    for a in arms.values():                 # warm-up pass (caches, clocks), not recorded
        a()
    raw = PA.collect(arms, args.paired, log=log)
    res, table = PA.summarize(raw, PA.DECODE_PAIRS)
    log(table)
    print(json.dumps({"paired": res, "steps_per_arm": args.steps, "raw": raw}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--quick", action="store_true", help="decode only (no roofline / GEMV / CPU legs)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 64 MiB device-to-device copy 4 times (HBM counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-4 prefill leg (for rocprofv3 MFMA counters), one JSON line")
    ap.add_argument("--paired", type=int, default=0, metavar="ROUNDS",
                    help="instead of the contract line: paired A/B rounds (graph vs persistent step, A/A control, "
                         "batched B=8), one JSON line of ratio statistics")
    ap.add_argument("--llama-bench", nargs=2, metavar=("BINARY", "GGUF"),
                    help="with --paired: add an external llama.cpp llama-bench arm")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              f"(the decode path is single-GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import torch
    from lab import qwen_model as QM
    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    if args.copy_probe:
        src = torch.ones(16 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4}))
        return
    if args.paired:
        paired(args)
        return
    cfg = QM.QWEN15
    t0 = time.time()
    w = QM.random_weights(cfg, seed=0)
    log(f"weights generated in {time.time() - t0:.1f} s")
    if args.prefill_only:
        dm = QM.DeviceModel(w, cfg, maxlen=2048 + 64)
        print(json.dumps({"prefill": prefill(dm)}), flush=True)
        return
    prompt_len = 128
    maxlen = prompt_len + args.warmup + args.steps + 64
    dm = QM.DeviceModel(w, cfg, maxlen=max(2048 + 64, maxlen))
    dec = QM.Decoder(dm, T=1, max_ctx=max(512, maxlen))
    prompt = np.random.default_rng(1).integers(0, cfg.V, prompt_len)
    t0 = time.time()
    dec.prefill_tokens(prompt)
    torch.cuda.synchronize()
    log(f"prompt ({prompt_len} tokens, token by token) in {time.time() - t0:.2f} s")
    pos0, tok0 = dec.pos.clone(), dec.tok.clone()
    g = dec.capture()
    for _ in range(args.warmup):
        g.replay()
    dec.pos.copy_(pos0)
    dec.tok.copy_(tok0)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    tok_s = 1e3 / ms
    wb = dm.weight_bytes_per_token()
    kv = 28_672 * (prompt_len + args.steps / 2)             # mean fp16 K+V bytes read per token
    algo = wb + kv
    out = {"metric": "decode tok/s at batch 1/8/32 (Qwen2.5-1.5B-shape Q4_0); GEMV HBM GB/s",
           "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int4 x int8 -> int32 block dots, f64 accumulation (Q4_0 x Q8_1)", "data": "synthetic (seeded random weights and prompt)",
           "config": {"workload": "BASELINE config 2: Qwen2.5-1.5B-shape 28 layers, tied Q4_0 head, "
                                  "128-token prompt + greedy decode, batch 1, one hipGraph per token",
                      "batch": 1, "prompt_len": prompt_len, "decode_positions": [prompt_len, prompt_len + args.steps - 1],
                      "parallelism": "single GPU"},
           "decode_bytes_per_token": int(algo),
           "decode_hbm_GBps": round(algo / (ms * 1e-3) / 1e9, 1),
           "decode_roofline_frac": round(algo / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if not args.quick:
        out["batched"] = [batched_decode(dm, B) for B in (8, 32)]
        log("batched:", out["batched"])
        out["batched_f16"] = [batched_decode(dm, B, act="f16") for B in (8, 32)]
        log("batched_f16:", out["batched_f16"])
        out["prefill"] = prefill(dm)
        log("prefill:", out["prefill"])
        out["roofline"] = gate_up_roofline(dm, dec)
        out["gemv"] = gemv_config0()
        if not args.no_cpu:
            t0 = time.time()
            out["cpu_baseline"] = cpu_baseline(w, cfg, prompt)
            log(f"cpu baseline in {time.time() - t0:.1f} s")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
