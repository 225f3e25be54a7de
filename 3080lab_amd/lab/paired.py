"""Paired A/B measurement: rotated rounds with an A/A control and central estimates.

Follows the protocol of scripts/decode_paired.py:47-150 (reference). Each round runs every arm once. The
order is a seeded shuffle rotated by one position per round, so slow drift (clocks, temperature, a
background load) hits each arm at each position equally. One arm is run twice per round under two names
(`graph` and `graph_dup`); the ratio between them is the A/A noise floor of every other comparison.

Per pair (num, den) the statistic is the per-round ratio num/den of throughputs. The summary gives its
median over rounds, its min and max, and a bootstrap 95 % interval of the mean log ratio, reported as a
ratio (scripts/decode_paired.py:boot_ci, ratios, summarize).

Arms are callables returning {key: tok/s}. `decode_arms()` builds the in-process arms of this library:
- the batch-1 hipGraph step (`graph`, `graph_dup`);
- the persistent single-launch step (`mega`);
- batched decode at B = 8 (`batched`).
`llama_bench_arm(binary, gguf)` wraps an external llama.cpp `llama-bench` build when one exists on the
machine (the reference's comparison target; none is installed on this image).
"""
from __future__ import annotations

import json
import math
import random
import statistics
import subprocess
from typing import Callable, Dict, List, Sequence, Tuple

Arm = Callable[[], Dict[str, float]]


def round_orders(names: Sequence[str], rounds: int, seed: int = 0) -> List[List[str]]:
    """Arm order per round: one seeded shuffle, rotated left by r positions in round r
    (scripts/decode_paired.py:collect)."""
    base = list(names)
    random.Random(seed).shuffle(base)
    n = len(base)
    return [base[r % n:] + base[:r % n] for r in range(rounds)]


def collect(arms: Dict[str, Arm], rounds: int, seed: int = 0, log: Callable[[str], None] | None = None) -> dict:
    """Run every arm once per round in the rotated order; returns {"order_seed", "rounds": [{round, order,
    arm: result}]}."""
    raw = {"order_seed": seed, "rounds": []}
    for r, order in enumerate(round_orders(list(arms), rounds, seed)):
        rec = {"round": r, "order": order}
        for a in order:
            rec[a] = {k: float(v) for k, v in arms[a]().items()}
            if log:
                log(f"round {r} {a:10s} " + " ".join(f"{k}={v:.1f}" for k, v in rec[a].items()))
        raw["rounds"].append(rec)
    return raw


def ratios(rounds: Sequence[dict], num: Tuple[str, str], den: Tuple[str, str]) -> List[float]:
    """Per-round ratios rec[num arm][num key] / rec[den arm][den key]; rounds missing either side, or with a
    zero denominator, are skipped."""
    out = []
    for rec in rounds:
        a = rec.get(num[0], {}).get(num[1])
        b = rec.get(den[0], {}).get(den[1])
        if a and b:
            out.append(a / b)
    return out


def boot_ci(xs: Sequence[float], n: int = 4000, seed: int = 1) -> Tuple[float, float]:
    """Percentile bootstrap 95 % interval of the mean of xs (resampling with replacement, n resamples)."""
    rng = random.Random(seed)
    k = len(xs)
    ms = sorted(sum(rng.choices(xs, k=k)) / k for _ in range(n))
    return ms[int(0.025 * n)], ms[int(0.975 * n) - 1]


def pair_stats(rs: Sequence[float]) -> dict:
    """Median, min, max of the ratios and the bootstrap 95 % interval of exp(mean log ratio)."""
    logs = [math.log(x) for x in rs]
    lo, hi = boot_ci(logs)
    return {"n": len(rs), "median": statistics.median(rs), "min": min(rs), "max": max(rs),
            "gmean": math.exp(statistics.mean(logs)), "ci95": [math.exp(lo), math.exp(hi)]}


def summarize(raw: dict, pairs: Sequence[Tuple[str, Tuple[str, str], Tuple[str, str]]]) -> Tuple[dict, str]:
    """Statistics for each (label, num, den) pair with at least one round, as a dict and as a markdown table
    (medians of each side's throughput alongside the ratio statistics)."""
    R = raw["rounds"]
    res = {}
    lines = [f"{len(R)} rounds, order seed {raw.get('order_seed')}", "",
             "| pair | num (median tok/s) | den (median tok/s) | ratio median [min, max] | mean log ratio 95% CI |",
             "|---|---:|---:|---:|---:|"]
    for label, num, den in pairs:
        rs = ratios(R, num, den)
        if not rs:
            continue
        st = pair_stats(rs)
        st["num_median"] = statistics.median([r[num[0]][num[1]] for r in R if num[1] in r.get(num[0], {})])
        st["den_median"] = statistics.median([r[den[0]][den[1]] for r in R if den[1] in r.get(den[0], {})])
        res[label] = st
        lines.append(f"| {label} | {st['num_median']:.1f} | {st['den_median']:.1f} | {st['median']:.4f} "
                     f"[{st['min']:.4f}, {st['max']:.4f}] | [{st['ci95'][0]:.4f}, {st['ci95'][1]:.4f}] |")
    return res, "\n".join(lines)


DECODE_PAIRS = [("A/A: graph_dup / graph", ("graph_dup", "tg_b1"), ("graph", "tg_b1")),
                ("mega / graph", ("mega", "tg_b1"), ("graph", "tg_b1")),
                ("llama.cpp / graph", ("llama", "tg_b1"), ("graph", "tg_b1"))]


def decode_arms(dm, prompt, steps: int = 128, batch: int = 8) -> Dict[str, Arm]:
    """In-process arms over one DeviceModel. Each decode arm restores the same state (the prompt's KV cache,
    token and position) and times `steps` greedy tokens with HIP events; the graph arms share one captured
    graph, so `graph_dup` differs from `graph` only by when it runs."""
    import numpy as np
    import torch
    from . import qwen_batched as QB
    from . import qwen_mega as QG
    from . import qwen_model as QM

    maxlen = len(prompt) + steps + 8
    dec = QM.Decoder(dm, T=1, max_ctx=maxlen)
    dec.prefill_tokens(prompt)
    g = dec.capture()
    mg = QG.MegaDecoder(dm, max_ctx=maxlen)
    mg.prefill_tokens(prompt)
    torch.cuda.synchronize()
    state = {id(d): (d.pos.clone(), d.tok.clone()) for d in (dec, mg)}

    def timed(d, run):
        pos0, tok0 = state[id(d)]
        d.pos.copy_(pos0)
        d.tok.copy_(tok0)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(steps):
            run()
        e.record()
        torch.cuda.synchronize()
        return {"tg_b1": steps * 1e3 / s.elapsed_time(e)}

    arms = {"graph": lambda: timed(dec, g.replay),
            "graph_dup": lambda: timed(dec, g.replay),
            "mega": lambda: timed(mg, mg.step)}
    if batch:
        rng = np.random.default_rng(3)
        ctx = rng.integers(256, 2049, batch)
        bd = QB.BatchedDecoder(dm, B=batch, max_ctx=2048 + steps + 1, page_seed=batch)
        bd.fill_random_context(ctx, seed=batch)
        bd.tok.copy_(torch.from_numpy(rng.integers(0, dm.cfg.V, batch).astype(np.int32)))
        bg = bd.capture()
        bpos, btok = bd.pos.clone(), bd.tok.clone()

        def batched():
            bd.pos.copy_(bpos)
            bd.tok.copy_(btok)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(steps):
                bg.replay()
            e.record()
            torch.cuda.synchronize()
            return {f"tg_b{batch}": batch * steps * 1e3 / s.elapsed_time(e)}
        arms["batched"] = batched
    return arms


def llama_bench_arm(binary: str, gguf: str, n: int = 256, reps: int = 5, timeout: int = 1800) -> Arm:
    """An external llama.cpp `llama-bench` run (-p 0 -n n, all layers offloaded, flash attention off and on),
    reporting the better of the two as tg_b1 (generous to llama.cpp, as scripts/decode_paired.py:summarize)."""
    def run():
        p = subprocess.run([binary, "-m", gguf, "-ngl", "99", "-p", "0", "-n", str(n), "-fa", "0,1",
                            "-r", str(reps), "-o", "json"], capture_output=True, text=True, timeout=timeout)
        txt = p.stdout
        try:
            rows = json.loads(txt[txt.find("["):txt.rfind("]") + 1])
        except ValueError:
            return {}
        ts = [float(x["avg_ts"]) for x in rows if "avg_ts" in x]
        return {"tg_b1": max(ts)} if ts else {}
    return run
