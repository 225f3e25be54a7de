"""GGUF test fixtures: a minimal GGUF v3 writer and a Qwen2-layout file writer (test infrastructure)."""
import struct
from pathlib import Path

import numpy as np


def write_gguf(path, tensors, meta):
    """tensors = {name: (ggml_type, dims, raw bytes)} (dims in ggml order, dims[0] contiguous);
    meta values: int -> uint32, float -> float32, str -> string, [str] / [int] -> array of string / int32."""
    def s(x):
        e = x.encode()
        return struct.pack("<Q", len(e)) + e
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for k, v in meta.items():
        if isinstance(v, float):
            out += s(k) + struct.pack("<I", 6) + struct.pack("<f", v)
        elif isinstance(v, str):
            out += s(k) + struct.pack("<I", 8) + s(v)
        elif isinstance(v, list) and v and isinstance(v[0], str):
            out += s(k) + struct.pack("<IIQ", 9, 8, len(v)) + b"".join(s(x) for x in v)
        elif isinstance(v, list):
            out += s(k) + struct.pack("<IIQ", 9, 5, len(v)) + struct.pack(f"<{len(v)}i", *v)
        else:
            out += s(k) + struct.pack("<I", 4) + struct.pack("<I", v)
    off = 0
    datas = []
    for name, (typ, dims, raw) in tensors.items():
        out += s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        out += struct.pack("<IQ", typ, off)
        datas.append(raw)
        off += -(-len(raw) // 32) * 32
    out += b"\0" * (-len(out) % 32)
    for raw in datas:
        out += raw + b"\0" * (-len(raw) % 32)
    Path(path).write_bytes(bytes(out))


def write_qwen_gguf(path, cfg, w):
    """A Qwen2 GGUF (llama.cpp tensor names) from a weight dict in the random_weights layout; w["head_q6k"]
    (Q6_K bytes of [V, H]) becomes output.weight."""
    Q4, F32, Q6 = 2, 0, 14
    H, HD = cfg.H, cfg.HD
    t = {"token_embd.weight": (Q4, (H, cfg.V), w["embed"].tobytes()),
         "output_norm.weight": (F32, (H,), np.asarray(w["norm"], np.float32).tobytes())}
    if "head_q6k" in w:
        t["output.weight"] = (Q6, (H, cfg.V), w["head_q6k"].tobytes())
    for i, L in enumerate(w["layers"]):
        p = f"blk.{i}."
        t[p + "attn_q.weight"] = (Q4, (H, cfg.NH * HD), L["wq"].tobytes())
        t[p + "attn_k.weight"] = (Q4, (H, cfg.NKV * HD), L["wk"].tobytes())
        t[p + "attn_v.weight"] = (Q4, (H, cfg.NKV * HD), L["wv"].tobytes())
        for b in ("q", "k", "v"):
            t[p + f"attn_{b}.bias"] = (F32, (len(L["b" + b]),), np.asarray(L["b" + b], np.float32).tobytes())
        t[p + "attn_output.weight"] = (Q4, (cfg.NH * HD, H), L["wo"].tobytes())
        t[p + "ffn_gate.weight"] = (Q4, (H, cfg.FFN), L["wg"].tobytes())
        t[p + "ffn_up.weight"] = (Q4, (H, cfg.FFN), L["wu"].tobytes())
        t[p + "ffn_down.weight"] = (Q4, (cfg.FFN, H), L["wd"].tobytes())
        t[p + "attn_norm.weight"] = (F32, (H,), np.asarray(L["ln1"], np.float32).tobytes())
        t[p + "ffn_norm.weight"] = (F32, (H,), np.asarray(L["ln2"], np.float32).tobytes())
    meta = {"qwen2.embedding_length": H, "qwen2.attention.head_count": cfg.NH,
            "qwen2.attention.head_count_kv": cfg.NKV, "qwen2.feed_forward_length": cfg.FFN,
            "qwen2.block_count": cfg.L, "qwen2.attention.layer_norm_rms_epsilon": float(cfg.eps),
            "qwen2.rope.freq_base": float(cfg.theta)}
    write_gguf(path, t, meta)


def random_q6_k(n_blocks, rng, d=0.002):
    """Random Q6_K blocks (any ql/qh/scales bytes form a valid block) with super-block scale d."""
    b = rng.integers(0, 256, (n_blocks, 210), dtype=np.uint8)
    b[:, 208:210] = np.array([d], np.float16).view(np.uint8)
    return b
