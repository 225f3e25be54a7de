"""Decode (batch 1..4) kernel specs: the reference's lab/qwen_kernels.py names, bound to libqwen355.so.

The reference's generators return CUDA C source compiled by NVRTC (lab/qwen_kernels.py:14-812). Here
each name returns a KernelSpec naming the C-ABI entry point that replaces it; lab.hip.Kern(spec)
.launch(grid, block, args) calls it with the entry point's argument order (include/qwen355.h). The
fused entry points fold neighbouring reference kernels together (RMSNorm into the GEMV prologue,
RoPE and the K/V write into the QKV epilogue, the Q8_1 quantizer into every producer).
"""
from __future__ import annotations

from dataclasses import dataclass, field

EPILOGUES = ("store", "bias", "biasf", "resid", "swiglu", "logits")
_EPI_CODE = {"store": 0, "logits": 0, "resid": 1, "bias": 2, "biasf": 2}


@dataclass(frozen=True)
class KernelSpec:
    symbol: str
    params: dict = field(default_factory=dict)


def gemv_source(S_: int = 1, epi: str = "store", quant: str = "q8_1", G: int = 1, timed: bool = False) -> KernelSpec:
    """Q4_0 x Q8_1 GEMV (reference: split-K Q4_0 x bf16 GEMV, lab/qwen_kernels.py:14-113).
    epi store/logits/resid/bias/biasf -> q355_gemv_q4_0_q8_1 with the matching epi code;
    epi swiglu -> q355_ffn_gate_up (fused RMSNorm prologue + SwiGLU + Q8_1 epilogue);
    epi biasf_kv -> q355_qkv_rope_kv. S_ (the reference's split-K warp count) has no counterpart: the
    library picks the K split (16 or 32 k-lanes per workgroup) from K."""
    if quant == "bf16":        # reference-parity mode: the reference's bf16-activation fp32 arithmetic
        if epi not in _EPI_CODE:
            raise ValueError(f"epilogue {epi!r} not in {EPILOGUES}")
        return KernelSpec("q355_gemv_q4_0_bf16", {"epi": _EPI_CODE[epi]})
    if quant != "q8_1":
        raise ValueError(f"quant={quant!r}: this build's GEMV consumes Q8_1 (or bf16) activations")
    if epi == "swiglu":
        return KernelSpec("q355_ffn_gate_up")
    if epi in ("biasf_kv", "qkv"):
        return KernelSpec("q355_qkv_rope_kv")
    if epi not in _EPI_CODE:
        raise ValueError(f"epilogue {epi!r} not in {EPILOGUES}")
    return KernelSpec("q355_gemv_q4_0_q8_1", {"epi": _EPI_CODE[epi]})


# Single kernels of the reference, by name
RMSNORM = KernelSpec("q355_rmsnorm_q8_1")             # RMSNORM / RMSNORM_F32W / RMSNORM_F32W_1P -> + Q8_1
RMSNORM_F32W = RMSNORM
RMSNORM_F32W_1P = RMSNORM
EMBED = KernelSpec("q355_embed_q4_0")                 # EMBED / EMBED_F32 (tied Q4_0 table)
EMBED_F32 = EMBED
ATTN = KernelSpec("q355_attn_decode")                 # ATTN, ATTN2 (split-K), ATTN3, ATTN4 -> one split-K kernel
ATTN2 = ATTN
ATTN3 = ATTN
ATTN4 = ATTN
FINISH = KernelSpec("q355_finish")                    # FINISH / FINISH_MB (argmax, tok, pos += 1)
FINISH_MB = FINISH
QUANT_Q8 = KernelSpec("q355_quant_q8_1")


def gemv_head_source(S_: int = 1) -> KernelSpec:
    """Tied Q4_0 head with fused final RMSNorm and argmax partials (the role of gemv_q6_source,
    lab/qwen_kernels.py:608-678, for BASELINE's tied Q4_0 head)."""
    return KernelSpec("q355_head_logits")
