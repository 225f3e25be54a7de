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
    """What a reference generator returns here: the C-ABI entry point that replaces the kernel, its parameters,
    and `ref`, the reference kernel whose argument list Kern(spec).launch accepts (lab/refcall.py)."""
    symbol: str
    params: dict = field(default_factory=dict)
    ref: str = ""

    def __mod__(self, _fmt):
        """The reference fills maxlen into kernel source with `%` (scripts/qwen_fused.py:102); the library's
        kernels take the cache geometry as arguments, so the spec is unchanged."""
        return self


def gemv_source(S_: int = 1, epi: str = "store", quant: str = "q8_1", G: int = 1, timed: bool = False) -> KernelSpec:
    """Q4_0 x Q8_1 GEMV (reference: split-K Q4_0 x bf16 GEMV, lab/qwen_kernels.py:14-113).
    Launched with the reference's arguments (W, S, X, Y, AUX, N, K) (lab/refcall.py:launch_gemv), the epilogue
    picks the fused entry point: bias on the qkv buffer -> q355_qkv_rope_kv (at the ATTN launch); resid on the
    attention output -> q355_attn_o_resid; swiglu -> q355_ffn_gate_up; resid on the fp32 SwiGLU output ->
    q355_ffn_down; logits -> q355_head_logits; otherwise q355_gemv_q4_0_q8_1 with the epilogue's code.
    S_ (the reference's split-K warp count) has no counterpart: the library picks the K split from K."""
    if quant == "bf16":        # reference-parity mode: the reference's bf16-activation fp32 arithmetic
        if epi not in _EPI_CODE:
            raise ValueError(f"epilogue {epi!r} not in {EPILOGUES}")
        return KernelSpec("q355_gemv_q4_0_bf16", {"epi": _EPI_CODE[epi]})
    # "g32f16" is how scripts/qwen_gguf.py:126 names GGUF's Q4_0 weights (groups of 32, fp16 scale): the
    # library's weight format, with Q8_1 activations
    if quant not in ("q8_1", "g32f16"):
        raise ValueError(f"quant={quant!r}: this build's GEMV takes Q4_0 weights ('g32f16') with Q8_1 (or bf16) "
                         "activations")
    if epi in ("biasf_kv", "qkv"):          # the fused QKV entry point, called in its own argument order
        return KernelSpec("q355_qkv_rope_kv")
    if epi not in EPILOGUES:
        raise ValueError(f"epilogue {epi!r} not in {EPILOGUES}")
    sym = {"swiglu": "q355_ffn_gate_up", "logits": "q355_head_logits"}.get(epi, "q355_gemv_q4_0_q8_1")
    return KernelSpec(sym, {"epi": _EPI_CODE.get(epi, 0), "epi_name": epi}, ref="gemv")


# Single kernels of the reference, by name (ref = the argument list Kern.launch accepts, lab/refcall.py)
RMSNORM = KernelSpec("q355_rmsnorm_fix_q8_1", ref="rmsnorm")   # RMSNORM / _F32W / _F32W_1P: fused into the consumer
RMSNORM_F32W = RMSNORM
RMSNORM_F32W_1P = RMSNORM
EMBED = KernelSpec("q355_embed_q4_0", ref="embed")             # EMBED / EMBED_F32 (tied Q4_0 table)
EMBED_F32 = EMBED
ATTN = KernelSpec("q355_attn_decode", ref="attn")              # ATTN, ATTN2 (split-K), ATTN3, ATTN4 -> one kernel
ATTN2 = ATTN
ATTN3 = ATTN
ATTN4 = ATTN
FINISH = KernelSpec("q355_finish", ref="finish")               # FINISH / FINISH_MB (argmax, tok, pos += 1)
FINISH_MB = FINISH
QUANT_Q8 = KernelSpec("q355_quant_q8_1")


def gemv_head_source(S_: int = 1) -> KernelSpec:
    """Tied Q4_0 head with fused final RMSNorm and argmax partials (the role of gemv_q6_source,
    lab/qwen_kernels.py:608-678, for BASELINE's tied Q4_0 head)."""
    return KernelSpec("q355_head_logits")
