"""ctypes binding of libqwen355.so (the gfx950 C ABI declared in include/qwen355.h).

Replaces the reference's NVRTC/cuda-python launch layer (lab/toolchain.py:107-110 build,
scripts/qwen_fused.py:30-42 Kern: cuModuleLoadData + cuLaunchKernel with ctypes argument arrays).
Kernels are compiled ahead of time by hipcc (3080lab_amd/build.py); every entry point enqueues on an
explicit stream (torch's current stream by default, so torch.cuda.CUDAGraph capture records them).

There is no CPU fallback: if the library is missing or fails to load, `lib()` raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, c_double, c_float, c_int, c_void_p
from pathlib import Path

# Q355_LIB selects another build of the same ABI (e.g. an instrumented one); default: the in-tree library
LIB_PATH = Path(os.environ.get("Q355_LIB") or Path(__file__).resolve().parents[1] / "lib" / "libqwen355.so")

_P = c_void_p
# name -> argtypes (all return int status)
_SIGS = {
    "q355_attn_decode_partials": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, _P, c_int, _P],
    "q355_mmq_attn_o_resid": [_P, _P, c_int, _P, c_int, _P, c_int, c_int, _P, _P, _P, c_int, _P],
    "q355_attn_decode_noalloc": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, _P, c_int, _P],
    "q355_attn_decode_noalloc_max_bytes": [],
    "q355_attn_decode_partials_f16": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, c_int, _P],
    "q355_gemm_f16_attn_o_resid": [_P, _P, c_int, _P, c_int, _P, c_int, c_int, _P, _P, c_int, _P],
    "q355_quant_q8_1": [_P, _P, _P, c_int, c_int, _P],
    "q355_rmsnorm_q8_1": [_P, _P, _P, _P, c_int, c_int, c_float, _P],
    "q355_gemv_q4_0_q8_1": [_P, _P, c_int, c_int, _P, _P, c_int, _P, _P, c_int, _P],
    "q355_gemv_q4_0_bf16": [_P, _P, c_int, c_int, _P, c_int, _P, _P, c_int, _P],
    "q355_gemv_blockdots": [_P, c_int, c_int, _P, c_int, _P, _P],
    "q355_qkv_rope_kv": [_P, _P, c_int, _P, _P, c_double, _P, _P, _P, _P, _P, c_int, c_int, _P, _P, _P,
                         c_int, c_int, c_int, _P],
    "q355_qkv_rope_kv_embed": [_P, _P, c_int, _P, _P, c_int, _P, _P, _P, c_double, _P, _P, _P, _P, _P, c_int,
                               c_int, _P, _P, _P, c_int, c_int, c_int, _P],
    "q355_ffn_gate_up": [_P, _P, c_int, c_int, _P, _P, c_double, _P, c_int, _P],
    "q355_ffn_down": [_P, _P, c_int, c_int, _P, _P, c_int, _P],
    "q355_head_logits": [_P, _P, c_int, c_int, _P, _P, c_double, _P, _P, _P, c_int, _P],
    "q355_head_nparts": [c_int],
    "q355_head_logits_q6k": [_P, _P, _P, _P, c_int, c_int, _P, _P, c_double, _P, _P, _P, c_int, _P],
    "q355_gemv_q6_k_q8_1": [_P, _P, _P, _P, c_int, c_int, _P, _P, c_int, _P, _P],
    "q355_finish": [_P, _P, c_int, _P, _P, c_int, _P],
    "q355_embed_q4_0": [_P, _P, c_int, c_int, _P, _P, c_int, _P],
    "q355_attn_decode": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, _P, _P, c_int, c_int, _P],
    "q355_attn_o_resid": [_P, _P, c_int, _P, c_int, _P, c_int, _P, c_int, _P],
    "q355_rmsnorm_fix_q8_1": [_P, _P, _P, _P, c_int, c_int, c_double, _P],
    "q355_mmq_q4_0_q8_1": [_P, _P, c_int, c_int, _P, _P, c_int, c_int, _P, _P, _P, _P, _P, _P, _P],
    "q355_mmq_q4_0_f32": [_P, _P, c_int, c_int, _P, c_int, _P, _P],
    "q355_rmsnorm_fix_f16": [_P, _P, _P, c_int, c_int, c_double, _P],
    "q355_gemm_q4_0_f16": [_P, _P, c_int, c_int, _P, c_int, c_int, _P, _P, _P, _P, _P, _P],
    "q355_attn_decode_f16": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, c_int, _P],
    "q355_mmq_nparts": [c_int],
    "q355_mmq_q6k_logits": [_P, _P, _P, _P, c_int, c_int, _P, _P, c_int, _P, _P, _P, _P],
    "q355_attn_prefill": [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float, _P, _P, ctypes.c_int64, _P],
    "q355_attn_prefill_q8_1": [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float, _P, _P, _P, ctypes.c_int64, _P],
    "q355_attn_prefill_ws_bytes": [c_int, c_int, c_int, c_int],
    "q355_mega_ws_bytes": [c_int, c_int],
    "q355_mega_layer_bytes": [],
    "q355_mega_decode": [_P, c_int, _P, _P, _P, c_int, _P, _P, _P, c_int, c_double, _P, _P, _P, _P, _P,
                         ctypes.c_int64, _P],
    "q355_qkv_finish": [_P, _P, _P, _P, _P, _P, c_int, c_int, _P, _P, _P, c_int, c_int, c_int, _P],
    "q355_mmq_qkv_rope": [_P, _P, c_int, c_int, _P, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int, _P, _P, _P, _P,
                          c_int, c_int, _P],
    "q355_attn_decode_f64": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, _P, _P, c_int, _P],
    "q355_attn_decode_f64_wl": [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_double, _P, _P, _P, _P, c_int, _P,
                                _P],
    "q355_attn_f64_worklist_bytes": [c_int, c_int, c_int],
    "q355_stream_read": [_P, ctypes.c_int64, _P],
    "q355_attn_f64_worklist": [_P, _P, c_int, c_int, c_int, c_int, _P, _P],
    "q355_gemm_f16_qkv_rope": [_P, _P, c_int, c_int, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int, _P, _P, _P,
                               c_int, c_int, _P],
}
# entry points returning something other than an int status
_VALUE_FUNCS = {"q355_attn_decode_noalloc_max_bytes", "q355_head_nparts", "q355_mmq_nparts", "q355_mega_ws_bytes", "q355_mega_layer_bytes",
                "q355_attn_prefill_ws_bytes", "q355_attn_f64_worklist_bytes"}

_lib = None


class HipError(RuntimeError):
    pass


def lib():
    """Load libqwen355.so once; raise HipError if it is not built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipError(f"{LIB_PATH} is not built: run `python 3080lab_amd/build.py` (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.q355_last_error.restype = c_char_p
        L.q355_last_error.argtypes = []
        L.q355_version.restype = c_char_p
        L.q355_version.argtypes = []
        for name, args in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int64 if name.endswith(("_ws_bytes", "_max_bytes", "_worklist_bytes")) else c_int
        _lib = L
    return _lib


def exported_symbols():
    return ["q355_last_error", "q355_version", *_SIGS]


def current_stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None passes NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def call(name: str, *args):
    """Call entry point `name`; the trailing stream argument is added (torch's current stream).
    Raises HipError with the library's message on a non-zero status."""
    L = lib()
    f = getattr(L, name)
    if name in _VALUE_FUNCS:
        return f(*args)
    rc = f(*args, current_stream())
    if rc != 0:
        raise HipError(f"{name}: status {rc}: {L.q355_last_error().decode()}")
    return rc


class Kern:
    """Reference-compatible launcher (scripts/qwen_fused.py:30-42): Kern(spec).launch(grid, block, args).
    `spec` is a KernelSpec from lab.qwen_kernels / lab.qwen_batched / lab.qwen_mega naming a C-ABI entry point.
    If the spec names a reference kernel (spec.ref), `args` is that kernel's own argument list in the reference's
    order, mapped onto the fused entry points by lab/refcall.py (spec.params carries the generator's choices,
    e.g. the GEMV epilogue). Otherwise `args` are the entry point's arguments in declaration order. The library
    picks the gfx950 launch geometry, so grid and block are accepted for signature compatibility and ignored."""

    def __init__(self, spec):
        self.spec = spec
        lib()

    def launch(self, grid=None, block=None, args=()):
        if getattr(self.spec, "ref", ""):
            from .refcall import LAUNCHERS
            return LAUNCHERS[self.spec.ref](self.spec, list(args), grid)
        conv = []
        for a in args:
            if hasattr(a, "data_ptr"):
                conv.append(a.data_ptr())
            elif isinstance(a, (ctypes.c_uint64, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double)):
                conv.append(a.value)
            else:
                conv.append(a)
        return call(self.spec.symbol, *conv)
