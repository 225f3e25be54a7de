"""MI355X (gfx950) Qwen2.5 Q4_0 inference hot path: host-side Python mirror of 3080lab's `lab` package.

Import with `3080lab_amd/` on sys.path (the directory name is not an identifier):
    from lab import qwen_kernels as KS, qwen_model, gguf
All compute goes through libqwen355.so (lab/hip.py); there is no CPU fallback.
"""
