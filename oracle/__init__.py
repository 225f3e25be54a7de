"""CPU oracle for the Qwen2.5 Q4_0 inference hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of 3080lab's Qwen2.5-1.5B Q4_0 decode /
batched-decode / prefill path (reference files cited per function) with the Q4_0 / Q8_1 /
fp16-KV contract of this build. It is the checker for the HIP product path and the CPU
baseline that bench.py times beside it.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it. The product
package (3080lab_amd/lab) never imports, links or runs anything here, and has no CPU fallback.

Modules:
  quant   Q4_0 block layout + quantizer, Q8_1 activation quantizer, per-block int32 dots, GEMV
  model   RMSNorm, RoPE, GQA attention (decode and causal prefill), SwiGLU, argmax, and the
          whole random-weight Qwen2.5-1.5B-shape model: decode, batched decode, prefill

Pinning status of each function is stated in its docstring ("pinned by: ..."); functions
without an independent check say "parity unpinned".
"""
