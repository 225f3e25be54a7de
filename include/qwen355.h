/* qwen355.h -- C ABI of libqwen355.so, the gfx950 (MI355X) Qwen2.5 Q4_0 inference hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as void*; NULL =
 * the default stream), enqueues its kernels on that stream, allocates nothing and returns 0 on
 * success, Q355_EINVAL for a shape/argument error (checked on the host before any launch), or the
 * hipError_t of a failed launch. q355_last_error() describes the last failure of the calling thread.
 * Entry points can be captured into a hipGraph (no host synchronisation, no allocation, scratch
 * counters reset themselves).
 *
 * Formats (see 3080lab_amd/csrc/common.h):
 *   Q4_0 matrix [N, K]: qs uint8 [N/16][K/32][16][16] (GGUF qs bytes per block), d fp16 [N/16][K/32][16].
 *   Q8_1 activations [T, K]: xq int8 [T][K], xds half2 [T][K/32] = (d, s = d * sum q).
 *   KV cache (per layer): fp16 [n_pages][nkv][64][128]; block_table int32 [n_seq][bt_stride] page ids.
 *   RoPE tables: fp32 [maxlen][64] (cos, sin). Token positions and ids are int32.
 *   Residual stream h [T][H]: int64 fixed point, value = h * 2^-48 (|h| < 2^15). K-split projections add
 *   into it with integer atomics, so every result is bitwise independent of workgroup timing.
 *
 * Each declaration names the reference interface it replaces (paths relative to the reference
 * repository lblommesteyn/3080lab).
 */
#ifndef QWEN355_H
#define QWEN355_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q355_OK 0
#define Q355_EINVAL 1

/* Replaces check()/RuntimeError reporting (scripts/qwen_e2e.py:38-41, lab/gpu.py:11-21). */
const char* q355_last_error(void);

/* Library version string, for the loader's sanity check (no reference counterpart needed by callers
 * beyond lab/toolchain.py:107-110's "build returned a module"). */
const char* q355_version(void);

/* Q8_1 activation quantizer: x fp32 [T][K] -> xq, xds.
 * Replaces QUANT_Q8 (lab/qwen_batched.py:1016-1041). K % 32 == 0. */
int q355_quant_q8_1(const float* x, int8_t* xq, void* xds, int T, int K, void* stream);

/* Fused RMSNorm + Q8_1: x = Q8_1(h * rsqrt(mean(h^2) + eps) * w) per token.
 * Replaces rmsnorm_q8_source (lab/qwen_batched.py:1044-1091) and RMSNORM_F32W_1P
 * (lab/qwen_kernels.py:683-705). H % 32 == 0, H <= 2048. */
int q355_rmsnorm_q8_1(const float* h, const float* w, int8_t* xq, void* xds, int T, int H, float eps,
                      void* stream);

/* Q4_0 x Q8_1 GEMV for T = 1..4 tokens: y[T][N] (epi 0: =, 1: +=, 2: = acc + bias[N]).
 * Deterministic: fixed reduction order, one writer per output.
 * Replaces gemv_source epilogues store / bias / biasf / resid / logits (lab/qwen_kernels.py:14-113).
 * N % 16 == 0, K % 32 == 0, K <= 9216. */
int q355_gemv_q4_0_q8_1(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq, const void* xds,
                        int T, float* y, const float* bias, int epi, void* stream);

/* Reference-parity mode: Q4_0 x bf16 activations x [T][K] (bf16 bits), fp32 arithmetic as the reference's
 * gemv_source (lab/qwen_kernels.py:14-113): per 32-block y += d * sum_i fmaf(q_i - 8, x_i); epi 0 store,
 * 1 += (resid), 2 + bias. N % 16 == 0, K % 32 == 0, K <= 9216, T = 1..4. */
int q355_gemv_q4_0_bf16(const uint8_t* qs, const void* d, int N, int K, const void* x, int T, float* y,
                        const float* bias, int epi, void* stream);

/* Debug: every per-block int32 dot out[T][N][K/32] = sum_i q_w,i (0..15) * q_x,i (bit-exact check).
 * Replaces the per-block timing/debug arguments of gemv_source (lab/qwen_kernels.py:46-53). */
int q355_gemv_blockdots(const uint8_t* qs, int N, int K, const int8_t* xq, int T, int32_t* out, void* stream);

/* Fused ln1 RMSNorm + Q8_1 + QKV GEMV + bias + RoPE(q, k) + fp16 K/V cache write + fp16 q out.
 * h is the fixed-point residual stream. Rows of q and k heads are stored interleaved (d, d + 64) and the
 * bias in the same order. Replaces RMSNORM_F32W_1P + gemv_source('biasf') + the RoPE/KV-write head of
 * ATTN4 (lab/qwen_kernels.py:33, 517-546) and gemm 'biasf_kv' (lab/qwen_batched.py:1316-1362).
 * Token j (j < T <= 4) is at position pos[j] of sequence j * seq_stride. K <= 1536. */
int q355_qkv_rope_kv(const uint8_t* qs, const void* d, int K, const int64_t* h, const float* nw, double eps,
                     const float* bias, const float* rope_cos, const float* rope_sin, const int32_t* pos,
                     const int32_t* block_table, int bt_stride, int seq_stride, void* kcache, void* vcache,
                     void* qout, int nh, int nkv, int T, void* stream);

/* Layer 0's q355_qkv_rope_kv with q355_embed_q4_0 in its prologue: h = the tied Q4_0 embedding row of
 * tok[j] (clamped to 0..V-1; q355_embed_q4_0 skips an out-of-range token instead), exact in fixed point,
 * written to h_out as the step's residual stream. Replaces the EMBED_F32 launch plus the first layer's
 * RMSNORM_F32W_1P + gemv_source('biasf') + ATTN4 RoPE/KV head (lab/qwen_kernels.py:284-290, 33, 517-546)
 * with one launch. K <= 1536. */
int q355_qkv_rope_kv_embed(const uint8_t* qs, const void* d, int K, const uint8_t* emb_qs, const void* emb_d,
                           int V, const int32_t* tok, int64_t* h_out, const float* nw, double eps,
                           const float* bias, const float* rope_cos, const float* rope_sin, const int32_t* pos,
                           const int32_t* block_table, int bt_stride, int seq_stride, void* kcache, void* vcache,
                           void* qout, int nh, int nkv, int T, void* stream);

/* Fused ln2 RMSNorm + Q8_1 + gate_up GEMV (rows interleaved gate, up) + SwiGLU: m fp32 [T][N2/2].
 * Replaces gemv_source('swiglu') (lab/qwen_kernels.py:21-28). K <= 1536. */
int q355_ffn_gate_up(const uint8_t* qs, const void* d, int N2, int K, const int64_t* h, const float* nw, double eps,
                     float* m, int T, void* stream);

/* Fused Q8_1 of m + down GEMV + residual: h[T][N] += Wd . Q8_1(m) (2 K slices, fixed-point atomics).
 * Replaces swiglu_q8's quantizer (lab/qwen_batched.py:1363-1396) + gemv_source('resid') for down (:34).
 * K % 128 == 0, K <= 9216. */
int q355_ffn_down(const uint8_t* qs, const void* d, int N, int K, const float* m, int64_t* h, int T, void* stream);

/* Final RMSNorm + Q8_1 + tied Q4_0 head: logits fp32 [T][V] and per-workgroup (max, lowest index)
 * partials pmax/pidx [T][q355_head_nparts(V)]. Replaces gemv_q6_source / 'logits'
 * (lab/qwen_kernels.py:608-678, 36) and the first stage of FINISH_MB (250-270). */
int q355_head_logits(const uint8_t* qs, const void* d, int V, int K, const int64_t* h, const float* nw, double eps,
                     float* logits, float* pmax, int32_t* pidx, int T, void* stream);
int q355_head_nparts(int V);

/* Tied-head variant for llama.cpp's Q6_K output.weight: the same fused final RMSNorm + Q8_1 + logits + argmax
 * partials over a Q6_K matrix in the library's Q6_K planes (lab/gguf.py:tile_q6_k): lo uint8
 * [V/16][K/32][16][16], hi uint8 [V/16][K/32][16][8], sc int8 [V/16][K/32][16][2], d fp16 [V/16][K/256][16];
 * per 16-weight sub-block the int32 dot sc * (sum (v - 32) q_x) is exact. K % 256 == 0, K <= 1536.
 * Replaces gemv_q6_source / head_v2_source (lab/qwen_kernels.py:608-678, lab/qwen_batched.py:681-833). */
int q355_head_logits_q6k(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int V, int K,
                         const int64_t* h, const float* nw, double eps, float* logits, float* pmax, int32_t* pidx,
                         int T, void* stream);

/* Q6_K x Q8_1 GEMV (store), T = 1..4, K <= 1536: the parity entry point of the Q6_K planes.
 * Replaces gemv_q6_source's plain form (lab/qwen_kernels.py:608-678). */
int q355_gemv_q6_k_q8_1(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int N, int K,
                        const int8_t* xq, const void* xds, int T, float* y, void* stream);

/* Greedy finish: tok[j] = argmax (lowest index on ties) over the head partials, pos[j] += 1.
 * Replaces FINISH / FINISH_MB (lab/qwen_kernels.py:222-282). */
int q355_finish(const float* pmax, const int32_t* pidx, int nparts, int32_t* tok, int32_t* pos, int T,
                void* stream);

/* Embedding lookup from the tied Q4_0 table into the fixed-point residual stream: h[j] = dequant(E[tok[j]]).
 * Replaces EMBED_F32 (lab/qwen_kernels.py:284-290). */
int q355_embed_q4_0(const uint8_t* qs, const void* d, int V, int H, const int32_t* tok, int64_t* h, int T,
                    void* stream);

/* Decode GQA attention, split-K over 64-position pages: token j attends to positions 0..pos[j] of its
 * sequence (block_table row j); max_chunks >= (max pos)/64 + 1, <= 64; GQA group nh/nkv in {4, 6, 8}.
 * fp32 = 0 (the batch-1 path, exact against the f64 oracle): scores, softmax and P.V in f64; writes the
 * unnormalised partials part f64 [T][nh][max_chunks][130] (o[128], running max, sum) of every live chunk,
 * and if oq/ods are given merges them (second launch) into Q8_1 oq int8 [T][nh*128], ods half2 [T][nh*4],
 * optionally fp32 o32 [T][nh*128].
 * fp32 = 1 (the batched path): fp16 matrix-core products, fp32 softmax, 4-page partials merged inside the
 * attention launch and the rest by a second launch; oq/ods required (o32 optional); part is scratch
 * (fp32 split partials, no initial contents needed).
 * Replaces ATTN2 / ATTN4 (lab/qwen_kernels.py:358-442, 517-605). */
int q355_attn_decode(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                     const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                     double* part, int8_t* oq, void* ods, float* o32, int T, int fp32, void* stream);

/* Allocation-free form of q355_attn_decode with fp32 = 1, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The fp32 split partials go to a fixed device array inside the library (one per GPU, held until the
 * process ends) instead of a caller buffer; it calls no hipMalloc/hipFree. Limit:
 * T * nh * ceil(max_chunks / 4) * 130 * 4 bytes <= q355_attn_decode_noalloc_max_bytes() (4 MiB), else
 * Q355_EINVAL. Every call on one GPU shares the array: serialise all calls on a device through one stream
 * (graphs or decoders replayed on different streams race and give wrong outputs with no error). Outputs and the
 * other arguments as q355_attn_decode; GQA group nh/nkv <= 16. */
int64_t q355_attn_decode_noalloc_max_bytes(void);
int q355_attn_decode_noalloc(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                             const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                             double scale, int8_t* oq, void* ods, float* o32, int T, void* stream);

/* Fused attention merge + Q8_1 + O-projection GEMV + residual: h[T][N] += Wo . Q8_1(merge(part))
 * (3 K slices of nh/3 heads, fixed-point atomics). part / max_chunks / pos as written by
 * q355_attn_decode; nh % 3 == 0, K = nh * 128 <= 1536.
 * Replaces the ATTN2 last-block combine (lab/qwen_kernels.py:424-440) + gemv_source('resid') for o (:34). */
int q355_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                      const int32_t* pos, int nh, int64_t* h, int T, void* stream);

/* ---- int8 MFMA path: batched decode (config 3) and prefill (config 4) ---- */

/* RMSNorm of the fixed-point residual stream -> Q8_1 (one token per workgroup).
 * Replaces rmsnorm_q8_source (lab/qwen_batched.py:1044-1091) / RMSNORM_F32W_1P batched by blockIdx.y. */
int q355_rmsnorm_fix_q8_1(const int64_t* h, const float* w, int8_t* xq, void* xds, int T, int H, double eps,
                          void* stream);

/* Q4_0 x Q8_1 product of T tokens on v_mfma_i32_16x16x32_i8 (exact int32 block dots), N % 64 == 0.
 * epi 0: y fp32 [T][N] = W x;  5: argmax partials pmax/pidx [T][q355_mmq_nparts(N)] and, if y is given, logits y [T][N];
 * 6: yfix [T][N] += W x (int64 fixed point, K-sliced, integer atomics);
 * 4: rows interleaved (gate, up): y fp32 [T][N/2] = silu(g) * u;
 * 7: rows interleaved (gate, up): Q8_1 of silu(g) * u into oq [T][N/2], ods [T][N/64].
 * Replaces gemm_q4i8_source / gemm_q4i8_ms_source with epilogues resid / swiglu_q8
 * (lab/qwen_batched.py:1093-1561; prefill), and serves batched decode in its Q8_1 mode. */
int q355_mmq_q4_0_q8_1(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq, const void* xds, int T,
                       int epi, float* y, int64_t* yfix, int8_t* oq, void* ods, float* pmax, int32_t* pidx,
                       void* stream);
int q355_mmq_nparts(int N);

/* Q6_K x Q8_1 LM head for decode batches on int8 MFMA: logits y fp32 [T][V] (optional, y may be NULL) and the
 * argmax partials pmax/pidx [T][V/64] (max, lowest row of every 64 rows; q355_finish reduces them), from
 * llama.cpp's Q6_K output.weight in the library's Q6_K planes (as q355_head_logits_q6k) and Q8_1 activations
 * xq/xds [T][K]. Each 16-weight sub-block is an exact int32 dot. V % 64 == 0, K % 256 == 0, K <= 1536, T <= 32.
 * Replaces head_v2_source (lab/qwen_batched.py:681-833). */
int q355_mmq_q6k_logits(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int V, int K,
                        const int8_t* xq, const void* xds, int T, float* y, float* pmax, int32_t* pidx, void* stream);

/* Decode batches (T <= 32): yfix [T][N] += W Q8_1(xf), the fp32 activations xf [T][K] (e.g. the SwiGLU output
 * of epi 4) quantized to Q8_1 inside the kernel (d = fp16(amax / 127) per 32-block, q = round(x / d)), then
 * the int8 MFMA product of q355_mmq_q4_0_q8_1 epi 6. N % 64 == 0.
 * Replaces the quantize + MMQ down pair of the batched step (swiglu_q8 -> gemv, lab/qwen_batched.py). */
int q355_mmq_q4_0_f32(const uint8_t* qs, const void* d, int N, int K, const float* xf, int T, int64_t* yfix,
                      void* stream);

/* ---- fp16-activation path: batched decode (config 3) ---- */

/* RMSNorm of the fixed-point residual stream -> fp16 xh [T][H] (one rounding of the f64 value).
 * Replaces the bf16 RMSNorm of the batched decode (scripts/qwen_batched_decode.py:156-187). */
int q355_rmsnorm_fix_f16(const int64_t* h, const float* w, void* xh, int T, int H, double eps, void* stream);

/* Q4_0 weights dequantized to fp16 (d (q - 8), one rounding) times fp16 activations xh [T][K] on
 * v_mfma_f32_16x16x32_f16 with fp32 accumulation, N % 64 == 0.
 * epi 0: y fp32 [T][N];  5: logits y [T][N] + argmax partials pmax/pidx [T][q355_mmq_nparts(N)];
 * 6: yfix [T][N] += W x (int64 fixed point, K-sliced, integer atomics);
 * 8: rows interleaved (gate, up): yh fp16 [T][N/2] = silu(g) * u.
 * Replaces gemv_v2_source (lab/qwen_batched.py:467-680: the same fp16 dequantization, fp16 tensor cores)
 * and head_v2_source (:681-833) for the tied Q4_0 head. */
int q355_gemm_q4_0_f16(const uint8_t* qs, const void* d, int N, int K, const void* xh, int T, int epi, float* y,
                       int64_t* yfix, void* yh, float* pmax, int32_t* pidx, void* stream);

/* The batched int8 path's attention without its merge launch: as q355_attn_decode with fp32 = 1, but tokens
 * whose context spans several 4-page splits leave only their split partials in part (for
 * q355_mmq_attn_o_resid); tokens of <= 256 positions are finished into oq/ods.
 * Replaces the batched ATTN4 of scripts/qwen_batched_decode.py:156-187 (its combine moves into the O product). */
int q355_attn_decode_partials(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                              const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                              double* part, int8_t* oq, void* ods, int T, void* stream);

/* The fp16 batched path's attention without its merge launch: as q355_attn_decode_f16, but tokens whose context
 * spans several 4-page splits leave only their split partials in part (for q355_gemm_f16_attn_o_resid); tokens
 * of <= 256 positions are finished into oh [T][nh*128] fp16.
 * Replaces the batched ATTN4 of scripts/qwen_batched_decode.py:156-187 (its combine moves into the O product). */
int q355_attn_decode_partials_f16(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                  const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                  double scale, double* part, void* oh, int T, void* stream);

/* O projection + residual of the fp16 batched path (T <= 16) with the attention merge in its activation staging:
 * h[T][N] += Wo . fp16(merge(part)) per head (one K slice per head), reading oh for tokens that
 * q355_attn_decode_partials_f16 finished itself. The activations are the bytes q355_attn_decode_f16 writes;
 * the product is the fp16-weight arithmetic of q355_gemm_q4_0_f16 (epi 6) with its own K split. K = nh * 128.
 * Replaces the batched combine + gemv_v2_source 'resid' for o (scripts/qwen_batched_decode.py:156-187). */
int q355_gemm_f16_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                               const int32_t* pos, int nh, int nkv, const void* oh, int64_t* h, int T, void* stream);

/* O projection + residual of the batched int8 path with the attention merge in its activation staging:
 * h[T][N] += Wo . Q8_1(merge(part)) per head (one K slice per head), reading xq/xds for tokens that
 * q355_attn_decode_partials finished itself. The same bytes as q355_attn_decode's merge followed by
 * q355_mmq_q4_0_q8_1 (epi 6). K = nh * 128.
 * Replaces the batched combine + gemv_v2_source 'resid' for o (scripts/qwen_batched_decode.py:156-187). */
int q355_mmq_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                          const int32_t* pos, int nh, int nkv, const int8_t* xq, const void* xds, int64_t* h, int T,
                          void* stream);

/* Batched decode attention (fp16 MFMA, fp32 softmax; the GQA group's heads as MFMA columns) + merge of the
 * page partials -> fp16 oh [T][nh*128]. Arguments and the part scratch as q355_attn_decode with fp32 = 1.
 * Replaces the batched ATTN4 + combine of scripts/qwen_batched_decode.py:156-187. */
int q355_attn_decode_f16(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                         const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                         double* part, void* oh, int T, void* stream);

/* QKV of the fp16 batched path: Q4_0 x fp16 activations xh [T][K] on fp16 MFMA (T <= 32, K <= 1536) with bias,
 * RoPE and the K/V cache write in the epilogue (arguments otherwise as q355_mmq_qkv_rope).
 * Replaces gemv_v2_source with the 'biasf_kv' epilogue (lab/qwen_batched.py:467-680, 1316-1362). */
int q355_gemm_f16_qkv_rope(const uint8_t* qs, const void* d, int N, int K, const void* xh, int T, const float* bias,
                           const float* rope_cos, const float* rope_sin, const int32_t* pos, const int32_t* block_table,
                           int bt_stride, int seq_stride, void* kcache, void* vcache, void* qout, int nh, int nkv,
                           void* stream);

/* QKV epilogue of the MFMA path: acc int64 fixed point [T][nqkv] (device row order) -> + bias, RoPE, fp16
 * q out [T][nh*128], fp16 K/V cache rows at pos[j] of sequence j * seq_stride; acc is zeroed.
 * Replaces 'biasf_kv' (lab/qwen_batched.py:1316-1362) and the RoPE/KV-write head of ATTN4. */
int q355_qkv_finish(int64_t* acc, const float* bias, const float* rope_cos, const float* rope_sin,
                    const int32_t* pos, const int32_t* block_table, int bt_stride, int seq_stride, void* kcache,
                    void* vcache, void* qout, int nh, int nkv, int T, void* stream);

/* QKV: Q4_0 x Q8_1 product of T tokens on int8 MFMA (register-resident for T <= 32 and K <= 1536, LDS-tiled
 * otherwise) with the QKV finish in its epilogue: + bias, RoPE, fp16 q out [T][nh*128], fp16 K/V cache rows at pos[j] of sequence j * seq_stride
 * (arguments as q355_qkv_finish). q64 (optional, may be NULL): the same fp16 q values widened to f64 [T][nh*128],
 * the input of q355_attn_decode_f64. N = (nh + 2 nkv) * 128 in the device row order, N % 128 == 0.
 * Replaces gemm_q4i8_ms_source with the 'biasf_kv' epilogue (lab/qwen_batched.py:1271-1561, 1316-1362). */
int q355_mmq_qkv_rope(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq, const void* xds, int T,
                      const float* bias, const float* rope_cos, const float* rope_sin, const int32_t* pos,
                      const int32_t* block_table, int bt_stride, int seq_stride, void* kcache, void* vcache,
                      void* qout, double* q64, int nh, int nkv, void* stream);

/* Batched decode attention of the int8 path, in f64 (the batch-1 arithmetic: f64 scores, softmax and P.V of
 * the fp16 q/K/V): T tokens, token j attends to positions 0 .. pos[j] of its paged K/V (block_table row j).
 * q64 [T][nh*128] f64 (q355_mmq_qkv_rope's q64). Splits of 2 pages, 4 waves per page, the GQA group's query
 * heads together; splits merged in f64 in split order -> Q8_1 oq [T][nh*128] / ods [T][nh*4] (and fp32 o32,
 * optional). part: scratch of T * nh * ceil(max_chunks / 2) * 130 doubles. GQA group 4, 6 or 8.
 * Replaces the batched ATTN4 + combine of scripts/qwen_batched_decode.py:156-187 (lab/qwen_kernels.py:517-605). */
int q355_attn_decode_f64(const double* q64, const void* kcache, const void* vcache, const int32_t* pos,
                         const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                         double* part, int8_t* oq, void* ods, float* o32, int T, void* stream);

/* The same attention over a list of the step's live (token, KV head, two-page split) items, built by
 * q355_attn_f64_worklist from pos / block_table after the positions last changed (once per step: every layer
 * reuses it). The list puts the live work first in grid order and carries each item's position and page ids,
 * so no workgroup waits on a dead split or a dependent block-table load. Up to 16 tokens the last split of each
 * (token, KV head) to finish merges that token's splits itself (arrival counters at the end of the work buffer),
 * so there is no merge launch. Bit-identical to q355_attn_decode_f64.
 * work: q355_attn_f64_worklist_bytes(T, nkv, max_chunks) bytes, zero-filled once before its first use (the
 * counters reset themselves; concurrent launches on one work buffer race); T <= 64 (decode batches).
 * No counterpart in the reference: ATTN4 (lab/qwen_kernels.py:517-605) launches one block per (token, head). */
int64_t q355_attn_f64_worklist_bytes(int T, int nkv, int max_chunks);
int q355_attn_f64_worklist(const int32_t* pos, const int32_t* block_table, int bt_stride, int nkv, int max_chunks,
                           int T, void* work, void* stream);
int q355_attn_decode_f64_wl(const double* q64, const void* kcache, const void* vcache, const int32_t* pos,
                            const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                            double* part, int8_t* oq, void* ods, float* o32, int T, const void* work, void* stream);

/* Causal GQA prefill attention (fp16 MFMA, fp32 accumulation) for one sequence: queries q fp16
 * [P][nh*128] at positions pos0 .. pos0 + P - 1 attend to keys 0 .. their own position in the paged cache
 * (block_table = the sequence's page ids, >= (pos0 + P - 1) / 64 + 1 of them; K/V of every attended
 * position already written); out fp32 [P][nh*128] = softmax(q k^T * scale) v. 4 to 8 query heads per KV
 * head. ws (optional, ws_bytes >= q355_attn_prefill_ws_bytes(P, pos0 + P, nh, nkv), zeroed once by the
 * caller and reused across calls) runs the persistent form: one workgroup per CU over (16-query block, KV
 * head, 1024-key split) items balanced across the CUs, splits merged in split order (the result does not
 * depend on scheduling). With ws = NULL, and where every query row fits one split and one round, each
 * 16-query block takes all its keys in one workgroup. Calls sharing a workspace must not overlap.
 * Replaces flash_prefill_v3_source (lab/qwen_batched.py:1795-2037). */
int q355_attn_prefill(const void* q, const void* kcache, const void* vcache, const int32_t* block_table, int pos0,
                      int P, int nh, int nkv, float scale, float* out, void* ws, int64_t ws_bytes, void* stream);
/* q355_attn_prefill with the output quantized to Q8_1 in the same launch (oq int8 [P][nh*128], ods half2
 * [P][nh*4]): the values q355_attn_prefill stores, quantized exactly as q355_quant_q8_1 does.
 * Replaces flash_prefill_v3_source(q8=True) (lab/qwen_batched.py:1811-1848). */
int q355_attn_prefill_q8_1(const void* q, const void* kcache, const void* vcache, const int32_t* block_table,
                           int pos0, int P, int nh, int nkv, float scale, int8_t* oq, void* ods, void* ws,
                           int64_t ws_bytes, void* stream);
/* Workspace bytes of q355_attn_prefill for chunks of up to P queries with pos0 + P <= max_ctx (-1: bad sizes). */
int64_t q355_attn_prefill_ws_bytes(int P, int max_ctx, int nh, int nkv);

/* ---- persistent whole-step decode (batch 1) ---- */

/* Bytes of the workspace q355_mega_decode needs for max_chunks pages and L layers. The caller zeroes it
 * once; it carries the synchronisation words across launches (do not clear it between steps). */
int64_t q355_mega_ws_bytes(int max_chunks, int L);
/* sizeof of one entry of the per-layer pointer table (13 pointers: qkv qs/d/bias, ln1, o qs/d, ln2,
 * gate_up qs/d, down qs/d, K cache, V cache). */
int q355_mega_layer_bytes(void);

/* One greedy decode step of the whole model in ONE launch of 256 workgroups (one per CU; fails with
 * Q355_EINVAL if the device cannot keep 256 resident): embed tok, L layers, final norm + tied Q4_0 head,
 * tok = argmax (lowest index on ties), pos += 1; logits fp32 [V]; h int64 [1536] receives the final
 * residual. logits == NULL: the launch stops after the layers (h receives the final residual, tok and pos are
 * left unchanged) so the caller can run another head, e.g. q355_head_logits_q6k + q355_finish for llama.cpp's Q6_K
 * output.weight. Shapes: H 1536, 12/2 heads of 128, FFN 8960, V % 16 == 0, max_chunks <= 64, pos < 64 max_chunks.
 * Waits between workgroups are bounded by spin_limit_us; on expiry (or a bad pos/tok) the workspace error
 * word is set and the launch completes with invalid outputs.
 * Replaces mega_source (lab/qwen_mega.py:43-361) and the graph of FusedQwen.step (scripts/qwen_fused.py:113-180). */
int q355_mega_decode(const void* layers, int L, const uint8_t* emb_qs, const void* emb_d, const float* norm, int V,
                     const float* rope_cos, const float* rope_sin, const int32_t* block_table, int max_chunks,
                     double eps, int32_t* tok, int32_t* pos, int64_t* h, float* logits, void* ws,
                     int64_t spin_limit_us, void* stream);

/* Measurement only: one streaming read of `bytes` (a multiple of 16) from p, 16-byte non-temporal loads all in
 * flight, nothing written. bench.py times it over distinct buffers in a graph to give the practical ceiling
 * for a weight stream of one GEMV's size. No counterpart in the reference. */
int q355_stream_read(const void* p, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QWEN355_H */
