// Kernel argument blocks and template dispatch shared by the kernel files and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace q355 {

enum Prologue { PRO_Q8 = 0, PRO_RMS = 1, PRO_ATTN = 2, PRO_F32 = 3, PRO_EMB = 4 };
enum Epilogue {
  EPI_STORE = 0,       // y = acc (fp32)
  EPI_RESID = 1,       // y += acc (fp32, one writer per element: no K split)
  EPI_BIAS = 2,        // y = acc + bias
  EPI_QKV = 3,         // + bias, RoPE, fp16 q out, fp16 K/V cache write
  EPI_SWIGLU = 4,      // rows interleaved (gate, up): y[row / 2] = silu(g) * u (fp32)
  EPI_LOGITS = 5,      // y = acc and per-workgroup (max, lowest index) partials
  EPI_RESID_FIX = 6,   // fixed-point residual: yfix += round(acc * 2^48) (int64 atomics; any K split)
  EPI_SWIGLU_Q8 = 7,   // as SWIGLU, quantized to Q8_1 (oq, ods): NT == 4 (64 rows -> one 32-output block)
  EPI_SWIGLU_F16 = 8,  // as SWIGLU, rounded to fp16 (yh [T][N / 2])
};

constexpr int HD = 128;        // head dim (Qwen2.5-1.5B)
constexpr int PAGE = 64;       // KV cache page: 64 positions of one KV head, [PAGE][HD] fp16
constexpr double FIX_SCALE = 281474976710656.0;    // residual stream fixed point: value * 2^48 as int64
constexpr double FIX_INV = 1.0 / 281474976710656.0;

// The residual stream h is kept as int64 fixed point (2^-48 resolution, |h| < 2^15). Split-K
// producers add their partial sums with integer atomics, which are associative, so the stream is
// bitwise independent of the order in which workgroups finish; 2^-48 is finer than the f64
// accumulation it receives, so the stream tracks an f64 residual to ~1e-14.
__device__ __forceinline__ long long to_fix(double v) { return __double2ll_rn(v * FIX_SCALE); }
__device__ __forceinline__ double from_fix(long long v) { return (double)v * FIX_INV; }

// Everything a GEMV-family launch may need; unused fields are null/zero.
// Weight formats of the GEMV: Q4_0 planes, or the Q6_K planes (lo nibbles, 2-bit hi plane, int8 sub-block
// scales, fp16 super-block scale; 6.5625 bits per weight as in the GGUF file).
enum { WF_Q4_0 = 0, WF_Q6_K = 1 };

struct GemvArgs {
  const uint8_t* qs;           // Q4_0 nibble plane [N/16][K/32][16][16] (Q6_K: the lo plane, same shape)
  const __half* d;             // Q4_0 scale plane  [N/16][K/32][16] (Q6_K: super-block scales [N/16][K/256][16])
  const uint8_t* qhi;          // Q6_K hi plane [N/16][K/32][16][8]
  const uint8_t* qsc;          // Q6_K sub-block scales [N/16][K/32][16][2] (int8)
  int N, K, T;
  // PRO_Q8 input
  const int8_t* xq;            // [T][K]
  const half2* xds;            // [T][K/32]
  // PRO_RMS input
  const long long* hfix;       // [T][K] residual stream, int64 fixed point
  const float* nw;             // [K] RMSNorm weight
  double eps;
  // PRO_EMB input: as PRO_RMS, with h = the tied Q4_0 embedding row of tok[j] (exact in fixed point, the
  // values k_embed_q4_0 writes); workgroup (0, 0) also writes that row to hout
  const uint8_t* emb_qs;
  const __half* emb_d;
  const int* tok;
  int emb_v;
  long long* hout;
  // PRO_F32 input (quantized to Q8_1 in the prologue)
  const float* xf;             // [T][K]
  // PRO_ATTN input: split-K attention partials [T][nh][attn_max_chunks][HD + 2], merged and quantized
  // in the prologue (K == nh * HD); the token positions come from `pos`
  const double* attn_part;
  int attn_max_chunks;
  // STORE / RESID / BIAS / SWIGLU / LOGITS output
  float* y;                    // [T][N] ([T][N/2] for SWIGLU)
  long long* yfix;             // RESID_FIX: [T][N] fixed-point residual stream
  const float* aux;            // bias [N] (BIAS, QKV: bias in the permuted row order)
  // QKV epilogue: RoPE on q/k (rows of each head interleaved (d, d+64)), fp16 q out, K/V cache write
  const float* rope_cos;       // [maxlen][HD/2]
  const float* rope_sin;
  const int* pos;              // [T] position of each token
  const int* block_table;      // [n_seq][bt_stride] page ids
  int bt_stride;
  int seq_stride;              // token j belongs to sequence (tok_base + j) * seq_stride (1: batched, 0: one sequence)
  int tok_base;                // index of token 0 of this launch's token group (MFMA kernels offset per group)
  int mmq_chunk;               // MFMA kernels: K blocks of activations staged in LDS at a time
  __half* kcache;              // [n_pages][nkv][PAGE][HD]
  __half* vcache;
  __half* qout;                // [T][nh*HD]
  double* qout64;              // optional: the same q values widened to f64 [T][nh*HD] (k_attn_batch_f64 input)
  int nh, nkv;
  // SWIGLU_Q8 output: Q8_1 of silu(g) * u, [T][N/2] and [T][N/64]
  int8_t* oq;
  half2* ods;
  // LOGITS: per-workgroup (max, index) partials [T][gridDim.x]
  float* pmax;
  int* pidx;
  // fp16-activation products (batched decode): x fp16 [T][K], SWIGLU_F16 output
  const __half* xh;
  __half* yh;
};

// Causal prefill attention over one sequence's paged KV cache (keys 0 .. pos0 + P - 1 already written).
struct PrefillAttnArgs {
  const __half* q;             // [P][nh*HD] RoPE'd fp16 queries of positions pos0 .. pos0 + P - 1
  const __half* kcache;        // [n_pages][nkv][PAGE][HD]
  const __half* vcache;
  const int* block_table;      // the sequence's page ids, >= (pos0 + P - 1) / PAGE + 1 entries
  int pos0, P, nh, nkv;
  float scale;
  float* out;                  // [P][nh*HD] fp32, or (oq set) instead:
  int8_t* oq;                  // Q8_1 of the output [P][nh*HD] int8 and
  half2* ods;                  //   [P][nh*HD/32] (d, d * sum q)
  // null: one workgroup per (query block, KV head) takes all its keys (k_attn_prefill). Otherwise the
  // persistent form (k_attn_prefill_pers) over n_items items (query block, KV head, key split of
  // PF_SPLIT_PAGES pages), with partials [n_qblocks][nkv][max_splits][G][8][64] float4 (O^T in MFMA
  // accumulator order), (m, l, -, -) [n_qblocks][nkv][max_splits][G][16] float4 and arrival counters
  // [n_qblocks][nkv][G] (zero before the first launch; each launch leaves them zero)
  float* ws;
  int max_splits, n_items;
};

constexpr int PF_QB = 16;              // queries per prefill-attention workgroup (16 per MFMA column block)
constexpr int PF_STAGERS = 2;          // K/V staging waves per prefill-attention workgroup (beside the G head waves)
constexpr int PF_SPLIT_PAGES = 16;     // KV pages per key split of the persistent form (1024 keys)
constexpr int PF_MAX_ROUNDS = 64;      // items per workgroup of the persistent form (one lane each)

// KV pages of query block qb (keys 0 .. its last query)
__host__ __device__ inline int pf_pages(int pos0, int qb, int P) {
  const int last = (pos0 + qb * PF_QB + PF_QB - 1 < pos0 + P - 1) ? pos0 + qb * PF_QB + PF_QB - 1 : pos0 + P - 1;
  return last / PAGE + 1;
}
// first query block that has a key split s (its pages reach page PF_SPLIT_PAGES s); nqb: none has
__host__ __device__ inline int pf_qmin(int pos0, int P, int s) {
  const int x = PAGE * PF_SPLIT_PAGES * s;               // the split's first key
  if (pos0 + P - 1 < x) return (P + PF_QB - 1) / PF_QB;
  const int q = (x - pos0 - (PF_QB - 1) + PF_QB - 1) / PF_QB;   // ceil((x - pos0 - 15) / 16) where positive
  return x - pos0 - (PF_QB - 1) <= 0 ? 0 : q;
}
__host__ __device__ inline int pf_max_splits(int pos0, int P) { return (pf_pages(pos0, (P + PF_QB - 1) / PF_QB - 1, P) - 1) / PF_SPLIT_PAGES + 1; }
// items of the persistent form: split-major, query blocks longest first, then KV head
__host__ __device__ inline int pf_items(int pos0, int P, int nkv) {
  const int nqb = (P + PF_QB - 1) / PF_QB;
  int n = 0;
  for (int s = 0; pf_qmin(pos0, P, s) < nqb; ++s) n += (nqb - pf_qmin(pos0, P, s)) * nkv;
  return n;
}
__host__ __device__ inline size_t pf_ws_floats(int nqb, int nkv, int G, int max_splits) {
  return (size_t)nqb * nkv * max_splits * G * (8 * 64 * 4 + 16 * 4) + (size_t)nqb * nkv * G;
}

struct AttnArgs {
  const __half* q;             // [T][nh*HD] RoPE'd fp16 queries
  const double* q64;           // the same queries widened to f64 (k_attn_batch_f64)
  const __half* kcache;        // [n_pages][nkv][PAGE][HD]
  const __half* vcache;
  const int* pos;              // [T] position of the token (attends to 0..pos)
  const int* block_table;      // [T][bt_stride]
  int bt_stride;
  int nh, nkv, max_chunks;     // chunk = one page
  double scale;
  double* part;                // [T][nh][max_chunks][HD + 2] partial (o, m, l), f64
  int8_t* oq;                  // [T][nh*HD] Q8_1 output for the O projection (standalone merge)
  half2* ods;                  // [T][nh*HD/32]
  float* o32;                  // optional fp32 output [T][nh*HD] (tests), may be null
  __half* oh;                  // fp16 merged output [T][nh*HD] (the fp16 batched path), instead of oq/ods
  // k_attn_batch_f64: optional list of the live (token, KV head, split) items of this step, one per workgroup in
  // grid order (k_attn_worklist): {token | kvh << 16 | split << 24 (-1: none), pos, page ids of the split's 2 pages}
  const int4* work;
  // with work: one arrival counter per (token, KV head) [T][nkv], zero before the first launch (they reset
  // themselves): the last split to finish merges the token's splits itself (no k_attn_merge_f64 launch)
  int* arrivals;
};

template <int T, int NT, int NW, int KPL, int PRO, int EPI, int WF>
__global__ void k_gemv(const GemvArgs a);
template <int TG, int NT, int NW, int EPI>
__global__ void k_mmq(const GemvArgs a);

}  // namespace q355
