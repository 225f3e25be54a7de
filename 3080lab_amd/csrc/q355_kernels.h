// Kernel argument blocks and template dispatch shared by the kernel files and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace q355 {

enum Prologue { PRO_Q8 = 0, PRO_RMS = 1 };
enum Epilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_BIAS = 2, EPI_QKV = 3, EPI_SWIGLU_Q8 = 4, EPI_LOGITS = 5 };

constexpr int HD = 128;        // head dim (Qwen2.5-1.5B)
constexpr int PAGE = 64;       // KV cache page: 64 positions of one KV head, [PAGE][HD] fp16

// Everything a GEMV-family launch may need; unused fields are null/zero.
struct GemvArgs {
  const uint8_t* qs;           // Q4_0 nibble plane [N/16][K/32][16][16]
  const __half* d;             // Q4_0 scale plane  [N/16][K/32][16]
  int N, K, T;
  // PRO_Q8 input
  const int8_t* xq;            // [T][K]
  const half2* xds;            // [T][K/32]
  // PRO_RMS input
  const float* h;              // [T][K] fp32 residual stream
  const float* nw;             // [K] RMSNorm weight
  float eps;
  // STORE / RESID / BIAS / LOGITS output
  float* y;                    // [T][N]
  const float* aux;            // bias [N] (BIAS, QKV: bias in the permuted row order)
  // QKV epilogue: RoPE on q/k (rows of each head interleaved (d, d+64)), fp16 q out, K/V cache write
  const float* rope_cos;       // [maxlen][HD/2]
  const float* rope_sin;
  const int* pos;              // [T] position of each token
  const int* block_table;      // [n_seq][bt_stride] page ids
  int bt_stride;
  int seq_stride;              // token j belongs to sequence j * seq_stride (1: batched decode, 0: one sequence)
  __half* kcache;              // [n_pages][nkv][PAGE][HD]
  __half* vcache;
  __half* qout;                // [T][nh*HD]
  int nh, nkv;
  // SWIGLU_Q8 output (rows interleaved gate, up): Q8_1 of silu(g) * u, [T][N/2]
  int8_t* oq;
  half2* ods;
  // LOGITS: per-workgroup (max, index) partials [T][gridDim.x]
  float* pmax;
  int* pidx;
};

struct AttnArgs {
  const __half* q;             // [T][nh*HD] RoPE'd fp16 queries
  const __half* kcache;        // [n_pages][nkv][PAGE][HD]
  const __half* vcache;
  const int* pos;              // [T] position of the token (attends to 0..pos)
  const int* block_table;      // [T][bt_stride]
  int bt_stride;
  int nh, nkv, max_chunks;     // chunk = one page
  float scale;
  float* part;                 // [T][nh][max_chunks][HD + 2] partial (o, m, l)
  unsigned* counter;           // [T][nkv] arrival counters (self-resetting)
  int8_t* oq;                  // [T][nh*HD] Q8_1 output for the O projection
  half2* ods;                  // [T][nh*HD/32]
  float* o32;                  // optional fp32 output [T][nh*HD] (tests), may be null
};

template <int T, int NT, int PRO, int EPI>
__global__ void k_gemv(const GemvArgs a);

}  // namespace q355
