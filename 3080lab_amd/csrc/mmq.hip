// Q4_0 x Q8_1 matrix product on int8 MFMA (v_mfma_i32_16x16x32_i8), gfx950: batched decode
// (T = 5..32 tokens per launch) and prefill (T up to 64 per launch, grid.z over token groups).
//
// One Q4_0 block (k = 32) of one 16-row tile against 16 tokens is exactly one MFMA: A = the tile's
// weights as int8 16 (q - 8), B = the tokens' int8 activations, C = 16 x the exact int32 block dots
// dot(q - 8, q_x) = dot - 8 sum q_x. Then acc[row][tok] += d_w[row] * (d_x[tok] / 16) * C in fp32, which
// equals d_w d_x (dot - 8 sum q_x) bit for bit -- the reference's MMQ formula
// (lab/qwen_batched.py:1099-1101, 1237-1243), per block so each block keeps its own scales.
// Operand layouts (checked on the GPU): lane l holds A[row l % 16][k = 8 (l / 16) .. +8],
// B[k = 8 (l / 16) .. +8][col l % 16], and C[row 4 (l / 16) + v][col l % 16], v = 0..3.
// Workgroup = NT tiles x one K slice (grid.y) x 16*TG tokens (grid.z token groups); its NW waves take
// the slice's blocks round robin; the activation slice is staged in LDS (rows padded against bank
// conflicts), the weights stream from HBM with a 2-deep register pipeline; partials reduce over waves
// through LDS (reusing the activation area) into the GEMV epilogues (bias / RoPE / KV write, SwiGLU +
// Q8_1, fixed-point residual atomics, logits + argmax partials).
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

typedef float v16f __attribute__((ext_vector_type(16)));

typedef int v4i __attribute__((ext_vector_type(4)));

// nibbles of one Q4_0 row half (8 bytes) -> the 8 int8 values 16 (q - 8) of k-group g
__device__ __forceinline__ long snib8(uint2 w, int g) {
  const int sh = g < 2 ? 4 : 0;
  const unsigned lo = ((w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u, hi = ((w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u;
  return (long)(((unsigned long)hi << 32) | lo);
}

constexpr int TILE_CB = 4;                           // K blocks per LDS chunk

#ifndef Q355_TRACE_POINT
#define Q355_TRACE_POINT(k)
#endif

// acc += (d_w d_x / 16) (16 dot'): both factors are exact in fp32 (a product of two fp16 values; an int32 below
// 2^20), so the f64 form adds the exact block term with one f64 rounding -- decode-batch products accumulate
// in f64, so every Q8_1 quantizer input downstream agrees with the f64 oracle far below a quantization step;
// prefill-size products keep fp32 (their outputs are checked at fp32 tolerance).
__device__ __forceinline__ float mac(float s, int c, float acc) { return fmaf(s, (float)c, acc); }
__device__ __forceinline__ double mac(float s, int c, double acc) { return fma((double)s, (double)c, acc); }
template <int TG> using MmqAcc = typename std::conditional<TG == 1, double, float>::type;

// One K block (LDS column bb) against NT tiles x TG token groups: all NT * TG MFMAs are issued before
// any of their results is scaled, so the matrix-core latency overlaps instead of stalling each product.
// Weights enter as 16 (q - 8) (snib8) and xd holds d_x / 16, so d_w xd (16 dot') = d_w d_x (dot - 8 sum q_x)
// exactly, with no activation sums.
// dwl[q]: d_w of row li of tile 4 q + lg (0 past NT); the d_w d_x products of all outputs come from 4-block
// outer products on the matrix cores (lane l receives d_w[tile][4 lg + v] d_x[token li] in register
// 4 (tile % 4) + v).
template <int NT, int TG, typename ACC, bool HALF = false>
__device__ __forceinline__ void mmq_block(const uint2 (&w)[NT], const float (&dwl)[(NT + 3) / 4], const int8_t* __restrict__ xq,
                                          int xstride, const float* xd, int ld, int bb, int li, int lg, ACC (&acc)[NT][TG][4]) {
  v4i c[NT][TG];
  float dx[TG];
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int j = 16 * g + li;
    const long bx = *(const long*)(xq + (size_t)j * xstride + bb * 32 + 8 * lg);
    dx[g] = xd[j * ld + bb];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      c[t][g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(snib8(w[t], lg), bx, zero, 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const v16f zf = {};
    v16f sc[(NT + 3) / 4];
#pragma unroll
    for (int q = 0; q < (NT + 3) / 4; ++q) sc[q] = __builtin_amdgcn_mfma_f32_16x16x1f32(dwl[q], dx[g], zf, 0, 0, 0);
    if constexpr (HALF) {                              // see k_mmq_r: rows 4 lg + 2, + 3 of token li on lane li + 8
      const bool hi = li >= 8;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const int cs = dpp<DPP_ROR8>(c[t][g][v + 2]);
          const float ss = dpp<DPP_ROR8>(sc[t >> 2][4 * (t & 3) + v + 2]);
          acc[t][g][v] = mac(hi ? ss : sc[t >> 2][4 * (t & 3) + v], hi ? cs : c[t][g][v], acc[t][g][v]);
        }
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][g][v] = mac(sc[t >> 2][4 * (t & 3) + v], c[t][g][v], acc[t][g][v]);
    }
  }
}

// Stage the activations of blocks c0 .. c0 + nbc - 1 for tokens tok0 .. tok0 + TT - 1 into LDS: int8 rows
// (xstride bytes per token) and the fp16 scale / 16 as fp32 (xd, [TT][ld]). One lane per (token, block
// half), 16 bytes each; tokens past ntok are staged as zero.
template <int TT, int NW>
__device__ __forceinline__ void stage_x(const GemvArgs& a, int8_t* xq, float* xd, int xstride, int ld,
                                        int tok0, int ntok, int c0, int nbc) {
  const int K = a.K, nb = K / 32;
  const int m = 2 * nbc;                               // pieces per token
  const float inv = 1.f / (float)m;
  for (int p = threadIdx.x; p < TT * m; p += NW * 64) {
    const int j = (int)(((float)p + 0.5f) * inv);      // exact: p / m lies >= 0.5 / m from an integer
    const int r = p - j * m, bb = r >> 1, h = r & 1;
    int4 q = make_int4(0, 0, 0, 0);
    float dx = 0.f;
    if (j < ntok) {
      q = *(const int4*)(a.xq + (size_t)(tok0 + j) * K + (size_t)(c0 + bb) * 32 + 16 * h);
      if (!h) dx = __low2float(a.xds[(size_t)(tok0 + j) * nb + c0 + bb]) * 0.0625f;
    }
    *(int4*)(xq + (size_t)j * xstride + bb * 32 + 16 * h) = q;
    if (!h) xd[j * ld + bb] = dx;
  }
}

// Stage the O projection's activations of one K slice that is exactly one query head (4 blocks) by merging
// the batched attention's split partials (k_attn_decode_mfma's workspace: per (token, KV head) record o
// [nsp][G][HD] then (M, L) [nsp][G]) and quantizing to Q8_1 -- the arithmetic of k_attn_merge_split, so the
// same bytes -- instead of reading a merged activation. Tokens whose context fits one split were finished by
// the attention kernel: their Q8_1 is read from xq / xds. Thread: token j = tid / 16, dims 8 (tid % 16) ..
// Merge of one (token, query head h, 8 dims dg) over its split-attention partials (the fp32 workspace of
// k_attn_decode_mfma): o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s in split order, the arithmetic of
// k_attn_merge_split. Returns false when the token has one split (the attention kernel finished it itself).
__device__ __forceinline__ bool attn_merge8(const GemvArgs& a, int tok, int h, int dg, float (&o)[8]) {
  const int G = a.nh / a.nkv, kvh = h / G, hl = h % G;
  const int nsp = (a.attn_max_chunks + 3) / 4;
  const int nsplit = (a.pos[tok] / PAGE + 1 + 3) / 4;
  if (nsplit == 1) return false;                       // uniform per token (16 threads)
  const float* wo = (const float*)a.attn_part + ((size_t)tok * a.nkv + kvh) * ((size_t)nsp * G * (HD + 2));
  const float* wm = wo + (size_t)nsp * G * HD;
  float2 ml[16];
  float4 x0[16], x1[16];
#pragma unroll
  for (int sp = 0; sp < 16; ++sp)
    if (sp < nsplit) {
      ml[sp] = *(const float2*)(wm + ((size_t)sp * G + hl) * 2);
      x0[sp] = *(const float4*)(wo + ((size_t)sp * G + hl) * HD + 8 * dg);
      x1[sp] = *(const float4*)(wo + ((size_t)sp * G + hl) * HD + 8 * dg + 4);
    }
  float M = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < 16; ++sp)
    if (sp < nsplit) M = fmaxf(M, ml[sp].x);
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
  for (int sp = 0; sp < 16; ++sp)
    if (sp < nsplit) {
      const float f = __builtin_amdgcn_exp2f(ml[sp].x - M);
      L = fmaf(f, ml[sp].y, L);
      o[0] = fmaf(f, x0[sp].x, o[0]); o[1] = fmaf(f, x0[sp].y, o[1]); o[2] = fmaf(f, x0[sp].z, o[2]);
      o[3] = fmaf(f, x0[sp].w, o[3]); o[4] = fmaf(f, x1[sp].x, o[4]); o[5] = fmaf(f, x1[sp].y, o[5]);
      o[6] = fmaf(f, x1[sp].z, o[6]); o[7] = fmaf(f, x1[sp].w, o[7]);
    }
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] *= inv;
  return true;
}

template <int TT, int NW>
__device__ __forceinline__ void stage_attn(const GemvArgs& a, int8_t* xq, float* xd, int xstride, int ld, int tok0,
                                           int ntok, int b0) {
  static_assert(TT * 16 == NW * 64, "one thread per (token, 8 dims)");
  const int j = threadIdx.x >> 4, dg = threadIdx.x & 15;
  const int h = b0 / 4;
  const int tok = tok0 + j;
  const bool live = j < ntok;
  uint2 pk = make_uint2(0, 0);
  float dx = 0.f;
  float o[8];
  if (live && attn_merge8(a, tok, h, dg, o)) {
    float df;
    int sq;
    pk = q8_1_x8(o, df, sq);                           // the 4 threads of a quad hold one 32-value block
    dx = df * 0.0625f;
  } else if (live) {
    pk = *(const uint2*)(a.xq + (size_t)tok * a.K + (size_t)h * HD + 8 * dg);
    dx = __low2float(a.xds[(size_t)tok * (a.K / 32) + h * 4 + (dg >> 2)]) * 0.0625f;
  }
  *(uint2*)(xq + (size_t)j * xstride + 8 * dg) = pk;
  if ((dg & 3) == 0) xd[j * ld + (dg >> 2)] = dx;
}

// Q8_1 of the 8 fp32 values this lane holds of one 32-block whose 4 quarters sit in lanes l, l ^ 16, l ^ 32,
// l ^ 48 (the MFMA B-operand layout), by the rule of q8_code; df = the fp16 d as float.
__device__ __forceinline__ long q8_1_mfma8(const float (&x)[8], float& df) {
  float amax = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) amax = fmaxf(amax, fabsf(x[u]));
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  const float d32 = q8_scale(amax);
  df = __half2float(__float2half_rn(d32));
  unsigned lo = 0, hi = 0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int v = q8_code(x[u], d32);
    if (u < 4) lo |= (unsigned)(v & 255) << (8 * u);
    else hi |= (unsigned)(v & 255) << (8 * (u - 4));
  }
  return (long)(((unsigned long)hi << 32) | lo);
}

// Decode-batch variant (T <= 16 TG tokens, all in one workgroup): every operand of the workgroup -- weights,
// row scales, activations and their scales -- is loaded before the first product, so a workgroup pays one
// memory latency. Wave wv takes blocks b0 + wv + NW i of the K slice (i < KPW); activations come straight
// from global memory (each element is used by one wave only): Q8_1 (xq / xds), or with XF32 fp32 values
// (xf, the SwiGLU output) quantized to Q8_1 in registers. Partials reduce over waves through LDS.
// HALF (T <= 8, TG == 1): the MFMA's token columns 8..15 are padding, so lane li + 8 takes over rows
// 4 lg + 2, 4 lg + 3 of token li (their products and scales arrive by a DPP swap of the row's halves) and every
// lane accumulates two rows instead of four: half the f64 work, the same arithmetic per output.
template <int TG, int NT, int NW, int KPW, int EPI, bool XF32, bool HALF = false>
__global__ void __launch_bounds__(NW * 64) k_mmq_r(const GemvArgs a) {
  static_assert(!HALF || TG == 1, "the half-column form is for one token group");
  Q355_TRACE_POINT(0);
  __shared__ double part[NW][NT][16 * TG][16];
  constexpr int TT = 16 * TG;
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;
  constexpr int NQ = (NT + 3) / 4;                      // 4-tile groups of the scale outer products
  uint2 w[KPW][NT];
  float dwl[KPW][NQ];                                   // d_w of row li of tile 4 q + lg (0 past NT)
  long xb[KPW][TG];
  float dx[KPW][TG];
  float4 xr[XF32 ? KPW : 1][XF32 ? TG : 1][2];
  constexpr bool DXS = !XF32 && KPW <= 4 && EPI == EPI_QKV;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int b = min(ks.b0 + wv + NW * i, ks.b1 - 1);   // clamped: blocks past the slice are skipped below
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t base = ((size_t)(tile0 + t) * nb + b) * 16;
      w[i][t] = ld_stream8((const uint2*)a.qs + (base + li) * 2 + (lg & 1));
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = 4 * q + lg;
      dwl[i][q] = t < NT ? __half2float(a.d[((size_t)(tile0 + t) * nb + b) * 16 + li]) : 0.f;
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const int tok = min(16 * g + li, a.T - 1);          // rows past T re-read the last token, never stored
      if constexpr (XF32) {
        const float4* src = (const float4*)(a.xf + (size_t)tok * K + (size_t)b * 32 + 8 * lg);
        xr[i][g][0] = src[0];
        xr[i][g][1] = src[1];
      } else {
        xb[i][g] = *(const long*)(a.xq + (size_t)tok * K + (size_t)b * 32 + 8 * lg);
        if constexpr (!DXS) dx[i][g] = __low2float(a.xds[(size_t)tok * nb + b]) * 0.0625f;
      }
    }
  }
  if constexpr (DXS) {
    // activation scales: the 4 lanes of a token (rows lg = 0..3) each load the scale of block i = lg, one
    // load instead of KPW (each touches 16 cache lines: one per token), and the cross-row lane swaps hand
    // every lane the other rows' values. Used by the QKV product (B=32: 9.36 -> 8.03 us per layer); the
    // gate/up product measured slower with it (8.31 -> 8.49 us at B=8)
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const int tok = min(16 * g + li, a.T - 1);
      const int b = min(ks.b0 + wv + NW * min(lg, KPW - 1), ks.b1 - 1);
      const unsigned own = __float_as_uint(__low2float(a.xds[(size_t)tok * nb + b]) * 0.0625f);
      const auto r16 = __builtin_amdgcn_permlane16_swap(own, own, false, false);
      const unsigned p1 = (lane & 16) == 0 ? r16[1] : r16[0];          // row lg ^ 1
      const auto r32 = __builtin_amdgcn_permlane32_swap(own, own, false, false);
      const unsigned p2 = lane < 32 ? r32[1] : r32[0];                 // row lg ^ 2
      const auto r16b = __builtin_amdgcn_permlane16_swap(p2, p2, false, false);
      const unsigned p3 = (lane & 16) == 0 ? r16b[1] : r16b[0];        // row lg ^ 3
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int sel = i ^ lg;
        dx[i][g] = __uint_as_float(sel == 0 ? own : sel == 1 ? p1 : sel == 2 ? p2 : p3);
      }
    }
  }
  if constexpr (XF32) {
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        const float x8[8] = {xr[i][g][0].x, xr[i][g][0].y, xr[i][g][0].z, xr[i][g][0].w,
                             xr[i][g][1].x, xr[i][g][1].y, xr[i][g][1].z, xr[i][g][1].w};
        float df;
        xb[i][g] = q8_1_mfma8(x8, df);
        dx[i][g] = df * 0.0625f;
      }
  }
  QkvPre qp = {};
  if constexpr (EPI == EPI_QKV) {
    static_assert(NT * TT * 16 <= NW * 64, "one QKV output per thread");
    qp = qkv_prefetch<TT, NT>(a, tile0);
  }
  Q355_TRACE_POINT(1);
  double acc[NT][TG][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0.0;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    if (ks.b0 + wv + NW * i < ks.b1) {                    // uniform per wave
      v4i c[NT][TG];
      const v4i zero = {0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const long wa = snib8(w[i][t], lg);
#pragma unroll
        for (int g = 0; g < TG; ++g) c[t][g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xb[i][g], zero, 0, 0, 0);
      }
      // d_w d_x of every output from 4-block outer products on the matrix cores (lane 16 b + r: d_w of row r
      // of tile 4 q + b; lane l receives d_w[tile][4 lg + v] d_x[token li] in register 4 (tile % 4) + v)
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        const v16f zf = {};
        v16f sc[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) sc[q] = __builtin_amdgcn_mfma_f32_16x16x1f32(dwl[i][q], dx[i][g], zf, 0, 0, 0);
        if constexpr (HALF) {
          const bool hi = li >= 8;
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 2; ++v) {
              const int cs = dpp<DPP_ROR8>(c[t][g][v + 2]);
              const float ss = dpp<DPP_ROR8>(sc[t >> 2][4 * (t & 3) + v + 2]);
              acc[t][g][v] = mac(hi ? ss : sc[t >> 2][4 * (t & 3) + v], hi ? cs : c[t][g][v], acc[t][g][v]);
            }
        } else {
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[t][g][v] = mac(sc[t >> 2][4 * (t & 3) + v], c[t][g][v], acc[t][g][v]);
        }
      }
    }
  }
  if constexpr (HALF) {
    const int tok = li & 7, r0 = 4 * lg + 2 * (li >> 3);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      part[wv][t][tok][r0] = acc[t][0][0];
      part[wv][t][tok][r0 + 1] = acc[t][0][1];
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < TG; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wv][t][16 * g + li][4 * lg + v] = acc[t][g][v];
  }
  Q355_TRACE_POINT(2);
  __syncthreads();
  Q355_TRACE_POINT(3);
  if constexpr (EPI == EPI_QKV) qkv_store<NW, TT, NT>(a, part, tile0, qp);
  else epilogue<NW, TT, NT, EPI>(a, part, tile0);
  Q355_TRACE_POINT(5);
}

template <int TG, int NT, int NW, int EPI>
__global__ void __launch_bounds__(NW * 64) k_mmq(const GemvArgs a) {
  extern __shared__ __align__(16) char lds[];
  Q355_TRACE_POINT(0);
  constexpr int TT = 16 * TG;                       // tokens per workgroup
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const int tok0 = blockIdx.z * TT;                 // first token of this workgroup
  const int ntok = min(TT, a.T - tok0);
  const int ch = a.mmq_chunk;                       // K blocks staged in LDS at a time
  const int xstride = ch * 32 + 16;                 // padded LDS row (bytes) per token
  int8_t* xq = (int8_t*)lds;
  float* xd = (float*)(lds + (size_t)TT * xstride);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;

  const uint2* __restrict__ qs = (const uint2*)a.qs;
  constexpr int NQ = (NT + 3) / 4;
  const uint2* wq[NT];                              // this lane's nibbles of block 0, per tile
  const __half* wd[NQ];                             // the scale of row li of tile 4 q + lg, block 0
#pragma unroll
  for (int t = 0; t < NT; ++t) wq[t] = qs + ((size_t)(tile0 + t) * nb * 16 + li) * 2 + (lg & 1);
#pragma unroll
  for (int q = 0; q < NQ; ++q) wd[q] = a.d + (size_t)(tile0 + min(4 * q + lg, NT - 1)) * nb * 16 + li;
  uint2 wA[NT], wB[NT];
  float dA[NQ], dB[NQ];
  using ACC = MmqAcc<TG>;
  ACC acc[NT][TG][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0;

  for (int c0 = ks.b0; c0 < ks.b1; c0 += ch) {      // chunks of the K slice
    const int nbc = min(ch, ks.b1 - c0);
    auto load_blk = [&](int bb, uint2 (&w)[NT], float (&dv)[NQ]) {
      const int b = c0 + min(bb, nbc - 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) w[t] = ld_stream8(wq[t] + b * 32);
#pragma unroll
      for (int q = 0; q < NQ; ++q) dv[q] = 4 * q + lg < NT ? __half2float(wd[q][b * 16]) : 0.f;
    };
    load_blk(wv, wA, dA);                           // first weights of the chunk before the staging
    if (c0 != ks.b0) __syncthreads();               // previous chunk's LDS reads are done
    stage_x<TT, NW>(a, xq, xd, xstride, ch, tok0, ntok, c0, nbc);
    __syncthreads();
    Q355_TRACE_POINT(1);

    auto compute_blk = [&](int bb, const uint2 (&w)[NT], const float (&dv)[NQ]) {
      mmq_block<NT, TG, ACC>(w, dv, xq, xstride, xd, ch, bb, li, lg, acc);
    };
    // 2-deep pipeline over this wave's blocks wv, wv + NW, ... of the chunk
    int bb = wv;
    for (; bb + NW < nbc; bb += 2 * NW) {
      load_blk(bb + NW, wB, dB);
      compute_blk(bb, wA, dA);
      if (bb + 2 * NW < nbc) load_blk(bb + 2 * NW, wA, dA);
      compute_blk(bb + NW, wB, dB);
    }
    if (bb < nbc) compute_blk(bb, wA, dA);
  }

  Q355_TRACE_POINT(2);
  // partials -> LDS (reusing the activation area), then the shared epilogues
  __syncthreads();
  Q355_TRACE_POINT(3);
  ACC(&part)[NW][NT][TT][16] = *reinterpret_cast<ACC(*)[NW][NT][TT][16]>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wv][t][16 * g + li][4 * lg + v] = acc[t][g][v];
  __syncthreads();
  GemvArgs b = a;
  b.T = ntok;                                       // epilogue sees this group's tokens as 0..ntok-1
  if (tok0) {
    b.y = a.y ? a.y + (size_t)tok0 * (EPI == EPI_SWIGLU ? a.N / 2 : a.N) : nullptr;
    b.yfix = a.yfix ? a.yfix + (size_t)tok0 * a.N : nullptr;
    b.pos = a.pos ? a.pos + tok0 : nullptr;
    b.qout = a.qout ? a.qout + (size_t)tok0 * a.nh * HD : nullptr;
    b.oq = a.oq ? a.oq + (size_t)tok0 * (a.N / 2) : nullptr;
    b.ods = a.ods ? a.ods + (size_t)tok0 * (a.N / 64) : nullptr;
    b.pmax = a.pmax ? a.pmax + (size_t)tok0 * gridDim.x : nullptr;
    b.pidx = a.pidx ? a.pidx + (size_t)tok0 * gridDim.x : nullptr;
    b.tok_base = a.tok_base + tok0;
  }
  epilogue<NW, TT, NT, EPI>(b, part, tile0);
  Q355_TRACE_POINT(5);
}

// Decode-sized variant: every weight block of this workgroup's K slice is loaded into registers before
// the activations are staged (wave wv takes blocks b0 + wv + NW i, i < KPW; the slice must have at most
// NW * KPW blocks), so the HBM latency is paid once per workgroup instead of once per pipeline step. The
// slice's scales go through LDS with the activations (registers hold only the nibbles).
template <int TG, int NT, int NW, int KPW, int EPI, bool ATT = false, bool HALF = false>
__global__ void __launch_bounds__(NW * 64) k_mmq_reg(const GemvArgs a) {
  static_assert(!HALF || TG == 1, "the half-column form is for one token group");
  extern __shared__ __align__(16) char lds[];
  Q355_TRACE_POINT(0);
  constexpr int TT = 16 * TG;
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const int nbs = ks.b1 - ks.b0;
  const int tok0 = blockIdx.z * TT;
  const int ntok = min(TT, a.T - tok0);
  const int xstride = nbs * 32 + 16;
  int8_t* xq = (int8_t*)lds;
  float* xd = (float*)(lds + (size_t)TT * xstride);
  uint2* wsc = (uint2*)(xd + 2 * TT * nbs);             // [NT][nbs][4] groups of 4 fp16 row scales
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;
  const uint2* __restrict__ qs = (const uint2*)a.qs;
  const uint2* __restrict__ dd = (const uint2*)a.d;
  uint2 w[KPW][NT];
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int b = ks.b0 + min(wv + NW * i, nbs - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) w[i][t] = ld_stream8(qs + (((size_t)(tile0 + t) * nb + b) * 16 + li) * 2 + (lg & 1));
  }
  __asm__ __volatile__("" ::: "memory");
  // scales of the slice -> LDS (zero for blocks past the slice is not needed: those blocks are skipped)
  for (int e = threadIdx.x; e < NT * nbs * 4; e += NW * 64) {
    const int t = e / (nbs * 4), bb = (e / 4) % nbs, q = e & 3;
    wsc[e] = dd[(((size_t)(tile0 + t) * nb + ks.b0 + bb) * 16 >> 2) + q];
  }
  // activations of the slice -> LDS (ATT: merged from the attention's split partials, one head per slice)
  if constexpr (ATT) stage_attn<TT, NW>(a, xq, xd, xstride, nbs, tok0, ntok, ks.b0);
  else stage_x<TT, NW>(a, xq, xd, xstride, nbs, tok0, ntok, ks.b0, nbs);
  __syncthreads();
  Q355_TRACE_POINT(1);
  using ACC = MmqAcc<TG>;
  ACC acc[NT][TG][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int bb = wv + NW * i;
    if (bb < nbs) {                                     // uniform per wave
      float dv[(NT + 3) / 4];                           // wsc as fp16 [NT][nbs][16 rows]
#pragma unroll
      for (int q = 0; q < (NT + 3) / 4; ++q)
        dv[q] = 4 * q + lg < NT ? __half2float(((const __half*)wsc)[((4 * q + lg) * nbs + bb) * 16 + li]) : 0.f;
      mmq_block<NT, TG, ACC, HALF>(w[i], dv, xq, xstride, xd, nbs, bb, li, lg, acc);
    }
  }
  Q355_TRACE_POINT(2);
  __syncthreads();
  Q355_TRACE_POINT(3);
  ACC(&part)[NW][NT][TT][16] = *reinterpret_cast<ACC(*)[NW][NT][TT][16]>(lds);
  if constexpr (HALF) {
    const int tok = li & 7, r0 = 4 * lg + 2 * (li >> 3);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      part[wv][t][tok][r0] = acc[t][0][0];
      part[wv][t][tok][r0 + 1] = acc[t][0][1];
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < TG; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wv][t][16 * g + li][4 * lg + v] = acc[t][g][v];
  }
  __syncthreads();
  GemvArgs b = a;
  b.T = ntok;
  if (tok0) {
    b.y = a.y ? a.y + (size_t)tok0 * (EPI == EPI_SWIGLU ? a.N / 2 : a.N) : nullptr;
    b.yfix = a.yfix ? a.yfix + (size_t)tok0 * a.N : nullptr;
    b.pos = a.pos ? a.pos + tok0 : nullptr;
    b.qout = a.qout ? a.qout + (size_t)tok0 * a.nh * HD : nullptr;
    b.oq = a.oq ? a.oq + (size_t)tok0 * (a.N / 2) : nullptr;
    b.ods = a.ods ? a.ods + (size_t)tok0 * (a.N / 64) : nullptr;
    b.pmax = a.pmax ? a.pmax + (size_t)tok0 * gridDim.x : nullptr;
    b.pidx = a.pidx ? a.pidx + (size_t)tok0 * gridDim.x : nullptr;
    b.tok_base = a.tok_base + tok0;
  }
  epilogue<NW, TT, NT, EPI>(b, part, tile0);
  Q355_TRACE_POINT(5);
}

// Prefill-size GEMM tile: a workgroup computes (RW * 64 rows) x (CW * 16 TG tokens) with RW x CW = 4 waves,
// each wave a 64 x 16 TG sub-tile (4 row tiles x TG token groups, 4 TG MFMAs per K block) over the full K slice.
// K advances in chunks of CB blocks staged in LDS, double-buffered: the global loads of chunk c + 1 are
// issued (16 B per lane, contiguous) before chunk c is computed, and written to the other buffer after.
// The weights enter the MFMA as signed int8 16 (q - 8): nibble moved to the high half of the byte with its
// top bit flipped, so no -8 sum(q_x) correction is needed; the 16 is folded into the activation scale,
// stored as d_x / 16 (exact), so d_w (d_x / 16) (16 dot) is bit-identical to d_w d_x dot.
// LDS per buffer (block-major inside each tile / token group, so every MFMA operand read is one
// contiguous, conflict-free 512 B wave read):
//   A  [RW*4 tiles][CB][16 rows][16 B]     nibbles as stored in HBM
//   W  [RW*4 tiles][CB][16]                row scales (fp32)
//   B  [CW*TG groups][CB][16 tokens][32 B] int8 activations; tokens 8..15 of a group swap their 16 B
//                                          halves, so the two half-wave reads of a B operand use all banks
//   X  [CB][CW*16*TG]                      activation scale / 16 (fp32)
// Epilogues from registers: STORE, RESID_FIX (plain read-add-write: each output has one writer),
// SWIGLU_Q8 (rows interleaved g0, u0, ...: each 64-row tile group is one Q8_1 block per token), LOGITS
// (fp32 logits + one (max, row) partial per 64 rows and token, the layout of the other LOGITS kernels).
template <int RW, int CW, int TG, int CB>
struct LdsTile {
  static constexpr int TW = CW * 16 * TG;            // tokens per workgroup
  static constexpr int A = RW * 4 * CB * 256, W = RW * 4 * CB * 64, B = CW * TG * CB * 512;
  static constexpr int X = CB * TW * 4;
  static constexpr int BUF = A + W + B + X;
};

template <int RW, int CW, int TG, int EPI>
__global__ void __launch_bounds__(256) k_mmq_tile(const GemvArgs a) {
  constexpr int CB = TILE_CB;
  using L = LdsTile<RW, CW, TG, CB>;
  constexpr int TW = L::TW;
  constexpr int NTH = RW * CW * 64;                  // threads
  constexpr int NA = RW * 4 * CB * 16;               // 16-byte pieces of A per chunk
  constexpr int NWp = RW * 4 * CB * 2;               // of W (fp16 in HBM)
  constexpr int NBp = TW * CB * 2;                   // of B (two per token and block)
  static_assert(NA % NTH == 0 && NBp % NTH == 0 && NWp <= NTH, "staging shape");
  extern __shared__ __align__(16) char lds[];
  const int K = a.K, nb = K / 32, N = a.N;
  const KSlice ks(nb);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int wr = wv / CW, wc = wv % CW;              // this wave's row block and token block
  const int tile0 = blockIdx.x * RW * 4;             // first 16-row tile of the workgroup
  const int tok0 = blockIdx.z * TW;                  // first token of the workgroup
  const int tid = threadIdx.x;

  // staging registers for one chunk
  uint4 rA[NA / NTH], rB[NBp / NTH], rW;
  half2 rX[NBp / NTH];
  const uint4* __restrict__ gA = (const uint4*)a.qs;
  const uint4* __restrict__ gW = (const uint4*)a.d;

#define Q355_TILE_LOAD(c0)                                                                        \
  {                                                                                               \
    const int cb_ = (c0);                                                                         \
    _Pragma("unroll") for (int i = 0; i < NA / NTH; ++i) {                                        \
      const int p = tid + NTH * i, t = p / (CB * 16), r = p % (CB * 16), blk = r >> 4;            \
      rA[i] = cb_ + blk < ks.b1 ? gA[((size_t)(tile0 + t) * nb + cb_) * 16 + r] : make_uint4(0, 0, 0, 0); \
    }                                                                                             \
    if (tid < NWp) {                                                                              \
      const int t = tid / (CB * 2), r = tid % (CB * 2), blk = r >> 1;                             \
      rW = cb_ + blk < ks.b1 ? gW[((size_t)(tile0 + t) * nb + cb_) * 2 + r] : make_uint4(0, 0, 0, 0); \
    }                                                                                             \
    _Pragma("unroll") for (int i = 0; i < NBp / NTH; ++i) {                                       \
      const int p = tid + NTH * i, h = p & 1, j = (p >> 1) % TW, blk = p / (2 * TW);              \
      const bool ok = tok0 + j < a.T && cb_ + blk < ks.b1;                                        \
      rB[i] = ok ? *(const uint4*)(a.xq + (size_t)(tok0 + j) * K + (size_t)(cb_ + blk) * 32 + 16 * h) \
                 : make_uint4(0, 0, 0, 0);                                                        \
      rX[i] = ok && !h ? a.xds[(size_t)(tok0 + j) * nb + cb_ + blk] : half2{};                    \
    }                                                                                             \
  }

#define Q355_TILE_STORE(buf)                                                                      \
  {                                                                                               \
    char* base_ = lds + (buf) * L::BUF;                                                           \
    _Pragma("unroll") for (int i = 0; i < NA / NTH; ++i)                                          \
      *(uint4*)(base_ + (size_t)(tid + NTH * i) * 16) = rA[i];                                    \
    if (tid < NWp) {                                                                              \
      const __half2* h_ = (const __half2*)&rW;                                                    \
      float4* dst_ = (float4*)(base_ + L::A + tid * 32);                                          \
      dst_[0] = make_float4(__low2float(h_[0]), __high2float(h_[0]), __low2float(h_[1]), __high2float(h_[1])); \
      dst_[1] = make_float4(__low2float(h_[2]), __high2float(h_[2]), __low2float(h_[3]), __high2float(h_[3])); \
    }                                                                                             \
    _Pragma("unroll") for (int i = 0; i < NBp / NTH; ++i) {                                       \
      const int p = tid + NTH * i, h = p & 1, j = (p >> 1) % TW, blk = p / (2 * TW);              \
      *(uint4*)(base_ + L::A + L::W + (((j >> 4) * CB + blk) * 16 + (j & 15)) * 32 +              \
                16 * (h ^ ((j >> 3) & 1))) = rB[i];                                               \
      if (!h) ((float*)(base_ + L::A + L::W + L::B))[blk * TW + j] = __low2float(rX[i]) * 0.0625f; \
    }                                                                                             \
  }

  float acc[4][TG][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0.f;

  int buf = 0;
  if (ks.b0 < ks.b1) {
    Q355_TILE_LOAD(ks.b0);
    Q355_TILE_STORE(0);
  }
  __syncthreads();
  for (int c0 = ks.b0; c0 < ks.b1; c0 += CB) {
    const bool more = c0 + CB < ks.b1;               // uniform
    if (more) Q355_TILE_LOAD(c0 + CB);
    const char* base = lds + buf * L::BUF;
    const char* sA = base + (size_t)(wr * 4) * CB * 256;
    const char* sW = base + L::A + (size_t)(wr * 4) * CB * 64;
    const char* sB = base + L::A + L::W + (size_t)(wc * TG) * CB * 512;
    const float* sX = (const float*)(base + L::A + L::W + L::B) + wc * 16 * TG;
#pragma unroll 1
    for (int blk = 0; blk < CB; ++blk) {
      long w[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = snib8(*(const uint2*)(sA + (t * CB + blk) * 256 + li * 16 + (lg & 1) * 8), lg);
      // the block scales d_w d_x of all 4 x 16 x 16 outputs of a token group in ONE 4-block outer product on
      // the matrix cores (v_mfma_f32_16x16x1f32: block t = tile t; lane 16 t + r supplies d_w of row r, every
      // lane d_x of its token li; lane l receives d_w[t][4 lg + v] d_x[li] in register 4 t + v): the 16
      // exact fp32 products that would otherwise be 16 VALU multiplies
      const float wl = *(const float*)(sW + (lg * CB + blk) * 64 + li * 4);
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        const long bx = *(const long*)(sB + ((g * CB + blk) * 16 + li) * 32 + (lg ^ ((li >> 3) << 1)) * 8);
        const float dx = sX[blk * TW + g * 16 + li];
        const v4i zero = {0, 0, 0, 0};
        const v16f zf = {};
        const v16f sc = __builtin_amdgcn_mfma_f32_16x16x1f32(wl, dx, zf, 0, 0, 0);
        v4i c[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) c[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(w[t], bx, zero, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][g][v] = fmaf(sc[4 * t + v], (float)c[t][v], acc[t][g][v]);
      }
    }
    if (more) {
      Q355_TILE_STORE(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
#undef Q355_TILE_LOAD
#undef Q355_TILE_STORE

  const int rt0 = tile0 + wr * 4;                    // this wave's first row tile
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int tok = tok0 + wc * 16 * TG + g * 16 + li;
    const bool ok = tok < a.T;
    if (EPI == EPI_STORE) {
      if (ok)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          *(float4*)(a.y + (size_t)tok * N + (rt0 + t) * 16 + 4 * lg) =
              make_float4(acc[t][g][0], acc[t][g][1], acc[t][g][2], acc[t][g][3]);
    } else if (EPI == EPI_RESID_FIX) {
      if (ok) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          long long* y = a.yfix + (size_t)tok * N + (rt0 + t) * 16 + 4 * lg;
          if (gridDim.y == 1) {                      // this lane owns these 4 sums: plain read-add-write
            longlong2* y2 = (longlong2*)y;
            longlong2 p0 = y2[0], p1 = y2[1];
            p0.x += to_fix((double)acc[t][g][0]); p0.y += to_fix((double)acc[t][g][1]);
            p1.x += to_fix((double)acc[t][g][2]); p1.y += to_fix((double)acc[t][g][3]);
            y2[0] = p0;
            y2[1] = p1;
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              atomicAdd((unsigned long long*)(y + v), (unsigned long long)to_fix((double)acc[t][g][v]));
          }
        }
      }
    } else if (EPI == EPI_LOGITS) {
      // fp32 logits, and this wave's (max, lowest row) over its 64 rows: partial rt0 / 4 of N / 64
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (ok && a.y)                                   // fp32 logits are optional: the argmax needs only partials
          *(float4*)(a.y + (size_t)tok * N + (rt0 + t) * 16 + 4 * lg) =
              make_float4(acc[t][g][0], acc[t][g][1], acc[t][g][2], acc[t][g][3]);
#pragma unroll
        for (int v = 0; v < 4; ++v)                      // rows increase with (t, v): strict '>' keeps the lowest
          if (acc[t][g][v] > bv) { bv = acc[t][g][v]; bi = (rt0 + t) * 16 + 4 * lg + v; }
      }
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (ok && lg == 0) {
        const int np = N / 64;
        a.pmax[(size_t)tok * np + rt0 / 4] = bv;
        a.pidx[(size_t)tok * np + rt0 / 4] = bi;
      }
    } else if (EPI == EPI_QKV) {
      // + bias, RoPE, fp16 q / K / V (one f64 -> fp16 rounding each, as k_qkv_finish): this lane's rows
      // 4 lg + v of each tile are the RoPE pairs (v = 0, 1) and (2, 3) of the device row order
      if (ok) {
        const int nq = a.nh * HD, nk = a.nkv * HD;
        const int pos = a.pos[tok];
        const int pg = a.block_table[(size_t)(tok * a.seq_stride) * a.bt_stride + pos / PAGE];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            const int row = (rt0 + t) * 16 + 4 * lg + 2 * pp;
            const double v0 = (double)acc[t][g][2 * pp] + (double)a.aux[row];
            const double v1 = (double)acc[t][g][2 * pp + 1] + (double)a.aux[row + 1];
            if (row < nq + nk) {
              const int i = (row % HD) >> 1;           // pair (dim i, dim i + 64)
              const double c = a.rope_cos[(size_t)pos * (HD / 2) + i], sn = a.rope_sin[(size_t)pos * (HD / 2) + i];
              const __half lo = half_rn(v0 * c - v1 * sn), hi = half_rn(v1 * c + v0 * sn);
              __half* dst = row < nq ? a.qout + (size_t)tok * nq + (row / HD) * HD
                                     : a.kcache + (((size_t)pg * a.nkv + (row - nq) / HD) * PAGE + pos % PAGE) * HD;
              dst[i] = lo;
              dst[i + HD / 2] = hi;
              if (row < nq && a.qout64) {
                double* d64 = a.qout64 + (size_t)tok * nq + (row / HD) * HD;
                d64[i] = (double)__half2float(lo);
                d64[i + HD / 2] = (double)__half2float(hi);
              }
            } else {
              const int rv = row - nq - nk;
              __half2* vd = (__half2*)(a.vcache + (((size_t)pg * a.nkv + rv / HD) * PAGE + pos % PAGE) * HD + rv % HD);
              *vd = __halves2half2(half_rn(v0), half_rn(v1));
            }
          }
      }
    } else if (EPI == EPI_SWIGLU_Q8) {
      // this lane holds outputs 8t + 2lg, 8t + 2lg + 1 of its wave's 32; the 4 lanes of token li hold all 32
      float o[4][2];
      float amax = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        o[t][0] = silu_mul_f(acc[t][g][0], acc[t][g][1]);
        o[t][1] = silu_mul_f(acc[t][g][2], acc[t][g][3]);
        amax = fmaxf(amax, fmaxf(fabsf(o[t][0]), fabsf(o[t][1])));
      }
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const float d32 = q8_scale(amax);
      int sq = 0;
      unsigned short pk[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int q0 = q8_code(o[t][0], d32), q1 = q8_code(o[t][1], d32);
        sq += q0 + q1;
        pk[t] = (unsigned short)((q0 & 255) | ((q1 & 255) << 8));
      }
      sq += __shfl_xor(sq, 16);
      sq += __shfl_xor(sq, 32);
      if (ok) {
        const int Nout = N / 2, ob = rt0 / 4;        // output Q8_1 block of this wave's 64 rows
        int8_t* dst = a.oq + (size_t)tok * Nout + ob * 32 + 2 * lg;
#pragma unroll
        for (int t = 0; t < 4; ++t) *(unsigned short*)(dst + 8 * t) = pk[t];
        if (lg == 0) a.ods[(size_t)tok * (Nout / 32) + ob] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
      }
    }
  }
}

}  // namespace q355
