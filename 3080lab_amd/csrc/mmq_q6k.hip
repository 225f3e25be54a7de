// Q6_K x Q8_1 LM head for decode batches on int8 MFMA (v_mfma_i32_16x16x32_i8), gfx950.
//
// Replaces the reference's batched Q6_K head (head_v2_source, lab/qwen_batched.py:681-833): logits of up to 32
// tokens over llama.cpp's Q6_K output.weight and the argmax partials of every 64 rows, read once from HBM.
//
// Weights come in the library's Q6_K planes (lab/gguf.py:tile_q6_k): per 16-row tile and 32-weight block, lo
// (16 B per row: low 4 bits of v_i and v_{i+16}), hi (8 B per row: bits 4-5 of v_{b+8j} at bits 2j of byte b),
// sc (2 int8 sub-block scales per row) and, per 256-weight super-block, d (fp16 per row); weight i of a block is
// d * sc[i / 16] * (v_i - 32). One 32-weight block against 16 tokens is two MFMAs, one per 16-weight sub-block
// (the A operand of the other sub-block's k-groups zeroed), each an exact int32 sum of (v - 32) q_x. Then per
// row sc0 C0 + sc1 C1 (exact int32, |.| < 2^24) is scaled by d d_x (exact fp32 product) into fp32 accumulators.
//
// Workgroup: 4 waves, one 16-row tile each = the 64 rows of one argmax partial; activations of all tokens staged
// in LDS (rows padded by 16 B); weights double-buffered in registers four blocks at a time.
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

constexpr int Q6M_WAVES = 4;
constexpr int Q6M_XPAD = 16;

// the 8 signed values v - 32 of k-group g of one block row: lo = bytes 8 (g & 1) .. + 7 of the row's lo
// bytes (nibble 4 (g >> 1)), hi = the row's 8 hi bytes (bits 2 g .. 2 g + 1). (v + 0x60) ^ 0x80 per byte is
// v - 32 in two's complement for v in 0..63, with no carry between bytes.
__device__ __forceinline__ long q6k_a8(uint2 lo, uint2 hi, int g) {
  const int ls = 4 * (g >> 1), hs = 2 * g;
  const unsigned l0 = (lo.x >> ls) & 0x0F0F0F0Fu, l1 = (lo.y >> ls) & 0x0F0F0F0Fu;
  const unsigned h0 = ((hi.x >> hs) & 0x03030303u) << 4, h1 = ((hi.y >> hs) & 0x03030303u) << 4;
  const unsigned v0 = ((l0 | h0) + 0x60606060u) ^ 0x80808080u, v1 = ((l1 | h1) + 0x60606060u) ^ 0x80808080u;
  return (long)(((unsigned long)v1 << 32) | v0);
}

struct Q6Group {                 // four consecutive blocks of this lane's row slice
  uint2 lo[4], hi[4], sc[4];
  uint2 d;                       // d of rows 4 lg .. 4 lg + 3 in the group's super-block
};

__device__ __forceinline__ void q6m_load(Q6Group& G, const GemvArgs& a, int tile, int grp, int nb, int li, int lg) {
  const int b0 = 4 * min(grp, nb / 4 - 1);             // clamped: loads stay unconditional
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const size_t rb = ((size_t)tile * nb + b0 + u) * 16;
    G.lo[u] = *(const uint2*)(a.qs + (rb + li) * 16 + 8 * (lg & 1));
    G.hi[u] = *(const uint2*)(a.qhi + (rb + li) * 8);
    G.sc[u] = *(const uint2*)(a.qsc + (rb + 4 * lg) * 2);
  }
  G.d = *(const uint2*)(a.d + ((size_t)tile * (nb / 8) + b0 / 8) * 16 + 4 * lg);
}

template <int TG>
__device__ __forceinline__ void q6m_group(const Q6Group& G, const int8_t* xs, int xstride, const float* xd, int nb,
                                          int grp, int li, int lg, float (&acc)[TG][4]) {
  const v4i zero = {0, 0, 0, 0};
  const __half2 d01 = *reinterpret_cast<const __half2*>(&G.d.x), d23 = *reinterpret_cast<const __half2*>(&G.d.y);
  const float dr[4] = {__low2float(d01), __high2float(d01), __low2float(d23), __high2float(d23)};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int b = 4 * grp + u;
    const long a8 = q6k_a8(G.lo[u], G.hi[u], lg);
    const long a0 = lg < 2 ? a8 : 0L, a1 = lg < 2 ? 0L : a8;
    const int sc[8] = {(int)(signed char)(G.sc[u].x), (int)(signed char)(G.sc[u].x >> 8),
                       (int)(signed char)(G.sc[u].x >> 16), (int)(signed char)(G.sc[u].x >> 24),
                       (int)(signed char)(G.sc[u].y), (int)(signed char)(G.sc[u].y >> 8),
                       (int)(signed char)(G.sc[u].y >> 16), (int)(signed char)(G.sc[u].y >> 24)};
    v4i c0[TG], c1[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const long bx = *(const long*)(xs + (size_t)(16 * g + li) * xstride + b * 32 + 8 * lg);
      c0[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bx, zero, 0, 0, 0);
      c1[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bx, zero, 0, 0, 0);
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const float dx = xd[(16 * g + li) * nb + b];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int s = sc[2 * v] * c0[g][v] + sc[2 * v + 1] * c1[g][v];
        acc[g][v] = fmaf(dr[v] * dx, (float)s, acc[g][v]);
      }
    }
  }
}

template <int TG>
__global__ void __launch_bounds__(Q6M_WAVES * 64) k_mmq_q6k_logits(const GemvArgs a) {
  extern __shared__ __align__(16) char q6m_lds[];
  constexpr int TT = 16 * TG;
  const int K = a.K, nb = K / 32, xstride = K + Q6M_XPAD;
  int8_t* xs = (int8_t*)q6m_lds;                                   // [TT][K + 16]
  float* xd = (float*)(q6m_lds + (size_t)TT * xstride);            // [TT][nb]
  __shared__ float pv[Q6M_WAVES][TT];
  __shared__ int pi[Q6M_WAVES][TT];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, li = lane & 15, lg = lane >> 4;
  const int tile = blockIdx.x * Q6M_WAVES + wv;
  Q6Group A, B;
  q6m_load(A, a, tile, 0, nb, li, lg);
  // stage the activations (tokens past T are zero)
  for (int e = threadIdx.x; e < TT * (K / 16); e += Q6M_WAVES * 64) {
    const int j = e / (K / 16), c = e % (K / 16);
    const uint4 v = j < a.T ? *(const uint4*)(a.xq + (size_t)j * K + 16 * c) : make_uint4(0, 0, 0, 0);
    *(uint4*)(xs + (size_t)j * xstride + 16 * c) = v;
  }
  for (int e = threadIdx.x; e < TT * nb; e += Q6M_WAVES * 64) {
    const int j = e / nb, b = e % nb;
    xd[e] = j < a.T ? __low2float(a.xds[(size_t)j * nb + b]) : 0.f;
  }
  __syncthreads();
  float acc[TG][4];
#pragma unroll
  for (int g = 0; g < TG; ++g)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[g][v] = 0.f;
  const int ng = nb / 4;                                            // even: K % 256 == 0
  for (int grp = 0; grp < ng; grp += 2) {
    q6m_load(B, a, tile, grp + 1, nb, li, lg);
    q6m_group<TG>(A, xs, xstride, xd, nb, grp, li, lg, acc);
    q6m_load(A, a, tile, grp + 2, nb, li, lg);
    q6m_group<TG>(B, xs, xstride, xd, nb, grp + 1, li, lg, acc);
  }
  // logits (optional) and the (max, lowest row) of this wave's 16 rows per token
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int tok = 16 * g + li;
    const int row0 = tile * 16 + 4 * lg;
    if (a.y && tok < a.T) *(float4*)(a.y + (size_t)tok * a.N + row0) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    float bv = acc[g][0];
    int bi = row0;
#pragma unroll
    for (int v = 1; v < 4; ++v)
      if (acc[g][v] > bv) { bv = acc[g][v]; bi = row0 + v; }
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lg == 0) { pv[wv][tok] = bv; pi[wv][tok] = bi; }
  }
  __syncthreads();
  if (threadIdx.x < TT && (int)threadIdx.x < a.T) {
    const int tok = threadIdx.x;
    float bv = pv[0][tok];
    int bi = pi[0][tok];
#pragma unroll
    for (int w = 1; w < Q6M_WAVES; ++w)                            // rows increase with w: '>' keeps the lowest
      if (pv[w][tok] > bv) { bv = pv[w][tok]; bi = pi[w][tok]; }
    const int np = a.N / 64;
    a.pmax[(size_t)tok * np + blockIdx.x] = bv;
    a.pidx[(size_t)tok * np + blockIdx.x] = bi;
  }
}

}  // namespace q355
