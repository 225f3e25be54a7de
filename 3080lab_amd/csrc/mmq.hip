// Q4_0 x Q8_1 matrix product on int8 MFMA (v_mfma_i32_16x16x32_i8), gfx950: batched decode
// (T = 5..32 tokens per launch) and prefill (T up to 64 per launch, grid.z over token groups).
//
// One Q4_0 block (k = 32) of one 16-row tile against 16 tokens is exactly one MFMA: A = the tile's
// nibbles (unsigned 0..15 as int8), B = the tokens' int8 activations, C = the exact int32 block dots.
// Then acc[row][tok] += d_w[row] * d_x[tok] * (dot - 8 * sum q_x[tok]) in fp32 -- the reference's MMQ
// formula (lab/qwen_batched.py:1099-1101, 1237-1243), per block so each block keeps its own scales.
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

typedef int v4i __attribute__((ext_vector_type(4)));

// nibbles of one Q4_0 row half (8 bytes) -> the 8 int8 A values of k-group g (g < 2: low, else high)
__device__ __forceinline__ long nib8(uint2 w, int g) {
  const int sh = (g >> 1) * 4;
  const unsigned lo = (w.x >> sh) & 0x0F0F0F0Fu, hi = (w.y >> sh) & 0x0F0F0F0Fu;
  return (long)(((unsigned long)hi << 32) | lo);
}

#ifndef Q355_TRACE_POINT
#define Q355_TRACE_POINT(k)
#endif

// One K block (LDS column bb) against NT tiles x TG token groups: all NT * TG MFMAs are issued before
// any of their results is scaled, so the matrix-core latency overlaps instead of stalling each product.
template <int NT, int TG>
__device__ __forceinline__ void mmq_block(const uint2 (&w)[NT], const uint2 (&dv)[NT], const int8_t* __restrict__ xq, int xstride,
                                          const float* xd, const int* xs, int ld, int bb, int li, int lg,
                                          float (&acc)[NT][TG][4]) {
  v4i c[NT][TG];
  float dx[TG];
  int s8[TG];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int j = 16 * g + li;
    const long bx = *(const long*)(xq + (size_t)j * xstride + bb * 32 + 8 * lg);
    dx[g] = xd[j * ld + bb];
    s8[g] = 8 * xs[j * ld + bb];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const v4i zero = {0, 0, 0, 0};
      c[t][g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(nib8(w[t], lg), bx, zero, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const __half2 d01 = *(const __half2*)&dv[t].x, d23 = *(const __half2*)&dv[t].y;
    const float dw[4] = {__low2float(d01), __high2float(d01), __low2float(d23), __high2float(d23)};
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = fmaf(dw[v] * dx[g], (float)(c[t][g][v] - s8[g]), acc[t][g][v]);
  }
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
  int* xs = (int*)(xd + TT * ch);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;

  const uint2* __restrict__ qs = (const uint2*)a.qs;
  const uint2* __restrict__ dd = (const uint2*)a.d;   // 4 fp16 scales = rows 4*lg .. 4*lg+3
  uint2 wA[NT], dA[NT], wB[NT], dB[NT];
  float acc[NT][TG][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0.f;

  for (int c0 = ks.b0; c0 < ks.b1; c0 += ch) {      // chunks of the K slice
    const int nbc = min(ch, ks.b1 - c0);
    auto load_blk = [&](int bb, uint2 (&w)[NT], uint2 (&dv)[NT]) {
      const int b = c0 + min(bb, nbc - 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const size_t base = ((size_t)(tile0 + t) * nb + b) * 16;
        w[t] = qs[(base + li) * 2 + (lg & 1)];
        dv[t] = dd[(base >> 2) + lg];
      }
    };
    load_blk(wv, wA, dA);                           // first weights of the chunk before the staging
    if (c0 != ks.b0) __syncthreads();               // previous chunk's LDS reads are done
    // stage the activation chunk: task = (token, block): 32 B + d + sum(q); tokens past T are zero
    for (int task = threadIdx.x; task < TT * nbc; task += NW * 64) {
      const int j = task / nbc, bb = task % nbc;
      int4 q0 = make_int4(0, 0, 0, 0), q1 = q0;
      float dx = 0.f;
      if (j < ntok) {
        const int4* src = (const int4*)(a.xq + (size_t)(tok0 + j) * K + (size_t)(c0 + bb) * 32);
        q0 = src[0];
        q1 = src[1];
        dx = __low2float(a.xds[(size_t)(tok0 + j) * nb + c0 + bb]);
      }
      int4* dst = (int4*)(xq + (size_t)j * xstride + bb * 32);
      dst[0] = q0;
      dst[1] = q1;
      const int xv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      xs[j * ch + bb] = sum_i8x32(xv);
      xd[j * ch + bb] = dx;
    }
    __syncthreads();
    Q355_TRACE_POINT(1);

    auto compute_blk = [&](int bb, const uint2 (&w)[NT], const uint2 (&dv)[NT]) {
      mmq_block<NT, TG>(w, dv, xq, xstride, xd, xs, ch, bb, li, lg, acc);
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
  float(&part)[NW][NT][TT][16] = *reinterpret_cast<float(*)[NW][NT][TT][16]>(lds);
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
template <int TG, int NT, int NW, int KPW, int EPI>
__global__ void __launch_bounds__(NW * 64) k_mmq_reg(const GemvArgs a) {
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
  int* xs = (int*)(xd + TT * nbs);
  uint2* wsc = (uint2*)(xs + TT * nbs);                 // [NT][nbs][4] groups of 4 fp16 row scales
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
    for (int t = 0; t < NT; ++t) w[i][t] = qs[(((size_t)(tile0 + t) * nb + b) * 16 + li) * 2 + (lg & 1)];
  }
  __asm__ __volatile__("" ::: "memory");
  // scales of the slice -> LDS (zero for blocks past the slice is not needed: those blocks are skipped)
  for (int e = threadIdx.x; e < NT * nbs * 4; e += NW * 64) {
    const int t = e / (nbs * 4), bb = (e / 4) % nbs, q = e & 3;
    wsc[e] = dd[(((size_t)(tile0 + t) * nb + ks.b0 + bb) * 16 >> 2) + q];
  }
  // activations of the slice -> LDS: task = (token, block): 32 B + d + sum(q); tokens past T are zero
  for (int task = threadIdx.x; task < TT * nbs; task += NW * 64) {
    const int j = task / nbs, bb = task % nbs;
    int4 q0 = make_int4(0, 0, 0, 0), q1 = q0;
    float dx = 0.f;
    if (j < ntok) {
      const int4* src = (const int4*)(a.xq + (size_t)(tok0 + j) * K + (size_t)(ks.b0 + bb) * 32);
      q0 = src[0];
      q1 = src[1];
      dx = __low2float(a.xds[(size_t)(tok0 + j) * nb + ks.b0 + bb]);
    }
    int4* dst = (int4*)(xq + (size_t)j * xstride + bb * 32);
    dst[0] = q0;
    dst[1] = q1;
    const int xv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    xs[j * nbs + bb] = sum_i8x32(xv);
    xd[j * nbs + bb] = dx;
  }
  __syncthreads();
  Q355_TRACE_POINT(1);
  float acc[NT][TG][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][g][v] = 0.f;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int bb = wv + NW * i;
    if (bb < nbs) {                                     // uniform per wave
      uint2 dv[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) dv[t] = wsc[(t * nbs + bb) * 4 + lg];
      mmq_block<NT, TG>(w[i], dv, xq, xstride, xd, xs, nbs, bb, li, lg, acc);
    }
  }
  Q355_TRACE_POINT(2);
  __syncthreads();
  Q355_TRACE_POINT(3);
  float(&part)[NW][NT][TT][16] = *reinterpret_cast<float(*)[NW][NT][TT][16]>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wv][t][16 * g + li][4 * lg + v] = acc[t][g][v];
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

}  // namespace q355
