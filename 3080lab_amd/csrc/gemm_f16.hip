// Q4_0 weights x fp16 activations on fp16 MFMA (v_mfma_f32_16x16x32_f16), gfx950: the batched decode path.
//
// The reference's batched decode GEMV (gemv_v2_source, lab/qwen_batched.py:467-680) dequantizes each Q4_0
// weight to fp16 as d_w (q - 8) -- (q | 0x6400) read as fp16 is 1024 + q, minus 1032 is q - 8 exactly, times
// d_w rounds once -- and multiplies fp16 activations on the tensor cores with fp32 accumulation. Here the
// same products run on the matrix cores: one Q4_0 block (k = 32) of a 16-row tile against 16 tokens is one
// MFMA whose A operand (lane l: row l % 16, k 8 (l / 16) .. +8) is dequantized in registers (8 nibbles ->
// 4 packed fp16 pairs: byte permute, packed subtract, packed multiply), and whose B operand is 8 fp16
// activations from LDS. The accumulator carries the whole K slice: no per-block scaling work.
//
// Workgroup = NT tiles x one K slice (grid.y) x 16 TG tokens (grid.z); NW waves take the slice's blocks
// round robin with a 2-deep register pipeline of weights; the activation chunk is staged in LDS (rows
// padded); partials reduce over waves through LDS into the shared epilogues (STORE, LOGITS, RESID_FIX,
// SWIGLU_F16).
#include "common.h"
#include "q355_kernels.h"

#ifndef Q355_TRACE_POINT
#define Q355_TRACE_POINT(k)
#endif

namespace q355 {

typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef float ff4 __attribute__((ext_vector_type(4)));

// 8 weights of one row (the 8 bytes of its half-block that k-group g reads; g >= 2: high nibbles) -> fp16
// d (q - 8), in k order
__device__ __forceinline__ fh8 deq8(uint2 w, int g, __half d) {
  const int sh = (g >> 1) * 4;
  const unsigned n0 = (w.x >> sh) & 0x0F0F0F0Fu, n1 = (w.y >> sh) & 0x0F0F0F0Fu;
  const __half2 d2 = __halves2half2(d, d), off = __float2half2_rn(1032.f);
  unsigned r[4] = {__builtin_amdgcn_perm(0x64646464u, n0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, n0, 0x04030402u),
                   __builtin_amdgcn_perm(0x64646464u, n1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, n1, 0x04030402u)};
  fh8 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const __half2 v = __hmul2(__hsub2(*reinterpret_cast<const __half2*>(&r[i]), off), d2);
    const unsigned u = *reinterpret_cast<const unsigned*>(&v);
    out[2 * i] = __builtin_bit_cast(_Float16, (unsigned short)(u & 0xFFFFu));
    out[2 * i + 1] = __builtin_bit_cast(_Float16, (unsigned short)(u >> 16));
  }
  return out;
}

template <int TG, int NT, int NW, int EPI>
__global__ void __launch_bounds__(NW * 64) k_gemm_f16(const GemvArgs a) {
  extern __shared__ __align__(16) char lds[];
  constexpr int TT = 16 * TG;                       // tokens per workgroup
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const int tok0 = blockIdx.z * TT;
  const int ntok = min(TT, a.T - tok0);
  const int ch = a.mmq_chunk;                       // K blocks staged in LDS at a time
  const int xrow = ch * 32 + 8;                     // padded LDS row (halves) per token
  _Float16* xs = (_Float16*)lds;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;

  const uint2* wq[NT];                              // this lane's nibbles / row scale of block 0, per tile
  const __half* wd[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    wq[t] = (const uint2*)a.qs + ((size_t)(tile0 + t) * nb * 16 + li) * 2 + (lg & 1);
    wd[t] = a.d + (size_t)(tile0 + t) * nb * 16 + li;
  }
  uint2 wA[NT], wB[NT];
  __half dA[NT], dB[NT];
  ff4 acc[NT][TG];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[t][g] = ff4{0.f, 0.f, 0.f, 0.f};

  for (int c0 = ks.b0; c0 < ks.b1; c0 += ch) {      // chunks of the K slice
    const int nbc = min(ch, ks.b1 - c0);
#define Q355_F16_LOAD(bb, w, dv)                                                                   \
    {                                                                                              \
      const int b_ = c0 + min((bb), nbc - 1);                                                      \
      _Pragma("unroll") for (int t = 0; t < NT; ++t) {                                             \
        w[t] = ld_stream8(wq[t] + b_ * 32);                                                        \
        dv[t] = wd[t][b_ * 16];                                                                    \
      }                                                                                            \
    }
    Q355_F16_LOAD(wv, wA, dA);                      // first weights of the chunk before the staging
    if (c0 != ks.b0) __syncthreads();               // previous chunk's LDS reads are done
    // stage the activation chunk: 16 B pieces (token j, block bb, quarter q); tokens past T are zero
    {
      const int m = 4 * nbc;
      const float inv = 1.f / (float)m;
      for (int p = threadIdx.x; p < TT * m; p += NW * 64) {
        const int j = (int)(((float)p + 0.5f) * inv);   // exact: p / m lies >= 0.5 / m from an integer
        const int r = p - j * m;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (j < ntok) v = *(const uint4*)(a.xh + (size_t)(tok0 + j) * K + (size_t)c0 * 32 + 8 * r);
        *(uint4*)(xs + j * xrow + 8 * r) = v;
      }
    }
    __syncthreads();

#define Q355_F16_BLOCK(bb, w, dv)                                                                  \
    {                                                                                              \
      fh8 A_[NT];                                                                                  \
      _Pragma("unroll") for (int t = 0; t < NT; ++t) A_[t] = deq8(w[t], lg, dv[t]);                \
      _Pragma("unroll") for (int g = 0; g < TG; ++g) {                                             \
        const fh8 B_ = *(const fh8*)(xs + (16 * g + li) * xrow + (bb) * 32 + 8 * lg);              \
        _Pragma("unroll") for (int t = 0; t < NT; ++t)                                             \
          acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_[t], B_, acc[t][g], 0, 0, 0);       \
      }                                                                                            \
    }
    // 2-deep pipeline over this wave's blocks wv, wv + NW, ... of the chunk
    int bb = wv;
    for (; bb + NW < nbc; bb += 2 * NW) {
      Q355_F16_LOAD(bb + NW, wB, dB);
      Q355_F16_BLOCK(bb, wA, dA);
      if (bb + 2 * NW < nbc) Q355_F16_LOAD(bb + 2 * NW, wA, dA);
      Q355_F16_BLOCK(bb + NW, wB, dB);
    }
    if (bb < nbc) Q355_F16_BLOCK(bb, wA, dA);
#undef Q355_F16_LOAD
#undef Q355_F16_BLOCK
  }

  // partials -> LDS (reusing the activation area), then the shared epilogues
  __syncthreads();
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
    b.y = a.y ? a.y + (size_t)tok0 * a.N : nullptr;
    b.yh = a.yh ? a.yh + (size_t)tok0 * (a.N / 2) : nullptr;
    b.yfix = a.yfix ? a.yfix + (size_t)tok0 * a.N : nullptr;
    b.pmax = a.pmax ? a.pmax + (size_t)tok0 * gridDim.x : nullptr;
    b.pidx = a.pidx ? a.pidx + (size_t)tok0 * gridDim.x : nullptr;
  }
  epilogue<NW, TT, NT, EPI>(b, part, tile0);
}

// Decode-batch variant (T <= 16 TG tokens, all in one workgroup): every operand of the workgroup is loaded
// before the first product, so a workgroup pays one memory latency. Wave wv takes blocks b0 + wv + NW i of
// the K slice (i < KPW): its weights, row scales and B operands (16 B of 16 tokens, read straight from
// global memory: each activation element is used by one wave only, so LDS staging would buy nothing) sit in
// registers; partials reduce over waves through LDS into the shared epilogues.
template <int TG, int NT, int NW, int KPW, int EPI>
__global__ void __launch_bounds__(NW * 64) k_gemm_f16r(const GemvArgs a) {
  Q355_TRACE_POINT(0);
  __shared__ float part[NW][NT][16 * TG][16];
  constexpr int TT = 16 * TG;
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT;
  uint2 w[KPW][NT];
  __half dsc[KPW][NT];
  fh8 xb[KPW][TG];
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int b = min(ks.b0 + wv + NW * i, ks.b1 - 1);   // clamped: blocks past the slice are skipped below
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t base = ((size_t)(tile0 + t) * nb + b) * 16 + li;
      w[i][t] = ld_stream8((const uint2*)a.qs + base * 2 + (lg & 1));
      dsc[i][t] = a.d[base];
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const int tok = min(16 * g + li, a.T - 1);          // rows past T re-read the last token, never stored
      xb[i][g] = *(const fh8*)(a.xh + (size_t)tok * K + (size_t)b * 32 + 8 * lg);
    }
  }
  QkvPre qp = {};
  if constexpr (EPI == EPI_QKV) {
    static_assert(NT * TT * 16 <= NW * 64, "one QKV output per thread");
    qp = qkv_prefetch<TT, NT>(a, tile0);
  }
  Q355_TRACE_POINT(1);
  ff4 acc[NT][TG];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[t][g] = ff4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    if (ks.b0 + wv + NW * i < ks.b1) {                    // uniform per wave
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const fh8 A = deq8(w[i][t], lg, dsc[i][t]);
#pragma unroll
        for (int g = 0; g < TG; ++g) acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, xb[i][g], acc[t][g], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wv][t][16 * g + li][4 * lg + v] = acc[t][g][v];
  Q355_TRACE_POINT(2);
  __syncthreads();
  Q355_TRACE_POINT(3);
  if constexpr (EPI == EPI_QKV) qkv_store<NW, TT, NT>(a, part, tile0, qp);
  else epilogue<NW, TT, NT, EPI>(a, part, tile0);
  Q355_TRACE_POINT(5);
}

// Decode-batch O product + residual in the fp16 arithmetic with the split-attention merge in its activation
// staging (T <= 16): workgroup (4 row tiles of 16, query head h = its K slice of 4 blocks, all tokens). Thread
// (token j, 8 dims dg) merges the head's partials (attn_merge8, then fp16 rounding: the bytes
// k_attn_merge_split writes) or reads the fp16 output the attention kernel finished; wave w multiplies block
// 4 h + w; partials reduce over the 4 waves into the fixed-point residual.
__global__ void __launch_bounds__(256) k_gemm_f16_attn_o(const GemvArgs a) {
  constexpr int NT = 4, NW = 4, TT = 16, XR = HD + 8;   // XR: padded LDS row (halves)
  __shared__ __align__(16) _Float16 xs[TT][XR];
  __shared__ float part[NW][NT][TT][16];
  const int K = a.K, nb = K / 32;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * NT, h = blockIdx.y, b = 4 * h + wv;
  uint2 w[NT];
  __half dsc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const size_t base = ((size_t)(tile0 + t) * nb + b) * 16 + li;
    w[t] = ld_stream8((const uint2*)a.qs + base * 2 + (lg & 1));
    dsc[t] = a.d[base];
  }
  {
    const int j = threadIdx.x >> 4, dg = threadIdx.x & 15;
    uint4 v = make_uint4(0, 0, 0, 0);                   // tokens past T stay zero (never stored)
    float o[8];
    if (j < a.T && attn_merge8(a, j, h, dg, o)) {
      unsigned pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const __half2 hv = __floats2half2_rn(o[2 * i], o[2 * i + 1]);
        pk[i] = *reinterpret_cast<const unsigned*>(&hv);
      }
      v = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else if (j < a.T) {
      v = *(const uint4*)(a.xh + (size_t)j * K + (size_t)h * HD + 8 * dg);
    }
    *(uint4*)&xs[j][8 * dg] = v;
  }
  __syncthreads();
  const fh8 xb = *(const fh8*)&xs[li][wv * 32 + 8 * lg];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const ff4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(deq8(w[t], lg, dsc[t]), xb, ff4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wv][t][li][4 * lg + v] = acc[v];
  }
  __syncthreads();
  epilogue<NW, TT, NT, EPI_RESID_FIX>(a, part, tile0);
}

}  // namespace q355
