// Q8_1 quantizers and the Q4_0 x Q8_1 GEMV (1..4 tokens) with fused prologues/epilogues, gfx950.
//
// GEMV work split: a workgroup of 4 waves owns NT 16-row tiles; the 4 waves x 4 lane slots split
// the K blocks 16 ways (block b goes to k-lane b % 16), lane (slot, row) streams 16 B of nibbles per
// block (1 KB contiguous per wave instruction) and dots it with the activation block held in LDS
// (v_dot4_i32_i8, exact int32). Partials reduce over slots (lane xor 16, 32) and over waves through
// LDS in a fixed order, so results are bitwise reproducible run to run.
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

// ---------------------------------------------------------------------------------------------
// Standalone Q8_1 quantizer: x fp32 [T][K] -> xq, xds. One 32-lane group per block.
__global__ void __launch_bounds__(256) k_quant_q8_1(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                    half2* __restrict__ xds, long nblk) {
  long blk = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  int lane = threadIdx.x & 31;
  if (blk >= nblk) return;  // whole 32-lane groups exit together
  float v = x[blk * 32 + lane];
  int q = q8_1_lane32(v, xds + blk, lane == 0);
  xq[blk * 32 + lane] = (int8_t)q;
}

// RMSNorm(h) * w -> Q8_1 for one token per workgroup (grid.x = T). H % 32 == 0, H <= 256 * 8.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
  return s;
}

__global__ void __launch_bounds__(256) k_rmsnorm_q8_1(const float* __restrict__ h, const float* __restrict__ w,
                                                      int8_t* __restrict__ xq, half2* __restrict__ xds, int H,
                                                      float eps) {
  __shared__ float red[8];
  const int tok = blockIdx.x;
  const float* hr = h + (size_t)tok * H;
  float ss = 0.f;
  float v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    int i = threadIdx.x + 256 * u;
    v[u] = i < H ? hr[i] : 0.f;
    ss += v[u] * v[u];
  }
  float r = 1.0f / sqrtf(block_sum_256(ss, red) / (float)H + eps);
  // values i = threadIdx.x + 256u: lanes 0..31 of a wave hold one 32-block for each u
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    int i = threadIdx.x + 256 * u;
    if (256 * u < H) {  // uniform per u: H % 256 may leave a partial row of blocks; i < H is 32-aligned per group
      bool act = i < H;
      float x = act ? v[u] * r * w[i] : 0.f;
      int q = q8_1_lane32(x, xds + (size_t)tok * (H / 32) + (i >> 5), act && (threadIdx.x & 31) == 0);
      if (act) xq[(size_t)tok * H + i] = (int8_t)q;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// LDS staging of the activation operand: xq bytes [T][K], dx float [T][nb], sq int [T][nb].
struct XStage {
  int8_t* q;
  float* d;
  int* s;
};

__device__ __forceinline__ XStage xstage_carve(char* lds, int T, int K) {
  XStage s;
  s.q = (int8_t*)lds;
  s.d = (float*)(lds + (size_t)T * K);
  s.s = (int*)(lds + (size_t)T * K + (size_t)T * (K / 32) * 4);
  return s;
}

// Pre-quantized input: copy xq/xds into LDS and precompute per-block sums.
__device__ __forceinline__ void prologue_q8(const XStage& st, const int8_t* __restrict__ xq,
                                            const half2* __restrict__ xds, int T, int K) {
  const int nb = K / 32;
  for (int task = threadIdx.x; task < T * nb; task += blockDim.x) {
    const int4* src = (const int4*)(xq + (size_t)task * 32);
    int4 a = src[0], b = src[1];
    int4* dst = (int4*)(st.q + (size_t)task * 32);
    dst[0] = a;
    dst[1] = b;
    int xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    st.s[task] = sum_i8x32(xv);
    st.d[task] = __low2float(xds[task]);
  }
}

// Fused RMSNorm + Q8_1 prologue: h fp32 [T][K] normalized with nw, quantized into LDS.
__device__ __forceinline__ void prologue_rms(const XStage& st, const float* __restrict__ h,
                                             const float* __restrict__ nw, float eps, int T, int K, float* red) {
  for (int tok = 0; tok < T; ++tok) {
    const float* hr = h + (size_t)tok * K;
    float v[8];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int i = threadIdx.x + 256 * u;
      v[u] = i < K ? hr[i] : 0.f;
      ss += v[u] * v[u];
    }
    float r = 1.0f / sqrtf(block_sum_256(ss, red) / (float)K + eps);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int i = threadIdx.x + 256 * u;
      if (256 * u < K) {
        bool act = i < K;
        float x = act ? v[u] * r * nw[i] : 0.f;
        float amax = wave_max<32>(fabsf(x));
        __half d16 = __float2half_rn(amax / 127.0f);
        float df = __half2float(d16);
        int q = 0;
        if (df != 0.0f) {
          q = (int)roundf(x / df);
          q = q > 127 ? 127 : (q < -127 ? -127 : q);
        }
        int sq = wave_isum<32>(q);
        if (act) {
          st.q[(size_t)tok * K + i] = (int8_t)q;
          if ((threadIdx.x & 31) == 0) {
            st.d[tok * (K / 32) + (i >> 5)] = df;
            st.s[tok * (K / 32) + (i >> 5)] = sq;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Epilogues. part[w][t][j][r] holds wave w's partial of row (tile0 + t) * 16 + r for token j.
template <int T, int NT>
__device__ __forceinline__ float row_value(float (&part)[4][NT][T][16], int t, int j, int r) {
  return ((part[0][t][j][r] + part[1][t][j][r]) + part[2][t][j][r]) + part[3][t][j][r];
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int T, int NT, int EPI>
__device__ __forceinline__ void epilogue(const GemvArgs& a, float (&part)[4][NT][T][16], int tile0) {
  const int N = a.N;
  if (EPI == EPI_SWIGLU_Q8) {
    // NT == 4: 64 interleaved rows (g0, u0, g1, u1, ...) -> 32 outputs = one Q8_1 block per token
    const int j = threadIdx.x >> 5, k = threadIdx.x & 31;
    if (j < T && j < a.T) {
      const int rg = 2 * k, ru = 2 * k + 1;
      float g = row_value<T, NT>(part, rg >> 4, j, rg & 15);
      float u = row_value<T, NT>(part, ru >> 4, j, ru & 15);
      float m = silu_mul(g, u);
      const int Nout = N / 2;
      int q = q8_1_lane32(m, a.ods + (size_t)j * (Nout / 32) + blockIdx.x, k == 0);
      a.oq[(size_t)j * Nout + blockIdx.x * 32 + k] = (int8_t)q;
    }
    return;
  }
  if (EPI == EPI_LOGITS) {
    __shared__ float vals[T][NT * 16];
    for (int e = threadIdx.x; e < NT * T * 16; e += blockDim.x) {
      const int t = e / (T * 16), j = (e >> 4) % T, r = e & 15;
      float v = row_value<T, NT>(part, t, j, r);
      vals[j][t * 16 + r] = v;
      if (j < a.T) a.y[(size_t)j * N + (tile0 + t) * 16 + r] = v;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      for (int j = 0; j < T && j < a.T; ++j) {
        float v = l < NT * 16 ? vals[j][l] : -INFINITY;
        int idx = l < NT * 16 ? tile0 * 16 + l : 0x7fffffff;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          float ov = __shfl_xor(v, o, 64);
          int oi = __shfl_xor(idx, o, 64);
          if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
        }
        if (l == 0) {
          a.pmax[(size_t)j * gridDim.x + blockIdx.x] = v;
          a.pidx[(size_t)j * gridDim.x + blockIdx.x] = idx;
        }
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < NT * T * 16; e += blockDim.x) {
    const int t = e / (T * 16), j = (e >> 4) % T, r = e & 15;
    if (j >= a.T) continue;
    const int row = (tile0 + t) * 16 + r;
    float v = row_value<T, NT>(part, t, j, r);
    if (EPI == EPI_STORE) {
      a.y[(size_t)j * N + row] = v;
    } else if (EPI == EPI_RESID) {
      if (gridDim.y == 1) a.y[(size_t)j * N + row] += v;
      else atomicAdd(a.y + (size_t)j * N + row, v);
    } else if (EPI == EPI_BIAS) {
      a.y[(size_t)j * N + row] = v + a.aux[row];
    } else if (EPI == EPI_QKV) {
      v += a.aux[row];
      const int nq = a.nh * HD, nk = a.nkv * HD;
      const int pos = a.pos[j];
      const int seq = j * a.seq_stride;
      if (row < nq + nk) {
        float v2 = row_value<T, NT>(part, t, j, r ^ 1) + a.aux[row ^ 1];
        const int e2 = row % HD, i = e2 >> 1, hi = e2 & 1;
        const float c = a.rope_cos[(size_t)pos * (HD / 2) + i], s = a.rope_sin[(size_t)pos * (HD / 2) + i];
        const float lo_v = hi ? v2 : v, hi_v = hi ? v : v2;
        const float out = hi ? (hi_v * c + lo_v * s) : (lo_v * c - hi_v * s);
        const int dim = i + (HD / 2) * hi;
        if (row < nq) {
          a.qout[(size_t)j * nq + (row / HD) * HD + dim] = __float2half_rn(out);
        } else {
          const int kvh = (row - nq) / HD;
          const int pg = a.block_table[(size_t)seq * a.bt_stride + pos / PAGE];
          a.kcache[(((size_t)pg * a.nkv + kvh) * PAGE + pos % PAGE) * HD + dim] = __float2half_rn(out);
        }
      } else {
        const int rv = row - nq - nk, kvh = rv / HD, dim = rv % HD;
        const int pg = a.block_table[(size_t)seq * a.bt_stride + pos / PAGE];
        a.vcache[(((size_t)pg * a.nkv + kvh) * PAGE + pos % PAGE) * HD + dim] = __float2half_rn(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// The GEMV. Template: T tokens (1..4), NT tiles per workgroup, prologue, epilogue.
template <int T, int NT, int PRO, int EPI>
__global__ void __launch_bounds__(256) k_gemv(const GemvArgs a) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red[8];
  __shared__ float part[4][NT][T][16];
  const int K = a.K, nb = K / 32;
  const XStage st = xstage_carve(lds, T, K);
  if (PRO == PRO_RMS) prologue_rms(st, a.h, a.nw, a.eps, T, K, red);
  else prologue_q8(st, a.xq, a.xds, T, K);
  __syncthreads();

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kl = wv * 4 + (lane >> 4);  // k-lane 0..15
  const int tile0 = blockIdx.x * NT;
  // k-split across grid.y (EPI_RESID only): block range [kb0, kb1)
  const int nks = gridDim.y;
  const int per = (nb + nks - 1) / nks;
  const int kb0 = blockIdx.y * per, kb1 = min(nb, kb0 + per);

  float acc[NT][T];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[t][j] = 0.f;

  const uint4* __restrict__ qs = (const uint4*)a.qs;
  const __half* __restrict__ dd = a.d;
#pragma unroll 2
  for (int b = kb0 + kl; b < kb1; b += 16) {
    uint4 w[NT];
    float dw[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      size_t idx = ((size_t)(tile0 + t) * nb + b) * 16 + r;
      w[t] = ld_stream16(qs + idx);
      dw[t] = __half2float(dd[idx]);
    }
#pragma unroll
    for (int j = 0; j < T; ++j) {
      const int4* xp = (const int4*)(st.q + (size_t)j * K + (size_t)b * 32);
      int4 xa = xp[0], xb = xp[1];
      int xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
      float dx = st.d[j * nb + b];
      int s8 = 8 * st.s[j * nb + b];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        int dot = q4_block_dot(w[t], xv);
        acc[t][j] = fmaf(dw[t] * dx, (float)(dot - s8), acc[t][j]);
      }
    }
  }
  // reduce the 4 slots of each row (lanes r, r+16, r+32, r+48), then the 4 waves in fixed order
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < T; ++j) {
      float v = acc[t][j];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (lane < 16) part[wv][t][j][r] = v;
    }
  __syncthreads();
  epilogue<T, NT, EPI>(a, part, tile0);
}

}  // namespace q355

namespace q355 {

// ---------------------------------------------------------------------------------------------
// Embedding: h[j] = dequant(E[tok[j]]) from the tiled Q4_0 planes (tied embedding/head).
__global__ void __launch_bounds__(64) k_embed_q4_0(const uint8_t* __restrict__ qs, const __half* __restrict__ d,
                                                   int V, int H, const int* __restrict__ tok, float* __restrict__ h) {
  const int j = blockIdx.x, nb = H / 32;
  const int t = tok[j];
  if (t < 0 || t >= V) return;
  const int tile = t >> 4, r = t & 15;
  for (int b = threadIdx.x; b < nb; b += blockDim.x) {
    const size_t idx = ((size_t)tile * nb + b) * 16 + r;
    const uint4 w = ((const uint4*)qs)[idx];
    const float dw = __half2float(d[idx]);
    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
    float* out = h + (size_t)j * H + b * 32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned byte = (ws[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      out[i] = dw * (float)((int)(byte & 15u) - 8);
      out[i + 16] = dw * (float)((int)(byte >> 4) - 8);
    }
  }
}

// Greedy finish: argmax over the head's per-workgroup partials (lowest index wins ties),
// tok[j] <- idx, pos[j] += 1. One workgroup per token.
__global__ void __launch_bounds__(256) k_finish(const float* __restrict__ pmax, const int* __restrict__ pidx,
                                                int nparts, int* __restrict__ tok, int* __restrict__ pos) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const int j = blockIdx.x;
  float v = -INFINITY;
  int idx = 0x7fffffff;
  for (int p = threadIdx.x; p < nparts; p += blockDim.x) {
    float x = pmax[(size_t)j * nparts + p];
    int i = pidx[(size_t)j * nparts + p];
    if (x > v || (x == v && i < idx)) { v = x; idx = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oi = __shfl_xor(idx, o, 64);
    if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
  }
  if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = v; bi[threadIdx.x >> 6] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = bv[0];
    idx = bi[0];
    for (int w = 1; w < 4; ++w)
      if (bv[w] > v || (bv[w] == v && bi[w] < idx)) { v = bv[w]; idx = bi[w]; }
    tok[j] = idx;
    pos[j] += 1;
  }
}

// Debug: every per-block int32 dot  out[j][n][b] = sum_i q_w(0..15) * q_x (bit-exactness checks).
__global__ void __launch_bounds__(256) k_blockdots(const uint8_t* __restrict__ qs, int N, int K,
                                                   const int8_t* __restrict__ xq, int T, int* __restrict__ out) {
  const int nb = K / 32;
  const long total = (long)T * N * nb;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (long)gridDim.x * blockDim.x) {
    const int b = e % nb, n = (e / nb) % N, j = e / ((long)nb * N);
    const uint4 w = ((const uint4*)qs)[((size_t)(n >> 4) * nb + b) * 16 + (n & 15)];
    const int* x = (const int*)(xq + (size_t)j * K + (size_t)b * 32);
    int xv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = x[i];
    out[e] = q4_block_dot(w, xv);
  }
}

}  // namespace q355
