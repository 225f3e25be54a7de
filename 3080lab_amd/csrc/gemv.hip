// Q8_1 quantizers and the Q4_0 x Q8_1 GEMV (1..4 tokens) with fused prologues/epilogues, gfx950.
//
// GEMV work split: workgroup (x, y) owns NT 16-row tiles and the y-th of gridDim.y slices of the K
// blocks; its NW waves x 4 lane slots split the slice 4*NW ways (block b of the slice goes to k-lane
// b % (4*NW)). Lane (slot, row) streams 16 B of nibbles per block (1 KB contiguous per wave
// instruction) and dots it with the activation block held in LDS (v_dot4_i32_i8, exact int32).
// Partials reduce over slots (lane xor 16, 32) and over waves through LDS in a fixed order. K slices
// of the residual projections meet in the int64 fixed-point residual stream (integer atomics), so
// every output is bitwise reproducible run to run.
//
// Per-CU streaming bandwidth on MI355X is ~20-28 GB/s (HBM needs all 256 CUs busy), so every launch
// is cut into >= ~300 workgroups: N = 1536 projections use K slices, gate_up uses one tile each.
#include "common.h"
#include "q355_kernels.h"
#include "attn.hip"

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
// GEMV building blocks. Latency plan of every GEMV launch:
//   1. issue the activation loads (residual + norm weight, fp32 input, or xq + xds),
//   2. issue every weight load of this lane (NT tiles x KPL blocks of 16 B, all in flight at once),
//   3. build the Q8_1 activation operand in LDS while the weights are in flight,
//   4. int8 dots from registers, fixed-order reductions, fused epilogue.
// LDS activation operand (indexed by absolute K block): xq bytes [T][K], dx float [T][nb], sq int [T][nb].
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

// Store one lane's 8 quantized values (and, from the first lane of the 4-lane block, d and sum q).
__device__ __forceinline__ void stage_x8(const XStage& st, int K, int j, int g, const float (&x)[8]) {
  float df;
  int sq;
  const uint2 pk = q8_1_x8(x, df, sq);
  *(uint2*)(st.q + (size_t)j * K + 8 * g) = pk;
  if ((g & 3) == 0) {
    st.d[j * (K / 32) + (g >> 2)] = df;
    st.s[j * (K / 32) + (g >> 2)] = sq;
  }
}

// K-block slice of this workgroup.
struct KSlice {
  int b0, b1;
  __device__ __forceinline__ KSlice(int nb) {
    const int per = (nb + gridDim.y - 1) / gridDim.y;
    b0 = min(nb, (int)blockIdx.y * per);
    b1 = min(nb, b0 + per);
  }
};

// Activation operand, stage 1 (loads into registers) and stage 2 (quantize / copy into LDS).
// RMS / F32 / ATTN: a task is 8 consecutive values of one token (4 lanes = one Q8_1 block).
template <int T, int NW, int PRO, int KPL>
struct XLoad {
  static constexpr int NTH = NW * 64;
  static constexpr bool R = PRO == PRO_RMS || PRO == PRO_EMB, F = PRO == PRO_F32, Q = PRO == PRO_Q8;
  static constexpr int P8 = (T * 1536 / 8 + NTH - 1) / NTH;   // RMS: 8-value tasks per thread (K <= 1536)
  static constexpr int PF = (T * 16 * NW * KPL + NTH - 1) / NTH;   // F32: tasks per thread (slice <= 4 NW KPL blocks)
  static constexpr int PT = (T * 288 + NTH - 1) / NTH;        // Q8: 32-blocks per thread (K <= 9216)
  static constexpr int NX = R ? P8 : (F ? PF : 1);
  long long hl[R ? P8 : 1][8];
  float4 xa[NX], xb[NX];                                       // F32 input, or RMS norm weights
  int4 qa[Q ? PT : 1], qb[Q ? PT : 1];
  float dx[Q ? PT : 1];

  __device__ __forceinline__ void load(const GemvArgs& a, const KSlice& ks) {
    const int K = a.K;
    // tasks past the end re-load the last valid task (clamped): unconditional, straight-line loads
    if (R) {
      const int ng = K / 8, ntask = a.T * ng;
#pragma unroll
      for (int p = 0; p < P8; ++p) {
        const int task = min(threadIdx.x + NTH * p, ntask - 1);
        const int j = task / ng, g = task % ng;
        if (PRO == PRO_EMB) {
          // values 8 g .. 8 g + 7 of the embedding row: block g / 4, bytes 8 (g & 1) .. + 7, low nibbles
          // for the block's first 16 values, high for the rest (k_embed_q4_0's arithmetic)
          const int t = min(max(a.tok[j], 0), a.emb_v - 1), b = g >> 2;
          const size_t idx = ((size_t)(t >> 4) * (K / 32) + b) * 16 + (t & 15);
          const uint2 w = ((const uint2*)a.emb_qs)[idx * 2 + (g & 1)];
          const double dw = (double)__half2float(a.emb_d[idx]);
          const int sh = (g & 2) ? 4 : 0;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const unsigned byte = ((u < 4 ? w.x : w.y) >> (8 * (u & 3))) & 0xFFu;
            hl[p][u] = to_fix(dw * (double)((int)((byte >> sh) & 15u) - 8));
          }
        } else {
          const longlong2* hp = (const longlong2*)(a.hfix + (size_t)j * K + 8 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) { const longlong2 v = hp[u]; hl[p][2 * u] = v.x; hl[p][2 * u + 1] = v.y; }
        }
        const float4* wp = (const float4*)(a.nw + 8 * g);
        xa[p] = wp[0];
        xb[p] = wp[1];
      }
    } else if (F) {
      const int g0 = ks.b0 * 4, ng = (ks.b1 - ks.b0) * 4, ntask = a.T * ng;
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int task = min(threadIdx.x + NTH * p, ntask - 1);
        const int j = task / ng, g = g0 + task % ng;
        const float4* xp = (const float4*)(a.xf + (size_t)j * K + 8 * g);
        xa[p] = xp[0];
        xb[p] = xp[1];
      }
    } else if (Q) {
      const int nbs = ks.b1 - ks.b0, ntask = a.T * nbs;
#pragma unroll
      for (int p = 0; p < PT; ++p) {
        const int task = min(threadIdx.x + NTH * p, ntask - 1);
        const int j = task / nbs, b = ks.b0 + task % nbs;
        const int4* src = (const int4*)(a.xq + (size_t)j * K + (size_t)b * 32);
        qa[p] = src[0];
        qb[p] = src[1];
        dx[p] = __low2float(a.xds[(size_t)j * (K / 32) + b]);
      }
    }
  }

  __device__ __forceinline__ void stage(const GemvArgs& a, const KSlice& ks, const XStage& st, float* red,
                                        char* extra) {
    const int K = a.K, nb = K / 32;
    if (PRO == PRO_ATTN) {
      // merge the split-K attention partials of the heads in this K slice (f64, one wave per head), then Q8_1
      double* ob = (double*)extra;                   // nhs * HD merged outputs of one token
      const int h0 = ks.b0 * 32 / HD, nhs = (ks.b1 - ks.b0) * 32 / HD;
      for (int j = 0; j < a.T; ++j) {
        const int nch = a.pos[j] / PAGE + 1;
        for (int h = threadIdx.x >> 6; h < nhs; h += NTH / 64)
          attn_merge_head(a.attn_part + ((size_t)j * a.nh + h0 + h) * a.attn_max_chunks * (HD + 2), a.attn_max_chunks, nch,
                          ob + h * HD);
        __syncthreads();
        for (int g = threadIdx.x; g < nhs * HD / 8; g += NTH) {   // quads stay whole (HD / 8 % 4 == 0)
          float x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) x[u] = (float)ob[8 * g + u];
          stage_x8(st, K, j, h0 * HD / 8 + g, x);
        }
        __syncthreads();
      }
    } else if (R) {
      // RMSNorm in f64: the quantizer input x = h * rsqrt(mean(h^2) + eps) * w matches the f64 oracle
      const int ng = K / 8, ntask = a.T * ng;
      if (PRO == PRO_EMB && blockIdx.x == 0 && blockIdx.y == 0) {   // the residual stream starts here
#pragma unroll
        for (int p = 0; p < P8; ++p) {
          const int task = threadIdx.x + NTH * p;
          if (task < ntask) {
            longlong2* dst = (longlong2*)(a.hout + (size_t)(task / ng) * K + 8 * (task % ng));
#pragma unroll
            for (int u = 0; u < 4; ++u) dst[u] = make_longlong2(hl[p][2 * u], hl[p][2 * u + 1]);
          }
        }
      }
      double ss[T];
#pragma unroll
      for (int j = 0; j < T; ++j) ss[j] = 0.0;
#pragma unroll
      for (int p = 0; p < P8; ++p) {
        const int task = threadIdx.x + NTH * p;
        double v = 0.0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const double hv = from_fix(hl[p][u]);
          v = fma(hv, hv, v);
        }
#pragma unroll
        for (int j = 0; j < T; ++j) ss[j] += (task < ntask && task / ng == j) ? v : 0.0;
      }
      double* redd = (double*)red;
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const double w = wave_sum_d(ss[j]);
        if ((threadIdx.x & 63) == 0) redd[(threadIdx.x >> 6) * T + j] = w;
      }
      __syncthreads();
      double rs[T];
#pragma unroll
      for (int j = 0; j < T; ++j) {
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += redd[w * T + j];
        rs[j] = 1.0 / sqrt(t / (double)K + a.eps);
      }
#pragma unroll
      for (int p = 0; p < P8; ++p) {
        const int task = threadIdx.x + NTH * p;
        if (task < ntask) {
          const int j = task / ng, g = task % ng;
          double r = rs[0];
#pragma unroll
          for (int jj = 1; jj < T; ++jj) r = (j == jj) ? rs[jj] : r;
          const float wv[8] = {xa[p].x, xa[p].y, xa[p].z, xa[p].w, xb[p].x, xb[p].y, xb[p].z, xb[p].w};
          float x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) x[u] = (float)(from_fix(hl[p][u]) * r * (double)wv[u]);
          stage_x8(st, K, j, g, x);
        }
      }
    } else if (F) {
      const int g0 = ks.b0 * 4, ng = (ks.b1 - ks.b0) * 4, ntask = a.T * ng;
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int task = threadIdx.x + NTH * p;
        if (task < ntask) {
          const int j = task / ng, g = g0 + task % ng;
          const float x[8] = {xa[p].x, xa[p].y, xa[p].z, xa[p].w, xb[p].x, xb[p].y, xb[p].z, xb[p].w};
          stage_x8(st, K, j, g, x);
        }
      }
    } else {
      const int nbs = ks.b1 - ks.b0, ntask = a.T * nbs;
#pragma unroll
      for (int p = 0; p < PT; ++p) {
        const int task = threadIdx.x + NTH * p;
        if (task < ntask) {
          const int j = task / nbs, b = ks.b0 + task % nbs;
          int4* dst = (int4*)(st.q + (size_t)j * K + (size_t)b * 32);
          dst[0] = qa[p];
          dst[1] = qb[p];
          const int xv[8] = {qa[p].x, qa[p].y, qa[p].z, qa[p].w, qb[p].x, qb[p].y, qb[p].z, qb[p].w};
          st.s[j * nb + b] = sum_i8x32(xv);
          st.d[j * nb + b] = dx[p];
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Epilogues. part[w][t][j][r] holds wave w's partial of row (tile0 + t) * 16 + r for token j (f64 on the
// batch-1 path, fp32 on the MFMA path); everything after the reduction is computed in f64.
template <int NW, int T, int NT, typename A>
__device__ __forceinline__ double row_value(A (&part)[NW][NT][T][16], int t, int j, int r) {
  double v = part[0][t][j][r];
#pragma unroll
  for (int w = 1; w < NW; ++w) v += part[w][t][j][r];
  return v;
}

__device__ __forceinline__ double silu_mul(double g, double u) { return g / (1.0 + exp(-g)) * u; }

// fp32 form for fp32 partials (the MFMA paths, whose block sums are already fp32): partial sum over
// waves in wave order, SiLU with the hardware exp2 and reciprocal
template <int NW, int T, int NT>
__device__ __forceinline__ float row_value_f(float (&part)[NW][NT][T][16], int t, int j, int r) {
  float v = part[0][t][j][r];
#pragma unroll
  for (int w = 1; w < NW; ++w) v += part[w][t][j][r];
  return v;
}
__device__ __forceinline__ float silu_mul_f(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)) * u;   // v_rcp_f32: 1 ulp
}

template <int NW, int T, int NT, int EPI, typename A>
__device__ __forceinline__ void epilogue(const GemvArgs& a, A (&part)[NW][NT][T][16], int tile0) {
  const int N = a.N;
  if (EPI == EPI_LOGITS) {
    // one wave computes the (value, row) argmax of the NT * 16 rows, lowest row on ties (fp32 logits)
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      for (int j = 0; j < T && j < a.T; ++j) {
        float v = -INFINITY;
        int idx = 0x7fffffff;
        for (int rr = l; rr < NT * 16; rr += 64) {   // rows in increasing order: strict '>' keeps the lowest
          const float x = (float)row_value<NW, T, NT>(part, rr >> 4, j, rr & 15);
          if (a.y) a.y[(size_t)j * N + tile0 * 16 + rr] = x;   // optional fp32 logits
          if (x > v) { v = x; idx = tile0 * 16 + rr; }
        }
        wave_argmax(v, idx);
        if (l == 0) {
          a.pmax[(size_t)j * gridDim.x + blockIdx.x] = v;
          a.pidx[(size_t)j * gridDim.x + blockIdx.x] = idx;
        }
      }
    }
    return;
  }
  if (EPI == EPI_SWIGLU_Q8) {
    // NT == 4: 64 interleaved rows (g0, u0, g1, u1, ...) -> 32 outputs = one Q8_1 block per token
    for (int e = threadIdx.x; e < 32 * T; e += blockDim.x) {   // 32-lane groups: one token each
      const int j = e >> 5, k = e & 31;
      if (j >= a.T) break;                                      // uniform per 32-lane group
      const int rg = 2 * k, ru = 2 * k + 1;
      float o;
      if constexpr (std::is_same<A, float>::value) {
        o = silu_mul_f(row_value_f<NW, T, NT>(part, rg >> 4, j, rg & 15),
                       row_value_f<NW, T, NT>(part, ru >> 4, j, ru & 15));
      } else {
        o = (float)silu_mul(row_value<NW, T, NT>(part, rg >> 4, j, rg & 15),
                            row_value<NW, T, NT>(part, ru >> 4, j, ru & 15));
      }
      const int Nout = N / 2;
      const int q = q8_1_lane32(o, a.ods + (size_t)j * (Nout / 32) + blockIdx.x, k == 0);
      a.oq[(size_t)j * Nout + blockIdx.x * 32 + k] = (int8_t)q;
    }
    return;
  }
  if (EPI == EPI_SWIGLU_F16) {
    // rows interleaved (g0, u0, g1, u1, ...): one thread per output pair, fp32 SiLU, fp16 out
    for (int e = threadIdx.x; e < NT * T * 8; e += blockDim.x) {
      const int t = e / (T * 8), j = (e >> 3) % T, k = e & 7;
      if (j >= a.T) continue;
      float g, u;
      if constexpr (std::is_same<A, float>::value) {
        g = row_value_f<NW, T, NT>(part, t, j, 2 * k);
        u = row_value_f<NW, T, NT>(part, t, j, 2 * k + 1);
      } else {
        g = (float)row_value<NW, T, NT>(part, t, j, 2 * k);
        u = (float)row_value<NW, T, NT>(part, t, j, 2 * k + 1);
      }
      a.yh[(size_t)j * (N / 2) + (tile0 + t) * 8 + k] = __float2half_rn(silu_mul_f(g, u));
    }
    return;
  }
  if (EPI == EPI_SWIGLU) {
    // rows interleaved (g0, u0, g1, u1, ...): one thread per output pair
    for (int e = threadIdx.x; e < NT * T * 8; e += blockDim.x) {
      const int t = e / (T * 8), j = (e >> 3) % T, k = e & 7;
      if (j >= a.T) continue;
      if constexpr (std::is_same<A, float>::value) {
        a.y[(size_t)j * (N / 2) + (tile0 + t) * 8 + k] =
            silu_mul_f(row_value_f<NW, T, NT>(part, t, j, 2 * k), row_value_f<NW, T, NT>(part, t, j, 2 * k + 1));
      } else {
        const double g = row_value<NW, T, NT>(part, t, j, 2 * k), u = row_value<NW, T, NT>(part, t, j, 2 * k + 1);
        a.y[(size_t)j * (N / 2) + (tile0 + t) * 8 + k] = (float)silu_mul(g, u);
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < NT * T * 16; e += blockDim.x) {
    const int t = e / (T * 16), j = (e >> 4) % T, r = e & 15;
    if (j >= a.T) continue;
    const int row = (tile0 + t) * 16 + r;
    double v = row_value<NW, T, NT>(part, t, j, r);
    if (EPI == EPI_STORE) {
      a.y[(size_t)j * N + row] = (float)v;
    } else if (EPI == EPI_RESID) {
      a.y[(size_t)j * N + row] += (float)v;
    } else if (EPI == EPI_RESID_FIX) {
      atomicAdd((unsigned long long*)(a.yfix + (size_t)j * N + row), (unsigned long long)to_fix(v));
    } else if (EPI == EPI_BIAS) {
      a.y[(size_t)j * N + row] = (float)(v + (double)a.aux[row]);
    } else if (EPI == EPI_QKV) {
      // f64: bias, RoPE; q, k and v rounded f64 -> fp16 once
      v += (double)a.aux[row];
      const int nq = a.nh * HD, nk = a.nkv * HD;
      const int pos = a.pos[j];
      const int seq = (a.tok_base + j) * a.seq_stride;
      const int pg = a.block_table[(size_t)seq * a.bt_stride + pos / PAGE];
      if (row < nq + nk) {
        const double v2 = row_value<NW, T, NT>(part, t, j, r ^ 1) + (double)a.aux[row ^ 1];
        const int e2 = row % HD, i = e2 >> 1, hi = e2 & 1;
        const double c = a.rope_cos[(size_t)pos * (HD / 2) + i], s = a.rope_sin[(size_t)pos * (HD / 2) + i];
        const double lo_v = hi ? v2 : v, hi_v = hi ? v : v2;
        const double out = hi ? (hi_v * c + lo_v * s) : (lo_v * c - hi_v * s);
        const int dim = i + (HD / 2) * hi;
        if (row < nq) {
          const __half hq = half_rn(out);
          a.qout[(size_t)j * nq + (row / HD) * HD + dim] = hq;
          if (a.qout64) a.qout64[(size_t)j * nq + (row / HD) * HD + dim] = (double)__half2float(hq);
        } else {
          const int kvh = (row - nq) / HD;
          a.kcache[(((size_t)pg * a.nkv + kvh) * PAGE + pos % PAGE) * HD + dim] = half_rn(out);
        }
      } else {
        const int rv = row - nq - nk, kvh = rv / HD, dim = rv % HD;
        a.vcache[(((size_t)pg * a.nkv + kvh) * PAGE + pos % PAGE) * HD + dim] = half_rn(v);
      }
    }
  }
}

// QKV epilogue whose per-element inputs (position, page id, RoPE cos/sin, the two biases) are loaded at kernel
// start: their dependent loads (position -> page and table rows) overlap the products instead of following
// the reduction. One output element per thread (NT * T * 16 <= blockDim.x); same f64 arithmetic as the
// EPI_QKV branch of epilogue().
struct QkvPre {
  int t, j, r, pos, pg;
  float c, s, b0, b1;
  bool live;
};

template <int T, int NT>
__device__ __forceinline__ QkvPre qkv_prefetch(const GemvArgs& a, int tile0) {
  QkvPre q = {};
  const int e = threadIdx.x;
  q.t = e / (T * 16);
  q.j = (e >> 4) % T;
  q.r = e & 15;
  q.live = e < NT * T * 16 && q.j < a.T;
  if (!q.live) return q;
  const int row = (tile0 + q.t) * 16 + q.r;
  q.pos = a.pos[q.j];
  q.pg = a.block_table[(size_t)((a.tok_base + q.j) * a.seq_stride) * a.bt_stride + q.pos / PAGE];
  const int i = (row % HD) >> 1;
  q.c = a.rope_cos[(size_t)q.pos * (HD / 2) + i];
  q.s = a.rope_sin[(size_t)q.pos * (HD / 2) + i];
  q.b0 = a.aux[row];
  q.b1 = a.aux[row ^ 1];
  return q;
}

template <int NW, int T, int NT, typename A>
__device__ __forceinline__ void qkv_store(const GemvArgs& a, A (&part)[NW][NT][T][16], int tile0, const QkvPre& q) {
  if (!q.live) return;
  const int row = (tile0 + q.t) * 16 + q.r;
  const int nq = a.nh * HD, nk = a.nkv * HD;
  const double v = row_value<NW, T, NT>(part, q.t, q.j, q.r) + (double)q.b0;
  if (row < nq + nk) {
    const double v2 = row_value<NW, T, NT>(part, q.t, q.j, q.r ^ 1) + (double)q.b1;
    const int e2 = row % HD, i = e2 >> 1, hi = e2 & 1;
    const double c = q.c, s = q.s;
    const double lo_v = hi ? v2 : v, hi_v = hi ? v : v2;
    const double out = hi ? (hi_v * c + lo_v * s) : (lo_v * c - hi_v * s);
    const int dim = i + (HD / 2) * hi;
    if (row < nq) {
      const __half hq = half_rn(out);
      a.qout[(size_t)q.j * nq + (row / HD) * HD + dim] = hq;
      if (a.qout64) a.qout64[(size_t)q.j * nq + (row / HD) * HD + dim] = (double)__half2float(hq);
    } else {
      a.kcache[(((size_t)q.pg * a.nkv + (row - nq) / HD) * PAGE + q.pos % PAGE) * HD + dim] = half_rn(out);
    }
  } else {
    const int rv = row - nq - nk;
    a.vcache[(((size_t)q.pg * a.nkv + rv / HD) * PAGE + q.pos % PAGE) * HD + rv % HD] = half_rn(v);
  }
}

// ---------------------------------------------------------------------------------------------
// The GEMV: T tokens (1..4), NT 16-row tiles per workgroup, NW waves splitting the K slice 4*NW ways,
// KPL K-blocks per lane (compile time, so all weight loads are issued before the first use).
// Optional timing hooks (defined by instrumented builds only; empty in the library).
#ifndef Q355_TRACE_POINT
#define Q355_TRACE_POINT(k)
#endif

template <int T, int NT, int NW, int KPL, int PRO, int EPI, int WF>
__global__ void __launch_bounds__(NW * 64) k_gemv(const GemvArgs a) {
  Q355_TRACE_POINT(0);
  extern __shared__ __align__(16) char lds[];
  __shared__ double red[NW * T];
  __shared__ double part[NW][NT][T][16];
  constexpr int NKL = 4 * NW;  // k-lanes
  const int K = a.K, nb = K / 32;
  const KSlice ks(nb);
  const XStage st = xstage_carve(lds, T, K);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kl = wv * 4 + (lane >> 4);
  const int tile0 = blockIdx.x * NT;

  XLoad<T, NW, PRO, KPL> xl;
  xl.load(a, ks);

  const uint4* __restrict__ qs = (const uint4*)a.qs;
  const unsigned short* __restrict__ dd = (const unsigned short*)a.d;
  constexpr bool Q6 = WF == WF_Q6_K;
  uint4 w[NT][KPL];
  unsigned dh[NT][KPL];   // fp16 scale bits, zero-extended: 16-bit register halves would serialise the loads
  uint2 hq[NT][Q6 ? KPL : 1];
  unsigned sc6[NT][Q6 ? KPL : 1];
  // Unconditional loads (clamped block index, scale zeroed past the slice): straight-line code lets
  // the compiler wait for exactly the loads each use needs instead of draining all of them.
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int b = ks.b0 + kl + NKL * i;
    const int bc = min(b, ks.b1 - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t idx = ((size_t)(tile0 + t) * nb + bc) * 16 + r;
      w[t][i] = ld_stream16(qs + idx);
      if constexpr (Q6) {
        hq[t][i] = ld_stream8((const uint2*)a.qhi + idx);
        sc6[t][i] = ld_stream2((const unsigned short*)a.qsc + idx);
        dh[t][i] = dd[((size_t)(tile0 + t) * (nb / 8) + bc / 8) * 16 + r];
      } else {
        dh[t][i] = ld_stream2(dd + idx);
      }
    }
  }
  // compiler barrier: keep every load above issued here (no sinking into the conditional code below)
  __asm__ __volatile__("" ::: "memory");
  Q355_TRACE_POINT(1);
#pragma unroll
  for (int i = 0; i < KPL; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) dh[t][i] = (ks.b0 + kl + NKL * i < ks.b1) ? dh[t][i] : 0u;

  xl.stage(a, ks, st, (float*)red, lds + (size_t)T * K + (size_t)T * nb * 8);
  __syncthreads();
  Q355_TRACE_POINT(2);

  // f64 accumulation: each block term d_w * d_x * (dot - 8 sum q) is exact in f64 (22 + 21 bits)
  double acc[NT][T];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[t][j] = 0.0;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int b = min(ks.b0 + kl + NKL * i, ks.b1 - 1);   // lanes past the slice re-read a valid block, scale 0
    {
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const int4* xp = (const int4*)(st.q + (size_t)j * K + (size_t)b * 32);
        const int4 xa = xp[0], xb = xp[1];
        const int xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const float dx = st.d[j * nb + b];
        const int s8 = 8 * st.s[j * nb + b];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const double sc = (double)__half2float(__ushort_as_half((unsigned short)dh[t][i])) * (double)dx;
          if constexpr (Q6) {
            acc[t][j] = fma(sc, (double)q6k_block_isum(w[t][i], hq[t][i], sc6[t][i], xv), acc[t][j]);
          } else {
            const int dot = q4_block_dot(w[t][i], xv);
            acc[t][j] = fma(sc, (double)(dot - s8), acc[t][j]);
          }
        }
      }
    }
  }
  Q355_TRACE_POINT(3);
  // reduce the 4 slots of each row (lanes r, r+16, r+32, r+48), then the NW waves in fixed order
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < T; ++j) {
      double v = acc[t][j];
      v = xsum32_d(xsum16_d(v));
      if (lane < 16) part[wv][t][j][r] = v;
    }
  __syncthreads();
  Q355_TRACE_POINT(4);
  epilogue<NW, T, NT, EPI>(a, part, tile0);
  Q355_TRACE_POINT(5);
}

}  // namespace q355

namespace q355 {

// ---------------------------------------------------------------------------------------------
// Embedding: h[j] = dequant(E[tok[j]]) from the tiled Q4_0 planes (tied embedding/head), written as
// the fixed-point residual stream (exact: d * (q - 8) has at most 15 significant bits).
__global__ void __launch_bounds__(64) k_embed_q4_0(const uint8_t* __restrict__ qs, const __half* __restrict__ d,
                                                   int V, int H, const int* __restrict__ tok,
                                                   long long* __restrict__ h) {
  const int j = blockIdx.x, nb = H / 32;
  const int t = tok[j];
  if (t < 0 || t >= V) return;
  const int tile = t >> 4, r = t & 15;
  for (int b = threadIdx.x; b < nb; b += blockDim.x) {
    const size_t idx = ((size_t)tile * nb + b) * 16 + r;
    const uint4 w = ((const uint4*)qs)[idx];
    const float dw = __half2float(d[idx]);
    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
    long long* out = h + (size_t)j * H + b * 32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned byte = (ws[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      out[i] = to_fix((double)dw * (double)((int)(byte & 15u) - 8));
      out[i + 16] = to_fix((double)dw * (double)((int)(byte >> 4) - 8));
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
  // 8 partials per thread per round, all loaded before the first comparison (one memory latency per round)
  for (int p0 = 0; p0 < nparts; p0 += 8 * blockDim.x) {
    float x[8];
    int ix[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = p0 + threadIdx.x + u * blockDim.x;
      x[u] = p < nparts ? pmax[(size_t)j * nparts + p] : -INFINITY;
      ix[u] = p < nparts ? pidx[(size_t)j * nparts + p] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (x[u] > v || (x[u] == v && ix[u] < idx)) { v = x[u]; idx = ix[u]; }
  }
  wave_argmax(v, idx);
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

// RMSNorm of the fixed-point residual stream -> Q8_1, one token per workgroup (batched / prefill path).
__global__ void __launch_bounds__(256) k_rmsnorm_fix_q8_1(const long long* __restrict__ h, const float* __restrict__ w,
                                                          int8_t* __restrict__ xq, half2* __restrict__ xds, int H,
                                                          double eps) {
  __shared__ double red[4];
  const int tok = blockIdx.x;
  const int g = threadIdx.x;                       // 8 consecutive values per thread, H / 8 <= 256
  const bool act = g < H / 8;
  // every load first (h as four 16-byte pieces, the norm weights beside them): one memory latency
  longlong2 hr[4] = {};
  float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
  if (act) {
    const longlong2* hp = (const longlong2*)(h + (size_t)tok * H + 8 * g);
#pragma unroll
    for (int u = 0; u < 4; ++u) hr[u] = hp[u];
    w0 = ((const float4*)w)[2 * g];
    w1 = ((const float4*)w)[2 * g + 1];
  }
  double hv[8];
  double ss = 0.0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    hv[2 * u] = from_fix(hr[u].x);
    hv[2 * u + 1] = from_fix(hr[u].y);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) ss = fma(hv[u], hv[u], ss);
  ss = wave_sum_d(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const double r = 1.0 / sqrt((red[0] + red[1] + red[2] + red[3]) / (double)H + eps);
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (act) {
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = (float)(hv[u] * r * (double)wv[u]);
  }
  float df, d32;
  int sq;
  const uint2 pk = q8_1_x8(x, df, sq, d32);         // H / 8 % 4 == 0: quads stay whole
  if (act) {
    *(uint2*)(xq + (size_t)tok * H + 8 * g) = pk;
    if ((g & 3) == 0) xds[(size_t)tok * (H / 32) + (g >> 2)] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
  }
}

// RMSNorm of the fixed-point residual stream -> fp16 (the fp16 batched path), one token per workgroup.
__global__ void __launch_bounds__(256) k_rmsnorm_fix_f16(const long long* __restrict__ h, const float* __restrict__ w,
                                                         __half* __restrict__ xh, int H, double eps) {
  __shared__ double red[4];
  const int tok = blockIdx.x;
  const int g = threadIdx.x;                       // 8 consecutive values per thread, H / 8 <= 256
  const bool act = g < H / 8;
  // every load first (h as four 16-byte pieces, the norm weights beside them): one memory latency
  longlong2 hr[4] = {};
  float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
  if (act) {
    const longlong2* hp = (const longlong2*)(h + (size_t)tok * H + 8 * g);
#pragma unroll
    for (int u = 0; u < 4; ++u) hr[u] = hp[u];
    w0 = ((const float4*)w)[2 * g];
    w1 = ((const float4*)w)[2 * g + 1];
  }
  double hv[8];
  double ss = 0.0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    hv[2 * u] = from_fix(hr[u].x);
    hv[2 * u + 1] = from_fix(hr[u].y);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) ss = fma(hv[u], hv[u], ss);
  ss = wave_sum_d(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const double r = 1.0 / sqrt((red[0] + red[1] + red[2] + red[3]) / (double)H + eps);
  if (act) {
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    __half o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = half_rn(hv[u] * r * (double)wv[u]);
    *(uint4*)(xh + (size_t)tok * H + 8 * g) = *(const uint4*)o;
  }
}

// QKV finish for the MFMA path: the K-sliced QKV product accumulated in int64 fixed point [T][nqkv]
// (device row order: q/k heads pair-interleaved) -> + bias, RoPE, fp16 q out, fp16 K/V cache write;
// the accumulator is cleared for the next use. One workgroup per token, one thread per row pair.
__global__ void __launch_bounds__(256) k_qkv_finish(GemvArgs a, long long* __restrict__ acc) {
  const int j = blockIdx.x;
  const int nq = a.nh * HD, nk = a.nkv * HD, N = nq + nk + nk;
  const int pos = a.pos[j];
  const int seq = j * a.seq_stride;
  const int pg = a.block_table[(size_t)seq * a.bt_stride + pos / PAGE];
  for (int p = threadIdx.x; p < N / 2; p += blockDim.x) {
    const int row = 2 * p;
    long long* ap = acc + (size_t)j * N + row;
    const double v0 = from_fix(ap[0]) + (double)a.aux[row], v1 = from_fix(ap[1]) + (double)a.aux[row + 1];
    ap[0] = 0;
    ap[1] = 0;
    if (row < nq + nk) {
      const int i = (row % HD) >> 1;               // pair (dim i, dim i + 64)
      const double c = a.rope_cos[(size_t)pos * (HD / 2) + i], s = a.rope_sin[(size_t)pos * (HD / 2) + i];
      const __half lo = half_rn(v0 * c - v1 * s), hi = half_rn(v1 * c + v0 * s);
      if (row < nq) {
        __half* q = a.qout + (size_t)j * nq + (row / HD) * HD;
        q[i] = lo;
        q[i + HD / 2] = hi;
      } else {
        __half* k = a.kcache + (((size_t)pg * a.nkv + (row - nq) / HD) * PAGE + pos % PAGE) * HD;
        k[i] = lo;
        k[i + HD / 2] = hi;
      }
    } else {
      const int rv = row - nq - nk;
      __half* v = a.vcache + (((size_t)pg * a.nkv + rv / HD) * PAGE + pos % PAGE) * HD + rv % HD;
      v[0] = half_rn(v0);
      v[1] = half_rn(v1);
    }
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

// ---------------------------------------------------------------------------------------------
// Measurement: a pure streaming read (16-byte non-temporal loads, 16 per lane, all in flight), the ceiling a
// weight stream of the same size reaches when launched the way the decode step launches its GEMVs.
__global__ void __launch_bounds__(256) k_stream_read(const uint4* __restrict__ p, long n16, unsigned* __restrict__ out) {
  constexpr int PER = 16;
  const long base = (long)blockIdx.x * 256 * PER + threadIdx.x;
  uint4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const long e = base + (long)i * 256;
    v[i] = e < n16 ? ld_stream16(p + e) : make_uint4(0, 0, 0, 0);
  }
  unsigned acc = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) acc ^= v[i].x ^ v[i].w;
  if (acc == 0x9e3779b9u && n16 < 0) out[blockIdx.x] = acc;   // never: keeps the loads
}

}  // namespace q355
