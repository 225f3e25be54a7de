// Decode GQA attention over the paged fp16 KV cache, split-K over pages (flash-decoding), gfx950.
//
// k_attn_decode: workgroup (chunk c, KV head g, token j) = one wave per query head of the GQA group
// (G waves). It stages one 64-position K page (row-padded against LDS bank conflicts) and V page in
// LDS, lane p scores position p for its wave's head, the softmax numerator is a wave reduction, and
// lane l accumulates dims 2l, 2l+1 of P.V. Output: the unnormalised partial (o[128], m, l) per
// (token, query head, chunk). No atomics and no cross-workgroup waits.
// attn_merge_*: merges the partials of one token in fixed chunk order (o = sum_c e^(m_c - M) o_c / L)
// and quantizes the result to Q8_1 -- fused into the O-projection GEMV prologue, or standalone.
// Scores, softmax and P.V are computed in f64 (fp16 K/V and q widened exactly): the result feeds a Q8_1
// quantizer, so it must agree with the f64 oracle far below a quantization step.
// Semantics follow ATTN2 / ATTN4 (lab/qwen_kernels.py:358-442, 517-605).
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

constexpr int KROW = HD + 8;  // padded K row in LDS (halves)

template <int G>
__global__ void __launch_bounds__(G * 64) k_attn_decode(const AttnArgs a) {
  __shared__ __align__(16) __half ks[PAGE][KROW];
  __shared__ __align__(16) __half vs[PAGE][HD];
  __shared__ __align__(16) double qf[G][HD];
  __shared__ double E[G][PAGE];

  const int j = blockIdx.y;
  const int kvh = blockIdx.x / a.max_chunks, c = blockIdx.x % a.max_chunks;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int pos = a.pos[j];
  const int pg = a.block_table[(size_t)j * a.bt_stride + c];
  const int hq = kvh * G + wv;
  const half2 qv = ((const half2*)(a.q + ((size_t)j * a.nh + hq) * HD))[lane];
  if (c * PAGE > pos) return;                       // chunk beyond the context: nothing to do
  const int nvalid = min(PAGE, pos + 1 - c * PAGE);

  const uint4* kp = (const uint4*)(a.kcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  const uint4* vp = (const uint4*)(a.vcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  constexpr int NT = G * 64, PER = (PAGE * HD / 8 + NT - 1) / NT;
  uint4 kr[PER], vr[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = min(threadIdx.x + NT * i, PAGE * HD / 8 - 1);   // clamped: loads stay unconditional
    kr[i] = kp[e];
    vr[i] = vp[e];
  }
  const float2 qq = __half22float2(qv);
  qf[wv][2 * lane] = (double)qq.x;
  qf[wv][2 * lane + 1] = (double)qq.y;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = threadIdx.x + NT * i;
    if (e < PAGE * HD / 8) {
      *(uint4*)&ks[e >> 4][(e & 15) * 8] = kr[i];
      ((uint4*)vs)[e] = vr[i];
    }
  }
  __syncthreads();

  // scores: lane p, this wave's head (f64)
  double s = 0.0;
  {
    const double* qh = qf[wv];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) {
      const uint4 kk = *(const uint4*)&ks[lane][8 * i];
      const __half2* k2 = (const __half2*)&kk;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 kf = __half22float2(k2[u]);
        s = fma(qh[8 * i + 2 * u], (double)kf.x, s);
        s = fma(qh[8 * i + 2 * u + 1], (double)kf.y, s);
      }
    }
  }
  s = lane < nvalid ? s * a.scale : -INFINITY;
  const double m = wave_max_d(s);
  const double e = lane < nvalid ? exp(s - m) : 0.0;
  const double l = wave_sum_d(e);
  E[wv][lane] = e;
  __syncthreads();

  // P.V: lane owns dims 2*lane, 2*lane+1
  double o0 = 0.0, o1 = 0.0, o2 = 0.0, o3 = 0.0;
  int p = 0;
  for (; p + 1 < nvalid; p += 2) {
    const float2 v0 = __half22float2(((const __half2*)vs[p])[lane]);
    const float2 v1 = __half22float2(((const __half2*)vs[p + 1])[lane]);
    const double e0 = E[wv][p], e1 = E[wv][p + 1];
    o0 = fma(e0, (double)v0.x, o0);
    o1 = fma(e0, (double)v0.y, o1);
    o2 = fma(e1, (double)v1.x, o2);
    o3 = fma(e1, (double)v1.y, o3);
  }
  if (p < nvalid) {
    const float2 v0 = __half22float2(((const __half2*)vs[p])[lane]);
    o0 = fma(E[wv][p], (double)v0.x, o0);
    o1 = fma(E[wv][p], (double)v0.y, o1);
  }
  double* P = a.part + (((size_t)j * a.nh + hq) * a.max_chunks + c) * (HD + 2);
  ((double2*)P)[lane] = make_double2(o0 + o2, o1 + o3);
  if (lane == 0) { P[HD] = m; P[HD + 1] = l; }
}

// ---------------------------------------------------------------------------------------------
// Merge of one token's partials (nh query heads, nch chunks), f64. Called by every thread of a workgroup of
// NTH threads; `wgt` is LDS scratch of 2 * nh * max_chunks doubles; writes o[h * HD + d] to `out` (LDS).
template <int NTH>
__device__ __forceinline__ void attn_merge_token(const double* __restrict__ part, int nh, int max_chunks, int nch,
                                                 double* wgt, double* out) {
  // 1. per (h, c): raw m, l -> per-head M, L -> weights e^(m_c - M) / L
  for (int hc = threadIdx.x; hc < nh * nch; hc += NTH) {
    const int h = hc / nch, c = hc % nch;
    const double* P = part + ((size_t)h * max_chunks + c) * (HD + 2);
    wgt[h * max_chunks + c] = P[HD];
    wgt[nh * max_chunks + h * max_chunks + c] = P[HD + 1];
  }
  __syncthreads();
  if (threadIdx.x < nh) {
    const int h = threadIdx.x;
    double M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmax(M, wgt[h * max_chunks + c]);
    double L = 0.0;
    for (int c = 0; c < nch; ++c) L = fma(exp(wgt[h * max_chunks + c] - M), wgt[nh * max_chunks + h * max_chunks + c], L);
    for (int c = 0; c < nch; ++c) wgt[h * max_chunks + c] = exp(wgt[h * max_chunks + c] - M) / L;
  }
  __syncthreads();
  // 2. o[h][d] = sum_c w[h][c] o_c[d], chunks in fixed order, 4 loads in flight per thread
  for (int e = threadIdx.x; e < nh * HD; e += NTH) {
    const int h = e / HD, d = e % HD;
    const double* P = part + (size_t)h * max_chunks * (HD + 2) + d;
    const double* w = wgt + h * max_chunks;
    double o = 0.0;
    int c = 0;
    for (; c + 3 < nch; c += 4) {
      const double p0 = P[(size_t)c * (HD + 2)], p1 = P[(size_t)(c + 1) * (HD + 2)];
      const double p2 = P[(size_t)(c + 2) * (HD + 2)], p3 = P[(size_t)(c + 3) * (HD + 2)];
      o = fma(w[c], p0, o);
      o = fma(w[c + 1], p1, o);
      o = fma(w[c + 2], p2, o);
      o = fma(w[c + 3], p3, o);
    }
    for (; c < nch; ++c) o = fma(w[c], P[(size_t)c * (HD + 2)], o);
    out[e] = o;
  }
  __syncthreads();
}

// Standalone merge: one workgroup per token -> fp32 o32 (optional) and Q8_1 oq/ods.
__global__ void __launch_bounds__(256) k_attn_merge(const AttnArgs a) {
  extern __shared__ double sm[];
  const int j = blockIdx.x;
  const int nch = a.pos[j] / PAGE + 1;
  double* wgt = sm;                                  // 2 * nh * max_chunks
  double* o = sm + 2 * a.nh * a.max_chunks;          // nh * HD
  attn_merge_token<256>(a.part + (size_t)j * a.nh * a.max_chunks * (HD + 2), a.nh, a.max_chunks, nch, wgt, o);
  const int n = a.nh * HD;
  for (int e = threadIdx.x; e < n; e += 256) {      // n % 256 == 0 keeps 32-lane groups whole
    const float v = (float)o[e];
    if (a.o32) a.o32[(size_t)j * n + e] = v;
    const int q = q8_1_lane32(v, a.ods + ((size_t)j * n + e) / 32, (e & 31) == 0);
    a.oq[(size_t)j * n + e] = (int8_t)q;
  }
}

}  // namespace q355
