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
      // V rows past the context are zeroed: P.V below runs over the whole page with p = 0 there
      ((uint4*)vs)[e] = (e >> 4) < nvalid ? vr[i] : make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();

  // scores: lane p, this wave's head (f64, 4 independent partial sums)
  double s = 0.0;
  {
    const double* qh = qf[wv];
    double sp[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) {
      const uint4 kk = *(const uint4*)&ks[lane][8 * i];
      const __half2* k2 = (const __half2*)&kk;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 kf = __half22float2(k2[u]);
        sp[u] = fma(qh[8 * i + 2 * u], (double)kf.x, sp[u]);
        sp[u] = fma(qh[8 * i + 2 * u + 1], (double)kf.y, sp[u]);
      }
    }
    s = (sp[0] + sp[1]) + (sp[2] + sp[3]);
  }
  s = lane < nvalid ? s * a.scale : -INFINITY;
  const double m = wave_max_d(s);
  const double e = lane < nvalid ? exp(s - m) : 0.0;
  const double l = wave_sum_d(e);

  // P.V: lane owns dims 2*lane, 2*lane+1; p(position) is broadcast from lane p with readlane
  double o[4][2] = {{0.0, 0.0}, {0.0, 0.0}, {0.0, 0.0}, {0.0, 0.0}};
  const int2 ei = *reinterpret_cast<const int2*>(&e);
#pragma unroll
  for (int p = 0; p < PAGE; ++p) {
    int2 bi;
    bi.x = __builtin_amdgcn_readlane(ei.x, p);
    bi.y = __builtin_amdgcn_readlane(ei.y, p);
    const double ep = *reinterpret_cast<const double*>(&bi);
    const float2 v = __half22float2(((const __half2*)vs[p])[lane]);
    o[p & 3][0] = fma(ep, (double)v.x, o[p & 3][0]);
    o[p & 3][1] = fma(ep, (double)v.y, o[p & 3][1]);
  }
  const double o0 = (o[0][0] + o[1][0]) + (o[2][0] + o[3][0]);
  const double o1 = (o[0][1] + o[1][1]) + (o[2][1] + o[3][1]);
  double* P = a.part + (((size_t)j * a.nh + hq) * a.max_chunks + c) * (HD + 2);
  ((double2*)P)[lane] = make_double2(o0, o1);
  if (lane == 0) { P[HD] = m; P[HD + 1] = l; }
}

// ---------------------------------------------------------------------------------------------
// Merge of the chunk partials of one (token, query head), f64, by ONE wave: lane c reads chunk c's
// (m_c, l_c) and forms w_c = e^(m_c - M) (M = max_c m_c); lane l then sums dims 2l, 2l+1 of
// sum_c w_c o_c in fixed chunk order (w_c broadcast from lane c) and divides by L = sum_c w_c l_c.
// All loads of a group of 8 chunks are issued before their first use. nch <= 64.
__device__ __forceinline__ void attn_merge_head(const double* __restrict__ P, int nch, double* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const double* pc = P + (size_t)min(lane, nch - 1) * (HD + 2);
  const double mc = pc[HD], lc = pc[HD + 1];
  double2 v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = ((const double2*)(P + (size_t)min(u, nch - 1) * (HD + 2)))[lane];
  const double M = wave_max_d(lane < nch ? mc : -INFINITY);
  const double w = lane < nch ? exp(mc - M) : 0.0;
  const double L = wave_sum_d(w * (lane < nch ? lc : 0.0));
  const int2 wi = *reinterpret_cast<const int2*>(&w);
  double o0 = 0.0, o1 = 0.0;
  for (int c0 = 0; c0 < nch; c0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int2 bi;
      bi.x = __builtin_amdgcn_readlane(wi.x, c0 + u);   // 0 for chunks >= nch (w = 0 there)
      bi.y = __builtin_amdgcn_readlane(wi.y, c0 + u);
      const double wc = *reinterpret_cast<const double*>(&bi);
      o0 = fma(wc, v[u].x, o0);
      o1 = fma(wc, v[u].y, o1);
    }
    if (c0 + 8 < nch) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = ((const double2*)(P + (size_t)min(c0 + 8 + u, nch - 1) * (HD + 2)))[lane];
    }
  }
  ((double2*)out)[lane] = make_double2(o0 / L, o1 / L);
}

// Standalone merge: one workgroup (4 waves) per token -> fp32 o32 (optional) and Q8_1 oq/ods.
__global__ void __launch_bounds__(256) k_attn_merge(const AttnArgs a) {
  extern __shared__ double sm[];                     // nh * HD
  const int j = blockIdx.x;
  const int nch = a.pos[j] / PAGE + 1;
  for (int h = threadIdx.x >> 6; h < a.nh; h += 4)
    attn_merge_head(a.part + ((size_t)j * a.nh + h) * a.max_chunks * (HD + 2), nch, sm + h * HD);
  __syncthreads();
  const int n = a.nh * HD;
  for (int e = threadIdx.x; e < n; e += 256) {      // n % 256 == 0 keeps 32-lane groups whole
    const float v = (float)sm[e];
    if (a.o32) a.o32[(size_t)j * n + e] = v;
    const int q = q8_1_lane32(v, a.ods + ((size_t)j * n + e) / 32, (e & 31) == 0);
    a.oq[(size_t)j * n + e] = (int8_t)q;
  }
}

}  // namespace q355
