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

// accumulation-type overloads (f64: the batch-1 path; fp32: the batched path)
__device__ __forceinline__ double rd_lane(double v, int l) { return readlane_d(v, l); }
__device__ __forceinline__ float rd_lane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double wmax(double v) { return wave_max_d(v); }
__device__ __forceinline__ double wsum(double v) { return wave_sum_d(v); }
__device__ __forceinline__ float wmax(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp<DPP_MIRROR>(v));
  return fmaxf(fmaxf(rd_lane(v, 0), rd_lane(v, 16)), fmaxf(rd_lane(v, 32), rd_lane(v, 48)));
}
__device__ __forceinline__ float wsum(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_MIRROR>(v);
  return (rd_lane(v, 0) + rd_lane(v, 16)) + (rd_lane(v, 32) + rd_lane(v, 48));
}
__device__ __forceinline__ double exp_t(double v) { return exp(v); }
__device__ __forceinline__ double max_t(double a, double b) { return fmax(a, b); }
__device__ __forceinline__ float max_t(float a, float b) { return fmaxf(a, b); }
template <int CTRL> __device__ __forceinline__ double dpp_t(double v) { return dpp_d<CTRL>(v); }
template <int CTRL> __device__ __forceinline__ float dpp_t(float v) { return dpp<CTRL>(v); }
__device__ __forceinline__ float exp_t(float v) { return expf(v); }

// F = double: every step in f64 (the batch-1 decode path, exact against the f64 oracle to ~1e-12);
// F = float: fp32 scores, softmax and P.V (the batched path, which also accumulates its GEMMs in fp32).
// W waves per query head (1 or 2): wave W h + w takes positions (64 / W) w .. of the page; its lane
// (position (64 / W) w + lane / W, dim part lane % W) scores 128 / W dims and the W lanes of a position sum;
// with W = 2 the two waves of a head exchange their maximum and sum through LDS, so their P.V halves
// (lane l: dims 2l, 2l+1) share the page maximum and add into one partial (o[128], m, l) per (head, page).
// W = 2 halves the serial f64 work of each wave (the batch-1 latency); W = 1 keeps more workgroups
// resident (the batched throughput).
template <int G, typename F, int W>
__global__ void __launch_bounds__(G * W * 64) k_attn_decode(const AttnArgs a) {
  constexpr int PPW = PAGE / W, DPL = HD / W;
  __shared__ __align__(16) __half ks[PAGE][KROW];
  __shared__ __align__(16) __half vs[PAGE][HD];
  __shared__ __align__(16) F qf[G][HD];
  __shared__ F xm[G][W], xl[G][W];
  __shared__ __align__(16) F xo[W == 2 ? G : 1][HD];

  const int j = blockIdx.y;
  const int kvh = blockIdx.x / a.max_chunks, c = blockIdx.x % a.max_chunks;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int hh = wv / W, part = wv % W;
  const int pos = a.pos[j];
  const int pg = a.block_table[(size_t)j * a.bt_stride + c];
  const int hq = kvh * G + hh;
  if (c * PAGE > pos) return;                       // chunk beyond the context: nothing to do
  const int nvalid = min(PAGE, pos + 1 - c * PAGE);

  const uint4* kp = (const uint4*)(a.kcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  const uint4* vp = (const uint4*)(a.vcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  constexpr int NT = G * W * 64, PER = (PAGE * HD / 8 + NT - 1) / NT;
  uint4 kr[PER], vr[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = min((int)threadIdx.x + NT * i, PAGE * HD / 8 - 1);   // clamped: loads stay unconditional
    kr[i] = kp[e];
    vr[i] = vp[e];
  }
  if (part == 0) {
    const half2 qv = ((const half2*)(a.q + ((size_t)j * a.nh + hq) * HD))[lane];
    const float2 qq = __half22float2(qv);
    qf[hh][2 * lane] = (F)qq.x;
    qf[hh][2 * lane + 1] = (F)qq.y;
  }
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

  // scores: position p, dims DPL * dh .. + DPL - 1, then the W lanes of the position sum
  const int p = PPW * part + lane / W, dh = lane % W;
  F s;
  {
    const F* qh = qf[hh] + DPL * dh;
    F sp[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < DPL / 8; ++i) {
      const uint4 kk = *(const uint4*)&ks[p][DPL * dh + 8 * i];
      const __half2* k2 = (const __half2*)&kk;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 kf = __half22float2(k2[u]);
        sp[u] = fma(qh[8 * i + 2 * u], (F)kf.x, sp[u]);
        sp[u] = fma(qh[8 * i + 2 * u + 1], (F)kf.y, sp[u]);
      }
    }
    s = (sp[0] + sp[1]) + (sp[2] + sp[3]);
    if (W == 2) s += dpp_t<DPP_XOR1>(s);
  }
  s = p < nvalid ? s * (F)a.scale : (F)-INFINITY;
  F m = wmax(s);                                    // with W = 2 each position twice: harmless
  if (W == 2) {
    if (lane == 0) xm[hh][part] = m;
    __syncthreads();
    m = max_t(xm[hh][0], xm[hh][1]);
  }
  const F e = p < nvalid ? exp_t(s - m) : (F)0;
  const F lw = wsum(dh == 0 ? e : (F)0);
  if (W == 2 && lane == 0) xl[hh][part] = lw;

  // P.V over this wave's positions: lane owns dims 2*lane, 2*lane+1; position q's weight from lane W q
  F o[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const F ep = rd_lane(e, W * q);
    const float2 v = __half22float2(((const __half2*)vs[PPW * part + q])[lane]);
    o[q & 3][0] = fma(ep, (F)v.x, o[q & 3][0]);
    o[q & 3][1] = fma(ep, (F)v.y, o[q & 3][1]);
  }
  F o0 = (o[0][0] + o[1][0]) + (o[2][0] + o[3][0]);
  F o1 = (o[0][1] + o[1][1]) + (o[2][1] + o[3][1]);
  F l = lw;
  if (W == 2) {
    if (part == 1) {
      xo[hh][2 * lane] = o0;
      xo[hh][2 * lane + 1] = o1;
    }
    __syncthreads();
    if (part == 1) return;
    o0 += xo[hh][2 * lane];
    o1 += xo[hh][2 * lane + 1];
    l = xl[hh][0] + xl[hh][1];
  }
  double* P = a.part + (((size_t)j * a.nh + hq) * a.max_chunks + c) * (HD + 2);
  ((double2*)P)[lane] = make_double2((double)o0, (double)o1);
  if (lane == 0) { P[HD] = (double)m; P[HD + 1] = (double)l; }
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

// Standalone merge: one wave per (token, query head) -> fp32 o32 (optional) and Q8_1 oq/ods of the head's
// 128 values (4 blocks).
__global__ void __launch_bounds__(64) k_attn_merge(const AttnArgs a) {
  __shared__ double sm[HD];
  const int j = blockIdx.x, h = blockIdx.y;
  const int nch = a.pos[j] / PAGE + 1;
  attn_merge_head(a.part + ((size_t)j * a.nh + h) * a.max_chunks * (HD + 2), nch, sm);
  __syncthreads();
  const int n = a.nh * HD;
#pragma unroll
  for (int u = 0; u < 2; ++u) {                         // 64 lanes = two 32-value blocks per pass
    const int e = h * HD + 64 * u + threadIdx.x;
    const float v = (float)sm[64 * u + threadIdx.x];
    if (a.o32) a.o32[(size_t)j * n + e] = v;
    const int q = q8_1_lane32(v, a.ods + ((size_t)j * n + e) / 32, (e & 31) == 0);
    a.oq[(size_t)j * n + e] = (int8_t)q;
  }
}

}  // namespace q355
