// Decode GQA attention over the paged fp16 KV cache, split-K over pages (flash-decoding), gfx950.
//
// k_attn_decode: workgroup (chunk c, query head or heads of KV head g, token j), W waves per query head.
// It stages one 64-position K page (row-padded against LDS bank conflicts) and V page in LDS, the lanes
// of a position score it for their wave's head, the softmax numerator is a wave reduction, and lane l
// accumulates dims 2l, 2l+1 of P.V. Output: the unnormalised partial (o[128], m, l) per
// (token, query head, chunk). No atomics and no cross-workgroup waits.
// attn_merge_*: merges the partials of one token in fixed chunk order (o = sum_c e^(m_c - M) o_c / L)
// and quantizes the result to Q8_1 -- fused into the O-projection GEMV prologue, or standalone.
// Scores, softmax and P.V are computed in f64 (fp16 K/V and q widened exactly): the result feeds a Q8_1
// quantizer, so it must agree with the f64 oracle far below a quantization step.
// Semantics follow ATTN2 / ATTN4 (lab/qwen_kernels.py:358-442, 517-605).
#include "common.h"
#include "q355_kernels.h"

#ifndef Q355_TRACE_POINT
#define Q355_TRACE_POINT(k)
#endif

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
// F = float: fp32 scores, softmax and P.V (not launched: the batched path runs k_attn_decode_mfma below).
// W waves per query head (1, 2, 4, 8 or 16): wave W h + w takes positions (64 / W) w .. of the page; its lane
// (position (64 / W) w + lane / W, dim part lane % W) scores 128 / W dims and the W lanes of a position sum;
// with W > 1 the waves of a head exchange their maximum and sum through LDS, so their P.V parts
// (lane l: dims 2l, 2l+1) share the page maximum and add, in wave order, into one partial (o[128], m, l) per
// (head, page). HS workgroups share a page, each taking G / HS heads of the group (its K/V page staged by
// each). The library launches W = 4, HS = G.
template <int G, typename F, int W, int HS>
__global__ void __launch_bounds__(G / HS * W * 64) k_attn_decode(const AttnArgs a) {
  static_assert(G % HS == 0 && (W == 1 || W == 2 || W == 4 || W == 8 || W == 16), "k_attn_decode: head split / wave count");
  constexpr int GH = G / HS, PPW = PAGE / W, DPL = HD / W;
  __shared__ __align__(16) __half ks[PAGE][KROW];
  __shared__ __align__(16) __half vs[PAGE][HD];
  __shared__ __align__(16) F qf[GH][HD];
  __shared__ F xm[GH][W], xl[GH][W];
  __shared__ __align__(16) F xo[W > 1 ? GH : 1][W > 1 ? W - 1 : 1][HD];

  // grid.x = (query-head groups) x CH chunk slots, CH = max_chunks rounded up to a multiple of 8: workgroup
  // x runs on XCD x mod 8 = c mod 8, so the G / HS workgroups that stage the same K/V page share one L2
  const int j = blockIdx.y;
  const int CH = (a.max_chunks + 7) & ~7;
  const int c = blockIdx.x % CH, r = blockIdx.x / CH;
  const int kvh = r / HS, hs = r % HS;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int hh = wv / W, part = wv % W;
  // the page id does not depend on the position: both loads are in flight together
  const int pg = a.block_table[(size_t)j * a.bt_stride + min(c, a.max_chunks - 1)];
  const int pos = a.pos[j];
  if (c >= a.max_chunks || c * PAGE > pos) return;  // chunk slot beyond the table or the context: nothing to do
  const int hq = kvh * G + hs * GH + hh;
  const int nvalid = min(PAGE, pos + 1 - c * PAGE);

  const uint4* kp = (const uint4*)(a.kcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  const uint4* vp = (const uint4*)(a.vcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  constexpr int NT = GH * W * 64, PER = (PAGE * HD / 8 + NT - 1) / NT;
  uint4 kr[PER], vr[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = min((int)threadIdx.x + NT * i, PAGE * HD / 8 - 1);   // clamped: loads stay unconditional
    kr[i] = ld_stream16(kp + e);
    vr[i] = ld_stream16(vp + e);
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
    if (W >= 2) s += dpp_t<DPP_XOR1>(s);
    if (W >= 4) s += dpp_t<DPP_XOR2>(s);
    if (W >= 8) s += dpp_t<DPP_HALF_MIRROR>(s);   // the two quads of each 8 lanes
    if (W == 16) s += dpp_t<DPP_MIRROR>(s);       // the two halves of each 16-lane row
  }
  s = p < nvalid ? s * (F)a.scale : (F)-INFINITY;
  F m = wmax(s);                                    // with W > 1 each position W times: harmless
  if (W > 1) {
    if (lane == 0) xm[hh][part] = m;
    __syncthreads();
    m = xm[hh][0];
#pragma unroll
    for (int w = 1; w < W; ++w) m = max_t(m, xm[hh][w]);
  }
  const F e = p < nvalid ? exp_t(s - m) : (F)0;
  const F lw = wsum(dh == 0 ? e : (F)0);
  if (W > 1 && lane == 0) xl[hh][part] = lw;

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
  if (W > 1) {
    if (part > 0) {
      xo[hh][part - 1][2 * lane] = o0;
      xo[hh][part - 1][2 * lane + 1] = o1;
    }
    __syncthreads();
    if (part > 0) return;
#pragma unroll
    for (int w = 1; w < W; ++w) {
      o0 += xo[hh][w - 1][2 * lane];
      o1 += xo[hh][w - 1][2 * lane + 1];
      l += xl[hh][w];
    }
  }
  double* P = a.part + (((size_t)j * a.nh + hq) * a.max_chunks + c) * (HD + 2);
  ((double2*)P)[lane] = make_double2((double)o0, (double)o1);
  if (lane == 0) { P[HD] = (double)m; P[HD + 1] = (double)l; }
}

// ---------------------------------------------------------------------------------------------
// fp32 path on the matrix cores (the batched decode). Workgroup (token j, KV head, split sp) = 4 pages
// c = 4 sp .. 4 sp + 3, one wave per KW keys of them (KW = 64: a page per wave); the G query heads of the
// group are the MFMA columns (16 columns, G used). S^T = K Q^T takes K rows straight from global memory as A operands; V is transposed
// into the wave's own LDS slice through dword gathers (lane l: dims 2l, 2l + 1 of 8 keys, packed in pairs),
// so O^T = Vt P^T reads 8-key runs. P is rounded to fp16 for the MFMA (fp32 accumulation), max and
// exponent in log2 units.
// The wave partials merge through LDS (o = sum_w 2^(m_w - M) o_w, L likewise). A token whose context
// fits one split (<= 4 pages) is finished there: Q8_1 (oq/ods) or fp16 (oh), and fp32 o32 if asked.
// Otherwise every split writes its unnormalised (o, M, L) to the workspace (the `part` buffer: per (token,
// KV head) o [nsp][G][HD] then (M, L) [nsp][G], nsp = ceil(max_chunks / 4)) and k_attn_merge_split
// finishes the token. A cross-workgroup last-arrival merge inside this kernel was measured slower than the
// second launch (its coherent stores, counter round trip and coherent reloads cost more than a launch).
typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef float af4 __attribute__((ext_vector_type(4)));

// the finished head values of one thread (head h, dims 8 dg .. 8 dg + 7) -> the outputs
__device__ __forceinline__ void attn_out8(const AttnArgs& a, int j, int h, int dg, const float (&o)[8], bool live) {
  const int n = a.nh * HD;
  const size_t e = (size_t)j * n + h * HD + 8 * dg;
  if (live && a.o32) {
    *(float4*)(a.o32 + e) = make_float4(o[0], o[1], o[2], o[3]);
    *(float4*)(a.o32 + e + 4) = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (a.oh) {
    if (live) {
      unsigned pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const __half2 v = __floats2half2_rn(o[2 * i], o[2 * i + 1]);
        pk[i] = *reinterpret_cast<const unsigned*>(&v);
      }
      *(uint4*)(a.oh + e) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    return;
  }
  float df, d32;
  int sq;
  const uint2 q = q8_1_x8(o, df, sq, d32);             // the 4 threads of a quad hold one 32-value block
  if (live) {
    *(uint2*)(a.oq + e) = q;
    if ((dg & 3) == 0) a.ods[e / 32] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
  }
}

template <int KW>
__global__ void __launch_bounds__(4 * PAGE / KW * 64) k_attn_decode_mfma(const AttnArgs a) {
  Q355_TRACE_POINT(0);
  constexpr int NWV = 4 * PAGE / KW, ROW = KW + 4;     // waves; Vt row (one dim, KW keys) in halves
  __shared__ __align__(16) _Float16 vt[NWV][HD][ROW];
  __shared__ float wml[NWV][16][2];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int G = a.nh / a.nkv;
  const int nsp = (a.max_chunks + 3) / 4;
  // split-major order over the grid (nkv * nsp, T): all first splits are dispatched first, so the live
  // workgroups start early and the splits past short contexts (which return at once) come last
  const int wid = blockIdx.x + gridDim.x * blockIdx.y, per = gridDim.y * a.nkv;
  const int sp = wid / per, j = (wid % per) / a.nkv, kvh = wid % a.nkv;
  const int c = sp * 4 + wv / (PAGE / KW), k0 = (wv % (PAGE / KW)) * KW;   // page, first key in it
  // the page index does not depend on the position: both loads are in flight together
  const int pg = a.block_table[(size_t)j * a.bt_stride + min(c, a.max_chunks - 1)];
  const int pos = a.pos[j];
  const int nch = pos / PAGE + 1, nsplit = (nch + 3) / 4;
  if (sp >= nsplit) return;                             // uniform per workgroup
  const int nvalid = min(KW, pos + 1 - c * PAGE - k0);  // keys of this wave inside the context
  const bool live = nvalid > 0;                         // uniform per wave; wave 0 is always live
  const _Float16* kp = (const _Float16*)a.kcache + (((size_t)pg * a.nkv + kvh) * PAGE + k0) * HD;
  const unsigned* vp = (const unsigned*)(a.vcache + (((size_t)pg * a.nkv + kvh) * PAGE + k0) * HD);
  const int hq = kvh * G + li;

  af4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = af4{0.f, 0.f, 0.f, 0.f};
  float ml2 = -INFINITY, rs = 0.f;
  if (live) {
    // every load first, in the order of use: q, K operands (16 B per lane per 16-key tile), V dwords; the
    // wait for q and K (in-order counter) then leaves the V loads in flight during the scores and softmax
    uint4 qr[4];                                        // unconditional (clamped head): straight-line loads
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qr[cc] = *(const uint4*)(a.q + ((size_t)j * a.nh + kvh * G + min(li, G - 1)) * HD + 32 * cc + 8 * lg);
    uint4 kA[KW / 16][4];
#pragma unroll
    for (int t = 0; t < KW / 16; ++t)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) kA[t][cc] = ld_stream16(kp + (16 * t + li) * HD + 32 * cc + 8 * lg);
    unsigned vr[KW / 8][8];
#pragma unroll
    for (int kg = 0; kg < KW / 8; ++kg)
#pragma unroll
      for (int u = 0; u < 8; ++u) vr[kg][u] = ld_stream4(vp + (kg * 8 + u) * (HD / 2) + lane);
    __asm__ __volatile__("" ::: "memory");              // keep every load above issued before the first product
    ah8 qB[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const uint4 q = li < G ? qr[cc] : make_uint4(0, 0, 0, 0);
      qB[cc] = *reinterpret_cast<const ah8*>(&q);
    }

    // S^T: keys 16t + 4lg + v (rows), head li (column)
    af4 sc[KW / 16];
#pragma unroll
    for (int t = 0; t < KW / 16; ++t) {
      sc[t] = af4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<ah8*>(&kA[t][cc]), qB[cc], sc[t], 0, 0, 0);
    }
    const float sl2 = (float)a.scale * 1.4426950408889634f;
    float bm = -INFINITY;
#pragma unroll
    for (int t = 0; t < KW / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (16 * t + 4 * lg + v >= nvalid) sc[t][v] = -INFINITY;
        bm = fmaxf(bm, sc[t][v]);
      }
    bm = col4_max(bm);                                  // key 0 of a live wave is valid: finite
    Q355_TRACE_POINT(1);
    ml2 = bm * sl2;
    ah8 pB[KW / 32];
#pragma unroll
    for (int t = 0; t < KW / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sc[t][v], sl2, -ml2));
        rs += p;
        pB[t >> 1][4 * (t & 1) + v] = (_Float16)p;
      }
    rs = col4_sum(rs);

    // V -> Vt in this wave's LDS slice (keys past the context zeroed: p = 0 there, V may hold anything)
#pragma unroll
    for (int kg = 0; kg < KW / 8; ++kg) {
      u32x4 lo, hi;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const unsigned v0 = kg * 8 + 2 * jj < nvalid ? vr[kg][2 * jj] : 0u;
        const unsigned v1 = kg * 8 + 2 * jj + 1 < nvalid ? vr[kg][2 * jj + 1] : 0u;
        lo[jj] = __builtin_amdgcn_perm(v1, v0, 0x05040100u);
        hi[jj] = __builtin_amdgcn_perm(v1, v0, 0x07060302u);
      }
      *(u32x4*)&vt[wv][2 * lane][kg * 8] = lo;
      *(u32x4*)&vt[wv][2 * lane + 1][kg * 8] = hi;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);                 // lgkmcnt(0): this wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();

    // O^T = Vt P^T; 32-key chunk cc2 in k-slot order 8g + i -> key 32 cc2 + 4g + i (i < 4), + 16 + 4g + i - 4
#pragma unroll
    for (int cc2 = 0; cc2 < KW / 32; ++cc2)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const _Float16* row = &vt[wv][16 * dt + li][0];
        const uint2 lo = *(const uint2*)(row + 32 * cc2 + 4 * lg);
        const uint2 hi = *(const uint2*)(row + 32 * cc2 + 16 + 4 * lg);
        uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<ah8*>(&vv), pB[cc2], acc[dt], 0, 0, 0);
      }
  }

  // the wave partials -> LDS (over the Vt slices), merged per (head, 8 dims) by thread t < 256
  Q355_TRACE_POINT(2);
  __syncthreads();
  Q355_TRACE_POINT(3);
  float* po = (float*)&vt[0][0][0];                     // [NWV waves][16 heads][HD]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) *(af4*)(po + (wv * 16 + li) * HD + 16 * dt + 4 * lg) = acc[dt];
  if (lg == 0) {
    wml[wv][li][0] = ml2;
    wml[wv][li][1] = rs;
  }
  __syncthreads();
  if (threadIdx.x >= 256) return;
  const int h = threadIdx.x >> 4, dg = threadIdx.x & 15;   // quads share h: whole quads are live or not
  const bool hl = h < G;
  float o[8], M = -INFINITY, L = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; ++w) M = fmaxf(M, wml[w][h][0]);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    const float f = __builtin_amdgcn_exp2f(wml[w][h][0] - M);   // 0 for waves past the context
    L = fmaf(f, wml[w][h][1], L);
    const float4 x0 = *(const float4*)(po + (w * 16 + h) * HD + 8 * dg);
    const float4 x1 = *(const float4*)(po + (w * 16 + h) * HD + 8 * dg + 4);
    o[0] = fmaf(f, x0.x, o[0]); o[1] = fmaf(f, x0.y, o[1]); o[2] = fmaf(f, x0.z, o[2]); o[3] = fmaf(f, x0.w, o[3]);
    o[4] = fmaf(f, x1.x, o[4]); o[5] = fmaf(f, x1.y, o[5]); o[6] = fmaf(f, x1.z, o[6]); o[7] = fmaf(f, x1.w, o[7]);
  }

  if (nsplit > 1) {                                     // split partial -> workspace; k_attn_merge_split ends it
    float* wo = (float*)a.part + ((size_t)j * a.nkv + kvh) * ((size_t)nsp * G * (HD + 2));
    float* wm = wo + (size_t)nsp * G * HD;
    if (hl) {
      float4* dst = (float4*)(wo + ((size_t)sp * G + h) * HD + 8 * dg);
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      dst[1] = make_float4(o[4], o[5], o[6], o[7]);
      if (dg == 0) *(float2*)(wm + ((size_t)sp * G + h) * 2) = make_float2(M, L);
    }
    return;
  }
  const float inv = hl ? 1.f / L : 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] *= inv;
  attn_out8(a, j, kvh * G + (hl ? h : 0), dg, o, hl);
}

// Merge of the split partials of k_attn_decode_mfma for tokens whose context spans several splits: one
// workgroup per (KV head, token), thread t = (head t / 16, dims 8 (t % 16) ..); every split's (M, L) and 8
// values are loaded before the first use (nsplit <= 16).
__global__ void __launch_bounds__(256) k_attn_merge_split(const AttnArgs a) {
  const int G = a.nh / a.nkv;
  const int nsp = (a.max_chunks + 3) / 4;
  const int kvh = blockIdx.x, j = blockIdx.y;
  const int nsplit = (a.pos[j] / PAGE + 1 + 3) / 4;
  if (nsplit == 1) return;                              // finished by the attention kernel
  const int h = threadIdx.x >> 4, dg = threadIdx.x & 15;
  const bool hl = h < G;
  const int hh = hl ? h : 0;
  const float* wo = (const float*)a.part + ((size_t)j * a.nkv + kvh) * ((size_t)nsp * G * (HD + 2));
  const float* wm = wo + (size_t)nsp * G * HD;
  float2 ml[16];
  float4 x0[16], x1[16];
#pragma unroll
  for (int s = 0; s < 16; ++s)
    if (s < nsplit) {
      ml[s] = *(const float2*)(wm + ((size_t)s * G + hh) * 2);
      x0[s] = *(const float4*)(wo + ((size_t)s * G + hh) * HD + 8 * dg);
      x1[s] = *(const float4*)(wo + ((size_t)s * G + hh) * HD + 8 * dg + 4);
    }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < 16; ++s)
    if (s < nsplit) M = fmaxf(M, ml[s].x);
  float o[8], L = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
  for (int s = 0; s < 16; ++s)
    if (s < nsplit) {
      const float f = __builtin_amdgcn_exp2f(ml[s].x - M);
      L = fmaf(f, ml[s].y, L);
      o[0] = fmaf(f, x0[s].x, o[0]); o[1] = fmaf(f, x0[s].y, o[1]); o[2] = fmaf(f, x0[s].z, o[2]);
      o[3] = fmaf(f, x0[s].w, o[3]); o[4] = fmaf(f, x1[s].x, o[4]); o[5] = fmaf(f, x1[s].y, o[5]);
      o[6] = fmaf(f, x1[s].z, o[6]); o[7] = fmaf(f, x1[s].w, o[7]);
    }
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] *= inv;
  attn_out8(a, j, kvh * G + hh, dg, o, hl);
}

// ---------------------------------------------------------------------------------------------
// Merge of the chunk partials of one (token, query head), f64, by ONE wave: lane c reads chunk c's
// (m_c, l_c) and forms w_c = e^(m_c - M) (M = max_c m_c); lane l then sums dims 2l, 2l+1 of
// sum_c w_c o_c in fixed chunk order (w_c broadcast from lane c) and divides by L = sum_c w_c l_c.
// All loads of a group of 8 chunks are issued before their first use. nch <= 64.
// The first batch of loads is clamped by maxc (the chunk slots the partials buffer holds), not by nch, so it
// does not wait for the position; chunks past nch are masked to 0 (stale slots may hold anything).
__device__ __forceinline__ void attn_merge_head(const double* __restrict__ P, int maxc, int nch, double* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const double* pc = P + (size_t)min(lane, maxc - 1) * (HD + 2);
  const double mc = pc[HD], lc = pc[HD + 1];
  double2 v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = ((const double2*)(P + (size_t)min(u, maxc - 1) * (HD + 2)))[lane];
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
      const bool live = c0 + u < nch;
      o0 = fma(wc, live ? v[u].x : 0.0, o0);
      o1 = fma(wc, live ? v[u].y : 0.0, o1);
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
// 128 values (4 blocks), or fp16 oh.
__global__ void __launch_bounds__(64) k_attn_merge(const AttnArgs a) {
  __shared__ double sm[HD];
  const int j = blockIdx.x, h = blockIdx.y;
  const int nch = a.pos[j] / PAGE + 1;
  attn_merge_head(a.part + ((size_t)j * a.nh + h) * a.max_chunks * (HD + 2), a.max_chunks, nch, sm);
  __syncthreads();
  const int n = a.nh * HD;
  if (a.oh) {                                           // fp16 output (the fp16 batched path)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = h * HD + 64 * u + threadIdx.x;
      a.oh[(size_t)j * n + e] = half_rn(sm[64 * u + threadIdx.x]);
      if (a.o32) a.o32[(size_t)j * n + e] = (float)sm[64 * u + threadIdx.x];
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {                         // 64 lanes = two 32-value blocks per pass
    const int e = h * HD + 64 * u + threadIdx.x;
    const float v = (float)sm[64 * u + threadIdx.x];
    if (a.o32) a.o32[(size_t)j * n + e] = v;
    const int q = q8_1_lane32(v, a.ods + ((size_t)j * n + e) / 32, (e & 31) == 0);
    a.oq[(size_t)j * n + e] = (int8_t)q;
  }
}

// Merge of k_attn_batch_f64's split partials, f64, in split order: o = sum_s e^(M_s - M) o_s / sum_s
// e^(M_s - M) L_s (M = max_s M_s). Workgroup (KV head, token), thread (head t / 64, dims 2 (t % 64), + 1):
// the splits' (M, L) and two values are loaded in batches of up to SB splits (one memory latency each; a
// later batch rescales the earlier sums to its maximum), then Q8_1 per 16-lane row (one 32-value block).
// COH: the partials were written by other workgroups of the same launch (device-scope stores), so they are read
// with device-scope loads; otherwise by an earlier launch, read with ordinary loads.
template <int G, int SPG, int SB, bool COH>
__device__ __forceinline__ void merge_f64(const AttnArgs& a, const int kvh, const int j, const int nsplit,
                                          const int tid) {
  const int nsp = (a.max_chunks + SPG - 1) / SPG;
  const int h = tid >> 6, dp = tid & 63;
  const double* P0 = a.part + (((size_t)j * a.nkv + kvh) * nsp * G + h) * (HD + 2);
  const size_t st = (size_t)G * (HD + 2);
  const Coh16 coh(P0, (unsigned)(nsp * st * 8));      // P0 is uniform per wave (one head per wave)
  auto ld2 = [&](size_t e) {                          // the double2 at P0 + e
    return COH ? __builtin_bit_cast(double2, coh.ld((unsigned)(e * 8))) : *(const double2*)(P0 + e);
  };
  double M = -INFINITY, o0 = 0.0, o1 = 0.0, L = 0.0;
  for (int s0 = 0; s0 < nsplit; s0 += SB) {             // one batch (one memory latency) up to SB splits
    double2 ml[SB], x[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s)
      if (s0 + s < nsplit) {
        ml[s] = ld2((s0 + s) * st + HD);
        x[s] = ld2((s0 + s) * st + 2 * dp);
      }
    double Mb = M;
#pragma unroll
    for (int s = 0; s < SB; ++s)
      if (s0 + s < nsplit) Mb = fmax(Mb, ml[s].x);
    if (s0) {                                           // rescale the earlier batches to the new maximum
      const double r = exp(M - Mb);
      o0 *= r; o1 *= r; L *= r;
    }
    M = Mb;
#pragma unroll
    for (int s = 0; s < SB; ++s)
      if (s0 + s < nsplit) {
        const double f = exp(ml[s].x - M);
        L = fma(f, ml[s].y, L);
        o0 = fma(f, x[s].x, o0);
        o1 = fma(f, x[s].y, o1);
      }
  }
  const float v0 = (float)(o0 / L), v1 = (float)(o1 / L);
  const size_t n = (size_t)a.nh * HD, e = (size_t)j * n + (size_t)(kvh * G + h) * HD + 2 * dp;
  if (a.o32) *(float2*)(a.o32 + e) = make_float2(v0, v1);
  // Q8_1 of the row's 32 values (16 lanes x 2), the rule of q8_code
  float amax = fmaxf(fabsf(v0), fabsf(v1));
  amax = fmaxf(amax, dpp<DPP_XOR1>(amax));
  amax = fmaxf(amax, dpp<DPP_XOR2>(amax));
  amax = fmaxf(amax, dpp<DPP_HALF_MIRROR>(amax));
  amax = fmaxf(amax, dpp<DPP_MIRROR>(amax));
  const float d32 = q8_scale(amax);
  const int q0 = q8_code(v0, d32), q1 = q8_code(v1, d32);
  int sq = q0 + q1;
  sq += dpp<DPP_XOR1>(sq);
  sq += dpp<DPP_XOR2>(sq);
  sq += dpp<DPP_HALF_MIRROR>(sq);
  sq += dpp<DPP_MIRROR>(sq);
  *(short*)(a.oq + e) = (short)((q0 & 255) | ((q1 & 255) << 8));
  if ((dp & 15) == 0) a.ods[e / 32] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
}

// ---------------------------------------------------------------------------------------------
// f64 batched decode attention (the int8 batched path): the arithmetic of the batch-1 kernel above -- f64
// scores, softmax and P.V from fp16 q/K/V widened exactly -- at the throughput of a batch. Workgroup
// (token j, KV head, split sp) = SPG pages c = SPG sp + pg, all G query heads of the group, 4 waves per page:
// wave (pg, dq) owns dims 32 dq .. 32 dq + 31 of page pg, so each wave's dependency chain is a quarter of
// a page's work and a batch launches four waves per page (the latency of one wave is hidden by the others).
//  1. scores: lane = key; its 32 K values widened once, then per head 32 FMAs whose q operands are the f64
//     queries (q64, written by the QKV epilogue), replicated in every 16-lane row and read as row-broadcast
//     DPP operands of v_fmac_f64; partials -> LDS;
//  2. softmax: wave h sums the 4 quarters in order, max / exp / sum over the split's keys (f64 exp);
//  3. P.V: lane (dim pair 32 dq + 2 (l % 16), keys 4 t + l / 16 of page pg); the p of the row's 16 keys sit
//     one per lane and reach the FMAs as row-broadcast DPP operands; the 4 key groups add through lane
//     swaps and the pages of the split in page order.
// A token whose context fits one split is finished here (Q8_1 oq/ods, fp32 o32 if asked); otherwise each
// split writes its unnormalised (o[G][HD], M[G], L[G]) to part [T][nkv][nsp][G][HD + 2] (nsp =
// ceil(max_chunks / SPG)) and k_attn_merge_f64 finishes the token in split order.
// acc += bcast(q, lane OFF + i of each 16-lane row) * k_i for i = 0..7: v_fmac_f64 with a DPP row_newbcast
// source (gfx950's 64-bit DPP), so a row-uniform f64 operand costs no broadcast instruction. s_nop 1: the two
// wait states a DPP source needs after a VALU write of it.
template <int OFF>
__device__ __forceinline__ void fma8_bcast(double& acc, double q, const double (&k)[8]) {
  asm("s_nop 1\n\t"
      "v_fmac_f64_dpp %0, %1, %2 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %3 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %4 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %5 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %6 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %7 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %8 row_newbcast:%16 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %0, %1, %9 row_newbcast:%17 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(q), "v"(k[0]), "v"(k[1]), "v"(k[2]), "v"(k[3]), "v"(k[4]), "v"(k[5]), "v"(k[6]), "v"(k[7]),
        "n"(OFF), "n"(OFF + 1), "n"(OFF + 2), "n"(OFF + 3), "n"(OFF + 4), "n"(OFF + 5), "n"(OFF + 6), "n"(OFF + 7));
}
// o[h][u], o[h + 1][u] += bcast(p[h], p[h + 1]: lane T of each row) * v_u (two heads of one P.V key)
template <int T>
__device__ __forceinline__ void fma_pv2(double& o00, double& o01, double& o10, double& o11, double p0, double p1,
                                        double v0, double v1) {
  asm("s_nop 1\n\t"
      "v_fmac_f64_dpp %0, %4, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %1, %4, %7 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %2, %5, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f64_dpp %3, %5, %7 row_newbcast:%8 row_mask:0xf bank_mask:0xf"
      : "+v"(o00), "+v"(o01), "+v"(o10), "+v"(o11)
      : "v"(p0), "v"(p1), "v"(v0), "v"(v1), "n"(T));
}
template <int T, int G>
__device__ __forceinline__ void pv_key(double (&o)[G][2], const double (&pr)[G], const unsigned (&vr)[16], int kg,
                                       int nvalid) {
  const unsigned vv = 4 * T + kg < nvalid ? vr[T] : 0u;   // rows past the context may hold anything
  const float2 vf = __half22float2(*(const __half2*)&vv);
  const double v0 = (double)vf.x, v1 = (double)vf.y;
#pragma unroll
  for (int h = 0; h < G; h += 2) fma_pv2<T>(o[h][0], o[h][1], o[h + 1][0], o[h + 1][1], pr[h], pr[h + 1], v0, v1);
  __builtin_amdgcn_sched_barrier(0);                    // one key's conversions live at a time
}
template <int G, int... T>
__device__ __forceinline__ void pv_keys(double (&o)[G][2], const double (&pr)[G], const unsigned (&vr)[16], int kg,
                                        int nvalid, std::integer_sequence<int, T...>) {
  (pv_key<T, G>(o, pr, vr, kg, nvalid), ...);
}

// EARLY (launches with few workgroups, where occupancy does not matter): a register budget of two waves per
// SIMD instead of six, spent on issuing the V loads together with the K loads (one memory latency instead of
// two on the workgroup's path) and on the in-kernel merge's load batches of 20 splits instead of 4.
template <int G, int SPG, bool EARLY = false>
__global__ void __launch_bounds__(SPG * 256) __attribute__((amdgpu_waves_per_eu(EARLY ? 2 : 6)))
k_attn_batch_f64(const AttnArgs a) {
  Q355_TRACE_POINT(0);
  static_assert(G % 2 == 0 && G <= 8, "heads per KV group");
  static_assert(SPG * 4 >= G, "the in-kernel merge takes one wave per query head");
  constexpr int KEYS = SPG * PAGE;
  __shared__ __align__(16) double sq[4][G][KEYS];      // score partials per dim quarter
  __shared__ __align__(16) double ps[KEYS][G];         // p per key (16-byte reads give two heads)
  __shared__ __align__(16) double po[SPG][G][HD];      // per-page P.V
  __shared__ double xm[G], xl[G];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pg = wv >> 2, dq = wv & 3;
  const int nsp = (a.max_chunks + SPG - 1) / SPG;
  const int wid = blockIdx.x + gridDim.x * blockIdx.y;
  int sp, j, kvh, pgid, pos;
  if (a.work) {
    // the step's live items, packed at the front of the grid: one load gives the item, its position and its
    // page ids, so the K loads follow after one memory latency, and the empty slots at the end exit at once
    static_assert(SPG <= 2, "a work item carries two page ids");
    const int4 it = a.work[wid];
    if (it.x < 0) return;                               // uniform per workgroup
    j = it.x & 0xffff;
    kvh = (it.x >> 16) & 0xff;
    sp = it.x >> 24;
    pos = it.y;
    pgid = pg == 0 ? it.z : it.w;
  } else {
    // split-major order over the grid (nkv * nsp, T): the first splits of every token are dispatched first
    const int per = gridDim.y * a.nkv;
    sp = wid / per;
    j = (wid % per) / a.nkv;
    kvh = wid % a.nkv;
    // the page id does not depend on the position: both loads are in flight together
    pgid = a.block_table[(size_t)j * a.bt_stride + min(sp * SPG + pg, a.max_chunks - 1)];
    pos = a.pos[j];
  }
  const int c = sp * SPG + pg;
  const int nch = pos / PAGE + 1, nsplit = (nch + SPG - 1) / SPG;
  if (sp >= nsplit) return;                             // uniform per workgroup
  const bool live = c < nch;                            // uniform per wave; page 0 of the split is always live
  const int nvalid = live ? min(PAGE, pos + 1 - c * PAGE) : 0;
  const size_t base = live ? (((size_t)pgid * a.nkv + kvh) * PAGE * HD) : 0;

  // this wave's f64 q values: qd[h][f] holds dims 32 dq + 16 f + (l % 16) of head h in every 16-lane row, so
  // the scores' FMAs take them as row-broadcast DPP operands
  double qd[G][2];
  const int kg = lane >> 4, dp = lane & 15;
  unsigned vr[16];
  if (live) {
    const double* q = a.q64 + ((size_t)j * a.nh + kvh * G) * HD + 32 * dq + (lane & 15);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      qd[h][0] = q[h * HD];
      qd[h][1] = q[h * HD + 16];
    }
  }
  Q355_TRACE_POINT(1);
  // 1. scores of this wave's dim quarter
  if (live) {
    uint4 kr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kr[i] = ld_stream16(a.kcache + base + (size_t)lane * HD + 32 * dq + 8 * i);
    if (EARLY) {
#pragma unroll
      for (int t = 0; t < 16; ++t)
        vr[t] = ld_stream4(a.vcache + base + (size_t)(4 * t + kg) * HD + 32 * dq + 2 * dp);
    }
    double acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {                       // 8 dims at a time (fewer live registers)
      double kd[8];
      const __half2* k2 = (const __half2*)&kr[c];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 kf = __half22float2(k2[u]);
        kd[2 * u] = (double)kf.x;
        kd[2 * u + 1] = (double)kf.y;
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        if (c & 1) fma8_bcast<8>(acc[h], qd[h][c >> 1], kd);
        else fma8_bcast<0>(acc[h], qd[h][c >> 1], kd);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) sq[dq][h][pg * PAGE + lane] = acc[h];
    // V operands of phase 3, in flight during the softmax: keys 4 t + l / 16, dims 32 dq + 2 (l % 16)
    if (!EARLY) {
#pragma unroll
      for (int t = 0; t < 16; ++t)
        vr[t] = ld_stream4(a.vcache + base + (size_t)(4 * t + kg) * HD + 32 * dq + 2 * dp);
    }
  } else {
#pragma unroll
    for (int h = 0; h < G; ++h) sq[dq][h][pg * PAGE + lane] = 0.0;
  }
  __syncthreads();
  Q355_TRACE_POINT(2);
  // 2. softmax: wave w takes heads w, w + 4 SPG, ... over the split's keys (SPG per lane)
  for (int h = wv; h < G; h += 4 * SPG) {
    double sv[SPG], m = -INFINITY;
#pragma unroll
    for (int g = 0; g < SPG; ++g) {
      const int key = g * PAGE + lane;
      const bool ok = sp * SPG * PAGE + key <= pos;
      const double v = ((sq[0][h][key] + sq[1][h][key]) + sq[2][h][key]) + sq[3][h][key];
      sv[g] = ok ? v * a.scale : -INFINITY;
      m = fmax(m, sv[g]);
    }
    const double M = wave_max_d(m);                     // key 0 of the split is valid: finite
    double l = 0.0;
#pragma unroll
    for (int g = 0; g < SPG; ++g) {
      const double p = sv[g] == -INFINITY ? 0.0 : exp(sv[g] - M);
      ps[g * PAGE + lane][h] = p;
      l += p;
    }
    l = wave_sum_d(l);
    if (lane == 0) { xm[h] = M; xl[h] = l; }
  }
  __syncthreads();
  Q355_TRACE_POINT(3);
  // 3. P.V of this wave's dims and page: lane (row kg, position t) holds p of key 4 t + kg of the page, which
  // the FMAs of key 4 t + kg read as a row broadcast
  if (live) {
    double pr[G];
    const double* prow = &ps[pg * PAGE + 4 * dp + kg][0];
#pragma unroll
    for (int h = 0; h < G; h += 2) {
      const double2 v = *(const double2*)(prow + h);
      pr[h] = v.x;
      pr[h + 1] = v.y;
    }
    double o[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) o[h][0] = o[h][1] = 0.0;
    pv_keys<G>(o, pr, vr, kg, nvalid, std::make_integer_sequence<int, 16>{});
    // the 4 key groups (lanes l, l ^ 16, l ^ 32, l ^ 48): two lane swaps; x + y == y + x, so all four lanes
    // end with the same bits
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        double x = o[h][u];
        {
          const int2 b = *reinterpret_cast<const int2*>(&x);
          const auto rl = __builtin_amdgcn_permlane16_swap((unsigned)b.x, (unsigned)b.x, false, false);
          const auto rh = __builtin_amdgcn_permlane16_swap((unsigned)b.y, (unsigned)b.y, false, false);
          const int2 a0 = make_int2((int)rl[0], (int)rh[0]), a1 = make_int2((int)rl[1], (int)rh[1]);
          x = *reinterpret_cast<const double*>(&a0) + *reinterpret_cast<const double*>(&a1);
        }
        {
          const int2 b = *reinterpret_cast<const int2*>(&x);
          const auto rl = __builtin_amdgcn_permlane32_swap((unsigned)b.x, (unsigned)b.x, false, false);
          const auto rh = __builtin_amdgcn_permlane32_swap((unsigned)b.y, (unsigned)b.y, false, false);
          const int2 a0 = make_int2((int)rl[0], (int)rh[0]), a1 = make_int2((int)rl[1], (int)rh[1]);
          x = *reinterpret_cast<const double*>(&a0) + *reinterpret_cast<const double*>(&a1);
        }
        o[h][u] = x;
      }
    if (lane < 16) {
#pragma unroll
      for (int h = 0; h < G; ++h) *(double2*)&po[pg][h][32 * dq + 2 * dp] = make_double2(o[h][0], o[h][1]);
    }
  }
  __syncthreads();
  Q355_TRACE_POINT(4);
  // 4. thread (head h, dims 8 dg .. 8 dg + 7): the split's live pages in page order
  const int t = threadIdx.x;
  if (t < G * 16) {                                     // whole quads (Q8_1 blocks) stay together
    const int h = t >> 4, dg = t & 15;
    const int nlive = min(SPG, nch - sp * SPG);
    double od[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) od[i] = po[0][h][8 * dg + i];
    for (int g = 1; g < nlive; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) od[i] += po[g][h][8 * dg + i];
    if (nsplit == 1) {
      float of[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) of[i] = (float)(od[i] / xl[h]);
      attn_out8(a, j, kvh * G + h, dg, of, true);
    } else if (a.arrivals) {
      // device-scope stores (written through to the memory every XCD reads): the merging workgroup may run on
      // another XCD and reads them with device-scope loads, so no cache writeback or invalidate is needed
      const Coh16 P(a.part + (((size_t)j * a.nkv + kvh) * nsp + sp) * G * (HD + 2), G * (HD + 2) * 8);
      const unsigned e = (unsigned)(h * (HD + 2) + 8 * dg) * 8;
#pragma unroll
      for (int i = 0; i < 8; i += 2) P.st16(e + i * 8, __builtin_bit_cast(int4, make_double2(od[i], od[i + 1])));
      if (dg == 0) P.st16((unsigned)(h * (HD + 2) + HD) * 8, __builtin_bit_cast(int4, make_double2(xm[h], xl[h])));
    } else {                                            // merged by a later launch
      double* P = a.part + ((((size_t)j * a.nkv + kvh) * nsp + sp) * G + h) * (HD + 2);
#pragma unroll
      for (int i = 0; i < 8; i += 2) *(double2*)(P + 8 * dg + i) = make_double2(od[i], od[i + 1]);
      if (dg == 0) *(double2*)(P + HD) = make_double2(xm[h], xl[h]);
    }
  }
  Q355_TRACE_POINT(5);
  if (nsplit == 1 || !a.arrivals) return;             // uniform per workgroup
  // 5. the last split of this (token, KV head) to finish merges all of them (no separate merge launch): every
  // thread's partial stores are acknowledged before the workgroup counts itself, so the last to count finds
  // every split's partials; it resets the counter for the next launch
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    int* cnt = a.arrivals + (size_t)j * a.nkv + kvh;
    last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
    if (last) stc(cnt, 0);
  }
  __syncthreads();
  Q355_TRACE_POINT(6);
  if (!last) return;
  if (t < G * 64) merge_f64<G, SPG, EARLY ? 20 : 4, true>(a, kvh, j, nsplit, t);   // splits per load batch: VGPR budget
  Q355_TRACE_POINT(7);
}

// The live work items of k_attn_batch_f64 for one step, built by one wave (T <= 64 tokens, lane t = token t):
// split-major, then token, then KV head -- the order of the plain grid with the dead splits left out -- followed
// by empty items (-1) up to cap, the grid size. Each item carries the token's position and the page ids of the
// split's (up to) two pages. Item index of (t, sp) = the live (token, split) pairs of earlier splits + the live
// tokens before t in split sp, from one ballot per split (no barriers). The positions do not change within a
// step, so one list serves all layers.
template <int SPG>
__global__ void __launch_bounds__(64) k_attn_worklist(const int* __restrict__ pos, const int* __restrict__ bt,
                                                      int bt_stride, int T, int nkv, int max_chunks,
                                                      int4* __restrict__ work, int cap) {
  const int t = threadIdx.x;
  const int nsp = (max_chunks + SPG - 1) / SPG;
  int ns = 0, p = 0;
  if (t < T) {
    p = pos[t];
    ns = min(nsp, (p / PAGE + 1 + SPG - 1) / SPG);
  }
  const int* row = bt + (size_t)min(t, T - 1) * bt_stride;
  int base = 0;
  for (int sp = 0; sp < nsp; ++sp) {
    const unsigned long long m = __ballot(sp < ns);
    if (m == 0ull) break;                               // no token has this split, nor any later one
    if (sp < ns) {
      int4 it = make_int4(t | (sp << 24), p, row[min(sp * SPG, max_chunks - 1)], row[min(sp * SPG + 1, max_chunks - 1)]);
      const size_t idx = (size_t)(base + __popcll(m & ((1ull << t) - 1ull))) * nkv;
      for (int k = 0; k < nkv; ++k, it.x += 1 << 16) work[idx + k] = it;
    }
    base += __popcll(m);
  }
  for (int i = base * nkv + t; i < cap; i += 64) work[i] = make_int4(-1, 0, 0, 0);
}

// The merge as its own launch: workgroup (KV head, token).
template <int G, int SPG>
__global__ void __launch_bounds__(G * 64) k_attn_merge_f64(const AttnArgs a) {
  const int kvh = blockIdx.x, j = blockIdx.y;
  const int nsplit = (a.pos[j] / PAGE + 1 + SPG - 1) / SPG;
  if (nsplit == 1) return;                              // finished by the attention kernel
  merge_f64<G, SPG, 20, false>(a, kvh, j, nsplit, threadIdx.x);   // 20 splits (2 KB of context each) per load batch
}

}  // namespace q355
