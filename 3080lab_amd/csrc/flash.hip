// Causal GQA flash attention for prefill on fp16 MFMA (v_mfma_f32_16x16x32_f16), gfx950.
//
// Semantics of flash_prefill_v3 (lab/qwen_batched.py:1795-2037) and the torch reference of
// scripts/flash_bench.py:51-65: query i of the chunk (position pos0 + i) attends to keys 0..pos0 + i of
// its sequence; scores q.k * scale, softmax with running max (exp2 of scores pre-scaled by log2 e),
// fp16 P, fp32 accumulation; output o = sum p v / sum p in fp32.
//
// Workgroup = 64 queries of one query head (grid (ceil(P/64), nh)); wave w owns queries 16w..16w+15.
// Per 64-key block (one KV page): K (row-padded) and V transposed (Vt[dim][key]) are staged in LDS,
// the next page is loaded into registers while the current one is used.
// The wave computes S^T = K Q^T (A = K rows from LDS, B = the wave's Q rows held in registers), so lane l
// holds scores of ONE query (l % 16) for keys 16t + 4(l/16) + v: the softmax statistics of a query live
// in the 4 lanes l % 16 + 16g and need only two cross-lane steps. The same registers, converted to fp16,
// are directly the B operand of O^T = Vt P^T when a 32-key chunk c is ordered as k-slot 8g + j ->
// key 32c + 4g + j (j < 4), 32c + 16 + 4g + j - 4 (j >= 4); Vt is read in that order (two 8-byte
// LDS reads). O^T accumulators are again per query l % 16 (dims 16dt + 4g + v), so the running-max
// rescale is per lane.
// MFMA operand layouts (16x16x32): lane l holds A[row l%16][k 8(l/16)..+8], B[k 8(l/16)..+8][col l%16],
// C[row 4(l/16)+v][col l%16].
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int FK_ROW = HD + 8;     // K row in LDS (halves), padded
constexpr int FV_ROW = PAGE + 8;   // Vt row (one dim, 64 keys) in LDS (halves), padded

__device__ __forceinline__ h8 as_h8(uint4 v) { return *reinterpret_cast<h8*>(&v); }

__global__ void __launch_bounds__(256) k_attn_prefill(const PrefillAttnArgs a) {
  __shared__ __align__(16) _Float16 ks[PAGE][FK_ROW];
  __shared__ __align__(16) _Float16 vt[HD][FV_ROW];
  const int qb = blockIdx.x, hq = blockIdx.y;
  const int kvh = hq / (a.nh / a.nkv);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int qi = qb * 64 + wv * 16 + li;                 // this lane's query (chunk index)
  const int qc = min(qi, a.P - 1);
  const int qpos = a.pos0 + qi;                          // its position
  const int nq = a.nh * HD;

  // the wave's Q rows as B operands: dims 32c + 8g .. +8 of query qc
  h8 qf[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qf[c] = as_h8(*(const uint4*)(a.q + (size_t)qc * nq + hq * HD + 32 * c + 8 * lg));

  const int last_key = min(a.pos0 + qb * 64 + 63, a.pos0 + a.P - 1);   // largest key any query here needs
  const int nkb = last_key / PAGE + 1;
  const float sl2 = a.scale * 1.4426950408889634f;       // scores in log2 units

  // staging: 1024 uint4 per page for K and for V; 4 per thread (key e / 16, dims 8 (e % 16) .. +8)
  u32x4 kr[4], vr[4];
#define Q355_LOAD_PAGE(kb)                                                                     \
  {                                                                                            \
    const int pg_ = a.block_table[kb];                                                         \
    const u32x4* kp_ = (const u32x4*)(a.kcache + ((size_t)pg_ * a.nkv + kvh) * PAGE * HD);     \
    const u32x4* vp_ = (const u32x4*)(a.vcache + ((size_t)pg_ * a.nkv + kvh) * PAGE * HD);     \
    kr[0] = kp_[threadIdx.x];                                                                  \
    kr[1] = kp_[threadIdx.x + 256];                                                            \
    kr[2] = kp_[threadIdx.x + 512];                                                            \
    kr[3] = kp_[threadIdx.x + 768];                                                            \
    vr[0] = vp_[threadIdx.x];                                                                  \
    vr[1] = vp_[threadIdx.x + 256];                                                            \
    vr[2] = vp_[threadIdx.x + 512];                                                            \
    vr[3] = vp_[threadIdx.x + 768];                                                            \
  }

  float m = -INFINITY, l = 0.f;
  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

  Q355_LOAD_PAGE(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();                                       // previous page's LDS reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = threadIdx.x + 256 * i;
      const int key = e >> 4, d0 = (e & 15) * 8;
      *(u32x4*)&ks[key][d0] = kr[i];
      const u32x4 w = vr[i];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        *reinterpret_cast<unsigned short*>(&vt[d0 + u][key]) = (unsigned short)(w[u >> 1] >> (16 * (u & 1)));
    }
    __syncthreads();
    Q355_LOAD_PAGE(min(kb + 1, nkb - 1));                  // next page (clamped: unconditional), in flight now

    // S^T tiles: keys 16t + (4g + v), query li
    f4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const h8 kA = as_h8(*(const uint4*)&ks[16 * t + li][32 * c + 8 * lg]);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kA, qf[c], s[t], 0, 0, 0);
      }
    }
    // causal mask + running max (keys beyond the query's position, and queries past P, get -inf)
    float bm = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = kb * PAGE + 16 * t + 4 * lg + v;
        const float x = (key <= qpos && qi < a.P) ? s[t][v] * sl2 : -INFINITY;
        s[t][v] = x;
        bm = fmaxf(bm, x);
      }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(m, bm);
    const float ms = mn == -INFINITY ? 0.f : mn;           // fully masked so far: keep exp2 finite
    const float alpha = exp2f(m - ms);
    float rs = 0.f;
    _Float16 ph[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = exp2f(s[t][v] - ms);
        rs += p;
        ph[t][v] = (_Float16)p;
      }
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] *= alpha;
    // O^T += Vt P^T over two 32-key chunks
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      h8 pB;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        pB[v] = ph[2 * c][v];
        pB[4 + v] = ph[2 * c + 1][v];
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const _Float16* row = &vt[16 * dt + li][0];
        const uint2 lo = *(const uint2*)(row + 32 * c + 4 * lg);
        const uint2 hi = *(const uint2*)(row + 32 * c + 16 + 4 * lg);
        const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(vv), pB, acc[dt], 0, 0, 0);
      }
    }
  }
#undef Q355_LOAD_PAGE
  if (qi < a.P) {
    const float inv = 1.f / l;
    float* o = a.out + (size_t)qi * nq + hq * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *(float4*)(o + 16 * dt + 4 * lg) = make_float4(acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv,
                                                     acc[dt][3] * inv);
  }
}

}  // namespace q355
