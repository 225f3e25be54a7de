// Decode GQA attention over the paged fp16 KV cache, split-K over pages (flash-decoding), gfx950.
//
// Workgroup (chunk c, KV head g, token j) stages one 64-position K page and V page in LDS (32 KB,
// every lane issues 8 x 16 B loads up front), scores all NH/NKV query heads of the group against
// it (each K/V byte is read once per group, not once per query head), and writes the partial
// (o[128], running max m, sum l) per query head. The last workgroup of (j, g) to arrive (arrival
// counter, self-resetting, so graph replays need no re-initialisation) merges the partials in
// fixed chunk order and writes the O-projection input already quantized to Q8_1.
// Semantics follow ATTN2 / ATTN4 (split-K flash decoding and softmax with max subtraction).
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

constexpr int MAXG = 8;  // query heads per KV head supported (Qwen2.5-1.5B: 6)

__global__ void __launch_bounds__(256) k_attn_decode(const AttnArgs a) {
  __shared__ __align__(16) __half ks[PAGE][HD];
  __shared__ __align__(16) __half vs[PAGE][HD];
  __shared__ float qf[MAXG][HD];
  __shared__ float S[MAXG][PAGE];
  __shared__ float ml[MAXG][2];
  __shared__ int am_last;

  const int j = blockIdx.y;
  const int kvh = blockIdx.x / a.max_chunks, c = blockIdx.x % a.max_chunks;
  const int pos = a.pos[j];
  const int nctx = pos + 1, nch = (nctx + PAGE - 1) / PAGE;
  if (c >= nch) return;                       // whole workgroup leaves; it is not counted
  const int grp = a.nh / a.nkv;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nvalid = min(PAGE, nctx - c * PAGE);

  const int pg = a.block_table[(size_t)j * a.bt_stride + c];
  const uint4* kp = (const uint4*)(a.kcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  const uint4* vp = (const uint4*)(a.vcache + ((size_t)pg * a.nkv + kvh) * PAGE * HD);
  uint4 kr[4], vr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { kr[i] = kp[t + 256 * i]; vr[i] = vp[t + 256 * i]; }
  // queries of the group: grp * 128 halves
  const __half* qh = a.q + (size_t)j * a.nh * HD + (size_t)kvh * grp * HD;
  for (int e = t; e < grp * HD; e += 256) qf[e / HD][e % HD] = __half2float(qh[e]);
#pragma unroll
  for (int i = 0; i < 4; ++i) { ((uint4*)ks)[t + 256 * i] = kr[i]; ((uint4*)vs)[t + 256 * i] = vr[i]; }
  __syncthreads();

  // scores: thread (p = t / 4, quarter qq = t % 4) covers dims [32qq, 32qq + 32) of position p
  {
    const int p = t >> 2, qq = t & 3;
    float kf[32];
    const __half2* krow = (const __half2*)&ks[p][32 * qq];
#pragma unroll
    for (int i = 0; i < 16; ++i) { float2 f = __half22float2(krow[i]); kf[2 * i] = f.x; kf[2 * i + 1] = f.y; }
    for (int h = 0; h < grp; ++h) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) s = fmaf(qf[h][32 * qq + i], kf[i], s);
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      if (qq == 0) S[h][p] = p < nvalid ? s * a.scale : -INFINITY;
    }
  }
  __syncthreads();
  // softmax numerators per head: wave w handles heads w, w + 4
  for (int h = wv; h < grp; h += 4) {
    float s = S[h][lane];
    float m = wave_max(s);
    float e = lane < nvalid ? expf(s - m) : 0.f;
    float l = wave_sum(e);
    S[h][lane] = e;
    if (lane == 0) { ml[h][0] = m; ml[h][1] = l; }
  }
  __syncthreads();
  // P V: thread (dim pair d2 = lane, heads wv, wv + 4)
  float* part = a.part + (size_t)j * a.nh * a.max_chunks * (HD + 2);
  for (int h = wv; h < grp; h += 4) {
    float o0 = 0.f, o1 = 0.f;
    for (int p = 0; p < nvalid; ++p) {
      const float pr = S[h][p];
      const float2 v = __half22float2(((const __half2*)vs[p])[lane]);
      o0 = fmaf(pr, v.x, o0);
      o1 = fmaf(pr, v.y, o1);
    }
    float* P = part + ((size_t)(kvh * grp + h) * a.max_chunks + c) * (HD + 2);
    P[2 * lane] = o0;
    P[2 * lane + 1] = o1;
    if (lane == 0) { P[HD] = ml[h][0]; P[HD + 1] = ml[h][1]; }
  }
  __threadfence();
  __syncthreads();
  if (t == 0) am_last = atomicAdd(a.counter + (size_t)j * a.nkv + kvh, 1u) == (unsigned)(nch - 1);
  __syncthreads();
  if (!am_last) return;
  __threadfence();
  // merge: thread (d = t % 128) for heads h = t / 128, +2, +4 ... ; 32-lane groups = one Q8_1 block
  const int d = t & (HD - 1);
  for (int h = t >> 7; h < grp; h += 2) {
    const float* P0 = part + (size_t)(kvh * grp + h) * a.max_chunks * (HD + 2);
    float M = -INFINITY;
    for (int cc = 0; cc < nch; ++cc) M = fmaxf(M, __builtin_nontemporal_load(P0 + (size_t)cc * (HD + 2) + HD));
    float L = 0.f, O = 0.f;
    for (int cc = 0; cc < nch; ++cc) {
      const float* Pc = P0 + (size_t)cc * (HD + 2);
      const float w = expf(__builtin_nontemporal_load(Pc + HD) - M);
      L = fmaf(w, __builtin_nontemporal_load(Pc + HD + 1), L);
      O = fmaf(w, __builtin_nontemporal_load(Pc + d), O);
    }
    const float o = O / L;
    const int hq = kvh * grp + h;
    if (a.o32) a.o32[(size_t)j * a.nh * HD + hq * HD + d] = o;
    const int q = q8_1_lane32(o, a.ods + ((size_t)j * a.nh * HD + hq * HD + d) / 32, (d & 31) == 0);
    a.oq[(size_t)j * a.nh * HD + hq * HD + d] = (int8_t)q;
  }
  if (t == 0) a.counter[(size_t)j * a.nkv + kvh] = 0u;
}

}  // namespace q355
