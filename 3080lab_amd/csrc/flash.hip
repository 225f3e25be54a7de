// Causal GQA flash attention for prefill on fp16 MFMA (v_mfma_f32_16x16x32_f16), gfx950.
//
// Semantics of flash_prefill_v3 (lab/qwen_batched.py:1795-2037) and the torch reference of
// scripts/flash_bench.py:51-65: query i of the chunk (position pos0 + i) attends to keys 0..pos0 + i of
// its sequence; scores q.k * scale, softmax with running max (exp2 of scores pre-scaled by log2 e),
// fp16 P, fp32 accumulation; output o = sum p v / sum p in fp32.
//
// Per 64-key block (one KV page): K (row-padded) and V transposed (Vt[dim][key]) are staged in LDS once for
// all query heads of the KV head; the next page is loaded into registers while the current one is used.
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

constexpr int KP = 2;              // KV pages per step of the key loop
constexpr int FK_ROW = HD + 8;     // K row in LDS (halves), padded
constexpr int FV_ROW = KP * PAGE + 4;   // Vt row (one dim, KP pages of keys) in LDS (halves), padded

__device__ __forceinline__ h8 as_h8(uint4 v) { return *reinterpret_cast<h8*>(&v); }

// Scheduling of an unrolled run of N LDS operand reads feeding N MFMA groups (CBN MFMAs each): PF_DEPTH reads
// first, then one MFMA group per further read, then the last groups (masks: 0x100 LDS read, 0x008 MFMA).
// phase accounting hooks of the key loop: empty here; an instrumented build defines them
#ifndef Q355_PF_PHASE
#define Q355_PF_PHASE_INIT()
#define Q355_PF_PHASE(k)
#define Q355_PF_PHASE_END()
#endif

#ifndef PF_DEPTH
#define PF_DEPTH 8
#endif
#define Q355_PIPELINE(N)                                                                       \
  do {                                                                                         \
    __builtin_amdgcn_sched_group_barrier(0x100, PF_DEPTH, 0);                                  \
    _Pragma("unroll") for (int i_ = 0; i_ < (N) - PF_DEPTH; ++i_) {                            \
      __builtin_amdgcn_sched_group_barrier(0x008, CBN, 0);                                     \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                       \
    }                                                                                          \
    __builtin_amdgcn_sched_group_barrier(0x008, CBN * PF_DEPTH, 0);                            \
  } while (0)

constexpr int CBN = PF_QB / 16;      // 16-query MFMA column blocks per wave

// Workgroup = one KV head x 16 queries x one key split of up to 32 pages. Waves 0 .. G-1 are the head waves
// (wave w: query head kvh * G + w), so each staged K/V page serves all G heads of the group; waves G and
// G + 1 stage K and Vt into a double buffer: while the head waves compute step s from buffer s & 1, they write
// step s + 1 into the other buffer and load step s + 2 into registers, so one barrier per step separates
// the two roles and the head waves hold no staging registers. Wave tile: 16 queries (one MFMA column block).
// grid (ceil(P / 16), max splits, nkv), the longest query blocks first; 64 (G + 2) threads. With several
// splits, each writes its unnormalized O, m and l to the workspace; the last to arrive (counter per query
// block and KV head, reset by it) merges them and writes the output. Partials and counters use
// device-coherent accesses: the splits may run on different XCDs.
// NT: the launch's thread bound (512 up to G = 6: two waves per SIMD, 256 VGPRs; 640 for G = 7, 8)
template <int NT>
__global__ void __launch_bounds__(NT) k_attn_prefill(const PrefillAttnArgs a) {
  __shared__ __align__(16) _Float16 ks[2][KP * PAGE][FK_ROW];
  __shared__ __align__(16) _Float16 vt[2][HD][FV_ROW];
  const int G = a.nh / a.nkv;
  const int qb = gridDim.x - 1 - blockIdx.x, split = blockIdx.y, kvh = blockIdx.z;
  const int nsplit = a.ws ? pf_splits(a.pos0, qb, a.P) : 1;
  if (split >= nsplit) return;                           // uniform per workgroup
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const bool stager = wv >= G;
  const int hq = kvh * G + min(wv, G - 1);
  const int nq = a.nh * HD;

  int qi[CBN], qpos[CBN];
  h8 qf[CBN][4];
#pragma unroll
  for (int cb = 0; cb < CBN; ++cb) {
    qi[cb] = qb * PF_QB + 16 * cb + li;
    qpos[cb] = a.pos0 + qi[cb];
    const int qc = min(qi[cb], a.P - 1);
    if (!stager)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[cb][c] = as_h8(*(const uint4*)(a.q + (size_t)qc * nq + hq * HD + 32 * c + 8 * lg));
  }

  const int last_key = min(a.pos0 + qb * PF_QB + PF_QB - 1, a.pos0 + a.P - 1);
  const int kb0 = a.ws ? split * PF_SPLIT_PAGES : 0;
  const int nkb = a.ws ? min(last_key / PAGE + 1, kb0 + PF_SPLIT_PAGES) : last_key / PAGE + 1;
  const float sl2 = a.scale * 1.4426950408889634f;       // scores in log2 units

  // staging (the two staging waves, thread st = 0..127): K as 1024 16 B pieces per page (key e / 16, dims
  // 8 (e % 16) ..); V transposed: lane l of staging wave sw takes dims 2l, 2l + 1 of the 8-key groups sw,
  // sw + 2, ...: 8 dword loads per group, packed into two 16 B rows
  constexpr int KPS = 1024 / (64 * PF_STAGERS), VPS = 8 / PF_STAGERS;
  const int st = threadIdx.x - 64 * G, sw = wv - G;
  u32x4 kr[KP][KPS];
  unsigned vr[KP][VPS][8];
  // the page ids of this workgroup's key range, read once (each page's loads then wait on one latency)
  __shared__ int pages[64];
  for (int i = threadIdx.x; i < nkb - kb0 && i < 64; i += blockDim.x) pages[i] = a.block_table[kb0 + i];
  __syncthreads();
#define Q355_LOAD_PAGE(kb)                                                                     \
  _Pragma("unroll") for (int p_ = 0; p_ < KP; ++p_) {                                          \
    const int kbp_ = min((kb) + p_, nkb - 1);   /* past the range: a repeat, masked (diag step) */ \
    const int pg_ = kbp_ - kb0 < 64 ? pages[kbp_ - kb0] : a.block_table[kbp_];                 \
    const u32x4* kp_ = (const u32x4*)(a.kcache + ((size_t)pg_ * a.nkv + kvh) * PAGE * HD);     \
    const unsigned* vp_ = (const unsigned*)(a.vcache + ((size_t)pg_ * a.nkv + kvh) * PAGE * HD); \
    _Pragma("unroll") for (int i = 0; i < KPS; ++i) kr[p_][i] = kp_[st + 64 * PF_STAGERS * i]; \
    _Pragma("unroll") for (int i = 0; i < VPS; ++i) {                                          \
      const int kg = sw + PF_STAGERS * i;                                                      \
      _Pragma("unroll") for (int u = 0; u < 8; ++u) vr[p_][i][u] = vp_[(kg * 8 + u) * (HD / 2) + lane]; \
    }                                                                                          \
  }
#define Q355_STORE_PAGE(bf)                                                                    \
  _Pragma("unroll") for (int p_ = 0; p_ < KP; ++p_) {                                          \
    _Pragma("unroll") for (int i = 0; i < KPS; ++i) {                                          \
      const int e = st + 64 * PF_STAGERS * i;                                                  \
      *(u32x4*)&ks[bf][p_ * PAGE + (e >> 4)][(e & 15) * 8] = kr[p_][i];                        \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < VPS; ++i) {                                          \
      const int kg = sw + PF_STAGERS * i;                                                      \
      u32x4 lo, hi;                                                                            \
      _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                          \
        lo[j] = __builtin_amdgcn_perm(vr[p_][i][2 * j + 1], vr[p_][i][2 * j], 0x05040100u);    \
        hi[j] = __builtin_amdgcn_perm(vr[p_][i][2 * j + 1], vr[p_][i][2 * j], 0x07060302u);    \
      }                                                                                        \
      *(u32x4*)&vt[bf][2 * lane][p_ * PAGE + kg * 8] = lo;                                     \
      *(u32x4*)&vt[bf][2 * lane + 1][p_ * PAGE + kg * 8] = hi;                                 \
    }                                                                                          \
  }

  float m[CBN], l[CBN];
  f4 acc[CBN][8];
#pragma unroll
  for (int cb = 0; cb < CBN; ++cb) {
    m[cb] = -INFINITY;
    l[cb] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[cb][t] = f4{0.f, 0.f, 0.f, 0.f};
  }

  if (stager) {                                            // the staging waves' own loop, same barriers
    Q355_LOAD_PAGE(kb0);
    Q355_STORE_PAGE(0);
    if (kb0 + KP < nkb) Q355_LOAD_PAGE(kb0 + KP);
    __syncthreads();
    for (int kb = kb0, bf = 0; kb < nkb; kb += KP, bf ^= 1) {
      if (kb + KP < nkb) {                                 // uniform
        Q355_STORE_PAGE(bf ^ 1);
        if (kb + 2 * KP < nkb) Q355_LOAD_PAGE(kb + 2 * KP);
      }
      __syncthreads();
    }
    if (nsplit > 1) {                                      // the split merge's two barriers
      __syncthreads();
      __syncthreads();
    }
    return;
  }
  __syncthreads();
  Q355_PF_PHASE_INIT();
  for (int kb = kb0, bf = 0; kb < nkb; kb += KP, bf ^= 1) {
    Q355_PF_PHASE(0);
    // S^T tiles: keys 16t + (4g + v), query li of column block cb; each K operand feeds both blocks
    // operand n = (c, t), t fastest: 4 KP independent accumulator chains; the schedule keeps PF_DEPTH LDS
    // reads in flight ahead of the MFMAs (left to itself the compiler issues one or two)
    f4 s[CBN][4 * KP];
#pragma unroll
    for (int t = 0; t < 4 * KP; ++t)
#pragma unroll
      for (int cb = 0; cb < CBN; ++cb) s[cb][t] = f4{0.f, 0.f, 0.f, 0.f};
    {
      constexpr int NS = 16 * KP;
      h8 kA[NS];
#pragma unroll
      for (int n = 0; n < NS; ++n)
        kA[n] = as_h8(*(const uint4*)&ks[bf][16 * (n % (4 * KP)) + li][32 * (n / (4 * KP)) + 8 * lg]);
#pragma unroll
      for (int n = 0; n < NS; ++n)
#pragma unroll
        for (int cb = 0; cb < CBN; ++cb)
          s[cb][n % (4 * KP)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kA[n], qf[cb][n / (4 * KP)], s[cb][n % (4 * KP)], 0, 0, 0);
      Q355_PIPELINE(NS);
    }
    Q355_PF_PHASE(3);
    h8 pB[CBN][2 * KP];
    // causal mask only where the step reaches past the block's first query (uniform; this includes the step
    // with a repeated page past the range); queries past P need none: each query column of S, P and O is
    // independent and is never stored
    const bool diag = (kb + KP) * PAGE - 1 > a.pos0 + qb * PF_QB;
#pragma unroll
    for (int cb = 0; cb < CBN; ++cb) {
      if (diag) {
#pragma unroll
        for (int t = 0; t < 4 * KP; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (kb * PAGE + 16 * t + 4 * lg + v > qpos[cb]) s[cb][t][v] = -INFINITY;
      }
      float bm = -INFINITY;                                // raw-score max; scaled once below
#pragma unroll
      for (int t = 0; t < 4 * KP; ++t) bm = fmaxf(bm, fmaxf(fmaxf(s[cb][t][0], s[cb][t][1]), fmaxf(s[cb][t][2], s[cb][t][3])));
      bm = col4_max(bm);
      const float mn = fmaxf(m[cb], bm * sl2);
      const float ms = mn == -INFINITY ? 0.f : mn;         // fully masked so far: keep exp2 finite
      const float alpha = __builtin_amdgcn_exp2f(m[cb] - ms);
      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < 4 * KP; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[cb][t][v], sl2, -ms));
          rs += p;
          pB[cb][t >> 1][4 * (t & 1) + v] = (_Float16)p;
        }
      rs = col4_sum(rs);
      l[cb] = l[cb] * alpha + rs;
      m[cb] = mn;
      if (__any(alpha != 1.f)) {                           // the running max moved for some query of the wave
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[cb][t] *= alpha;
      }
    }
    // O^T += Vt P^T over 2 KP 32-key chunks; each Vt operand feeds every block
    Q355_PF_PHASE(4);
    {
      constexpr int NV = 16 * KP;                          // operand n = (c, dt), dt fastest
      h8 vA[NV];
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        const _Float16* row = &vt[bf][16 * (n % 8) + li][32 * (n / 8)];
        const uint2 lo = *(const uint2*)(row + 4 * lg);
        const uint2 hi = *(const uint2*)(row + 16 + 4 * lg);
        vA[n] = as_h8(make_uint4(lo.x, lo.y, hi.x, hi.y));
      }
#pragma unroll
      for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int cb = 0; cb < CBN; ++cb)
          acc[cb][n % 8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vA[n], pB[cb][n / 8], acc[cb][n % 8], 0, 0, 0);
      Q355_PIPELINE(NV);
    }
    Q355_PF_PHASE(5);
    __syncthreads();                                       // this buffer is free; the next one is staged
  }
  Q355_PF_PHASE_END();
#undef Q355_LOAD_PAGE
#undef Q355_STORE_PAGE
  if (nsplit > 1) {
    // partial -> workspace (same lane order on both sides), then arrival count
    const size_t slot = (((size_t)qb * a.nkv + kvh) * a.max_splits + split) * G + wv;
    float4* po = (float4*)a.ws + slot * (CBN * 8 * 64);
    float* pml = a.ws + (size_t)gridDim.x * a.nkv * a.max_splits * G * (CBN * 8 * 64 * 4) + slot * (CBN * 16 * 2);
#pragma unroll
    for (int cb = 0; cb < CBN; ++cb) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int v = 0; v < 4; ++v) stc((float*)&po[(cb * 8 + dt) * 64 + lane] + v, acc[cb][dt][v]);
      if (lg == 0) {
        stc(pml + (cb * 16 + li) * 2, m[cb]);
        stc(pml + (cb * 16 + li) * 2 + 1, l[cb]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);                         // this wave's coherent stores have completed
    __syncthreads();
    __shared__ int last;
    int* cnt = (int*)(a.ws + pf_ws_floats(gridDim.x, a.nkv, G, a.max_splits) - (size_t)gridDim.x * a.nkv) +
               qb * a.nkv + kvh;
    if (threadIdx.x == 0) {
      last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
      if (last) stc(cnt, 0);                             // every split has arrived: ready for the next call
    }
    __syncthreads();
    if (!last) return;
    // merge: rescale every split to the common max
    const size_t slot0 = (((size_t)qb * a.nkv + kvh) * a.max_splits) * G + wv;
    const float4* pa = (const float4*)a.ws + slot0 * (CBN * 8 * 64);   // read with coherent loads
    const float* pmla = a.ws + (size_t)gridDim.x * a.nkv * a.max_splits * G * (CBN * 8 * 64 * 4) + slot0 * (CBN * 16 * 2);
#pragma unroll
    for (int cb = 0; cb < CBN; ++cb) {
      float mt = m[cb];
      for (int s2 = 0; s2 < nsplit; ++s2)
        if (s2 != split) mt = fmaxf(mt, ldc(pmla + (size_t)s2 * G * (CBN * 32) + (cb * 16 + li) * 2));
      const float f0 = __builtin_amdgcn_exp2f(m[cb] - mt);
      l[cb] *= f0;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[cb][dt] *= f0;
      for (int s2 = 0; s2 < nsplit; ++s2) {
        if (s2 == split) continue;
        const float* ml = pmla + (size_t)s2 * G * (CBN * 32) + (cb * 16 + li) * 2;
        const float f = __builtin_amdgcn_exp2f(ldc(ml) - mt);
        l[cb] += f * ldc(ml + 1);
        const float4* src = pa + (size_t)s2 * G * (CBN * 8 * 64) + cb * 8 * 64 + lane;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[cb][dt][v] += f * ldc((const float*)&src[dt * 64] + v);
        }
      }
    }
  }
#pragma unroll
  for (int cb = 0; cb < CBN; ++cb) {
    const float inv = 1.f / l[cb];
    if (a.oq) {
      // Q8_1 of the output row (the values the fp32 path stores, quantized as q355_quant_q8_1 does): block
      // bk = dims 32 bk .. 32 bk + 31 lives in tiles dt = 2 bk, 2 bk + 1 of the 4 lanes li + 16 g
#pragma unroll
      for (int bk = 0; bk < 4; ++bk) {
        float x[2][4];
        float amax = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            x[h][v] = acc[cb][2 * bk + h][v] * inv;
            amax = fmaxf(amax, fabsf(x[h][v]));
          }
        amax = col4_max(amax);
        const float d32 = q8_scale(amax);
        int sq = 0;
        unsigned pk[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          pk[h] = 0;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int q = q8_code(x[h][v], d32);
            sq += q;
            pk[h] |= (unsigned)(q & 255) << (8 * v);
          }
        }
        sq = col4_isum(sq);
        if (qi[cb] < a.P) {
          int8_t* o = a.oq + (size_t)qi[cb] * nq + hq * HD;
          *(unsigned*)(o + 32 * bk + 4 * lg) = pk[0];
          *(unsigned*)(o + 32 * bk + 16 + 4 * lg) = pk[1];
          if (lg == 0)
            a.ods[((size_t)qi[cb] * nq + hq * HD) / 32 + bk] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
        }
      }
    } else if (qi[cb] < a.P) {
      float* o = a.out + (size_t)qi[cb] * nq + hq * HD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *(float4*)(o + 16 * dt + 4 * lg) = make_float4(acc[cb][dt][0] * inv, acc[cb][dt][1] * inv,
                                                       acc[cb][dt][2] * inv, acc[cb][dt][3] * inv);
    }
  }
}

}  // namespace q355
