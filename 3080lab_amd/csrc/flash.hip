// Causal GQA flash attention for prefill on fp16 MFMA (v_mfma_f32_16x16x32_f16), gfx950.
//
// Semantics of flash_prefill_v3 (lab/qwen_batched.py:1795-2037) and the torch reference of
// scripts/flash_bench.py:51-65: query i of the chunk (position pos0 + i) attends to keys 0..pos0 + i of
// its sequence; scores q.k * scale, softmax with running max (exp2 of scores pre-scaled by log2 e),
// fp16 P, fp32 accumulation; output o = sum p v / sum p in fp32.
//
// Per 64-key block (one KV page): K and V (key-major, rows padded) are staged in LDS once for all query heads
// of the KV head by two staging waves, a step ahead (double buffer). The head wave computes S^T = K Q^T
// (A = K rows from LDS, B = the wave's Q rows held in registers), so lane l holds scores of ONE query (l % 16)
// for keys 16t + 4(l/16) + v: the softmax statistics of a query live in the 4 lanes l % 16 + 16g and need only
// two cross-lane steps. The same registers, converted to fp16, are directly the B operand of O^T = Vt P^T when
// a 32-key chunk c is ordered as k-slot 8g + j -> key 32c + 4g + j (j < 4), 32c + 16 + 4g + j - 4 (j >= 4);
// the Vt operand is read in that order from the key-major V by two transposed LDS reads. O^T accumulators are
// again per query l % 16 (dims 16dt + 4g + v), so the running-max rescale is per lane.
// MFMA operand layouts (16x16x32): lane l holds A[row l%16][k 8(l/16)..+8], B[k 8(l/16)..+8][col l%16],
// C[row 4(l/16)+v][col l%16].
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int KP = 2;              // KV pages per step of the key loop
constexpr int FK_ROW = HD + 8;     // K row in LDS (halves), padded
// V row (one key) in LDS (halves): rows 8 banks apart, so the four rows of a transposed read use disjoint banks
constexpr int FV_ROW = HD + 16;

__device__ __forceinline__ h8 as_h8(uint4 v) { return *reinterpret_cast<h8*>(&v); }

// phase accounting hooks: empty here; an instrumented build defines them
#ifndef Q355_PF_PHASE
#define Q355_PF_PHASE_INIT()
#define Q355_PF_PHASE(k)
#define Q355_PF_PHASE_END()
#endif

// Scheduling of an unrolled run of N LDS operands (R reads each) feeding N MFMA groups (CBN MFMAs each):
// PF_DEPTH operands first, then one MFMA group per further operand, then the last groups (masks: 0x100 LDS
// read, 0x008 MFMA).
#ifndef PF_DEPTH
#define PF_DEPTH 8
#endif
#define Q355_PIPELINE(N, R)  /* R LDS reads per operand */                                \
  do {                                                                                         \
    __builtin_amdgcn_sched_group_barrier(0x100, (R) * PF_DEPTH, 0);                            \
    _Pragma("unroll") for (int i_ = 0; i_ < (N) - PF_DEPTH; ++i_) {                            \
      __builtin_amdgcn_sched_group_barrier(0x008, CBN, 0);                                     \
      __builtin_amdgcn_sched_group_barrier(0x100, (R), 0);                                     \
    }                                                                                          \
    __builtin_amdgcn_sched_group_barrier(0x008, CBN * PF_DEPTH, 0);                            \
  } while (0)

constexpr int CBN = PF_QB / 16;      // 16-query MFMA column blocks per wave

static_assert(CBN == 1, "one 16-query MFMA column block per query block");

// One key-loop step of a head wave over the staged pages kb, kb + 1: S^T = K Q^T, the online softmax (causal
// mask on diagonal steps; queries past P need none: each query column of S, P and O is independent and is
// never stored) and O^T += Vt P^T. Operand n of each product is read PF_DEPTH MFMAs ahead (Q355_PIPELINE).
__device__ __forceinline__ void pf_consume(const _Float16 (&ks)[KP * PAGE][FK_ROW], const _Float16 (&vs)[KP * PAGE][FV_ROW],
                                           const h8 (&qf)[4], int kb, int qpos, bool diag, float sl2, int li, int lg,
                                           float& m, float& l, f4 (&acc)[8]) {
  // S^T tiles: keys 16 t + (4 g + v), query li; operand n = (c, t), t fastest: 4 KP independent chains
  f4 s[4 * KP];
#pragma unroll
  for (int t = 0; t < 4 * KP; ++t) s[t] = f4{0.f, 0.f, 0.f, 0.f};
  {
    constexpr int NS = 16 * KP;
    h8 kA[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n)
      kA[n] = as_h8(*(const uint4*)&ks[16 * (n % (4 * KP)) + li][32 * (n / (4 * KP)) + 8 * lg]);
#pragma unroll
    for (int n = 0; n < NS; ++n)
      s[n % (4 * KP)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kA[n], qf[n / (4 * KP)], s[n % (4 * KP)], 0, 0, 0);
    Q355_PIPELINE(NS, 1);
  }
  h8 pB[2 * KP];
  if (diag) {
#pragma unroll
    for (int t = 0; t < 4 * KP; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (kb * PAGE + 16 * t + 4 * lg + v > qpos) s[t][v] = -INFINITY;
  }
  float bm = -INFINITY;                                  // raw-score max; scaled once below
#pragma unroll
  for (int t = 0; t < 4 * KP; ++t) bm = fmaxf(bm, fmaxf(fmaxf(s[t][0], s[t][1]), fmaxf(s[t][2], s[t][3])));
  bm = col4_max(bm);
  const float mn = fmaxf(m, bm * sl2);
  const float ms = mn == -INFINITY ? 0.f : mn;           // fully masked so far: keep exp2 finite
  const float alpha = __builtin_amdgcn_exp2f(m - ms);
  float rs = 0.f;
#pragma unroll
  for (int t = 0; t < 4 * KP; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float p = __builtin_amdgcn_exp2f(fmaf(s[t][v], sl2, -ms));
      rs += p;
      pB[t >> 1][4 * (t & 1) + v] = (_Float16)p;
    }
  rs = col4_sum(rs);
  l = l * alpha + rs;
  m = mn;
  if (__any(alpha != 1.f)) {                             // the running max moved for some query of the wave
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] *= alpha;
  }
  // O^T += Vt P^T over 2 KP 32-key chunks; operand n = (c, dt), dt fastest
  {
    constexpr int NV = 16 * KP;
    // A operand of chunk c, dim tile dt: keys 32 c + 4 lg + (0..3) and 32 c + 16 + 4 lg + (0..3) of dim 16 dt + li,
    // two transposed reads (ds_read_b64_tr_b16: lane j of a 16-lane group receives element j % 4 of the 4-value
    // segments named by lanes j / 4 + 4 k, k = 0..3; here lane x names key 4 lg + x / 4, dims 4 (x % 4) ..)
    h8 vA[NV];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const _Float16* seg = &vs[32 * (n / 8) + 4 * lg + (li >> 2)][16 * (n % 8) + 4 * (li & 3)];
      typedef short s4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s4* lds_s4;
      const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(seg));
      const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(seg + 16 * FV_ROW));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      vA[n] = as_h8(make_uint4(l2.x, l2.y, h2.x, h2.y));
    }
#pragma unroll
    for (int n = 0; n < NV; ++n)
      acc[n % 8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vA[n], pB[n / 8], acc[n % 8], 0, 0, 0);
    Q355_PIPELINE(NV, 2);
  }
}

// The normalized output of query qi, head hq: fp32, or Q8_1 for the O projection (the values the fp32 path
// stores, quantized as q355_quant_q8_1 does): block bk = dims 32 bk .. 32 bk + 31 lives in tiles dt = 2 bk,
// 2 bk + 1 of the 4 lanes li + 16 g.
__device__ __forceinline__ void pf_out(const PrefillAttnArgs& a, int qi, int hq, int lg, const f4 (&acc)[8], float l) {
  const int nq = a.nh * HD;
  const float inv = 1.f / l;
  if (a.oq) {
#pragma unroll
    for (int bk = 0; bk < 4; ++bk) {
      float x[2][4];
      float amax = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          x[h][v] = acc[2 * bk + h][v] * inv;
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
      if (qi < a.P) {
        int8_t* o = a.oq + (size_t)qi * nq + hq * HD;
        *(unsigned*)(o + 32 * bk + 4 * lg) = pk[0];
        *(unsigned*)(o + 32 * bk + 16 + 4 * lg) = pk[1];
        if (lg == 0)
          a.ods[((size_t)qi * nq + hq * HD) / 32 + bk] = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
      }
    }
  } else if (qi < a.P) {
    float* o = a.out + (size_t)qi * nq + hq * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *(float4*)(o + 16 * dt + 4 * lg) =
          make_float4(acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv);
  }
}

// Staging registers of one step (two pages) for the staging waves (thread st = 0 .. 64 PF_STAGERS - 1 of them):
// K and V each as 1024 16 B pieces per page (key e / 16, dims 8 (e % 16) ..), stored key-major (16-byte
// loads keep a wave's loads of a step within the 63 it can have in flight).
constexpr int PF_KPS = 1024 / (64 * PF_STAGERS);
struct PfStage {
  u32x4 kr[KP][PF_KPS];
  u32x4 vr[KP][PF_KPS];
};
__device__ __forceinline__ void pf_stage_load(PfStage& r, const PrefillAttnArgs& a, int kvh, int pg0, int pg1, int st) {
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const size_t off = ((size_t)(p ? pg1 : pg0) * a.nkv + kvh) * PAGE * HD;
    const u32x4* kp = (const u32x4*)(a.kcache + off);
    const u32x4* vp = (const u32x4*)(a.vcache + off);
#pragma unroll
    for (int i = 0; i < PF_KPS; ++i) r.kr[p][i] = kp[st + 64 * PF_STAGERS * i];
#pragma unroll
    for (int i = 0; i < PF_KPS; ++i) r.vr[p][i] = vp[st + 64 * PF_STAGERS * i];
  }
}
__device__ __forceinline__ void pf_stage_store(const PfStage& r, _Float16 (&ks)[KP * PAGE][FK_ROW],
                                               _Float16 (&vs)[KP * PAGE][FV_ROW], int st) {
#pragma unroll
  for (int p = 0; p < KP; ++p)
#pragma unroll
    for (int i = 0; i < PF_KPS; ++i) {
      const int e = st + 64 * PF_STAGERS * i;
      *(u32x4*)&ks[p * PAGE + (e >> 4)][(e & 15) * 8] = r.kr[p][i];
      *(u32x4*)&vs[p * PAGE + (e >> 4)][(e & 15) * 8] = r.vr[p][i];
    }
}
// the 16 queries of block qb for head hq (rows past P repeat the last; they are never stored)
__device__ __forceinline__ void pf_load_q(h8 (&qf)[4], const PrefillAttnArgs& a, int qb, int hq, int li, int lg) {
  const int qc = min(qb * PF_QB + li, a.P - 1);
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qf[c] = as_h8(*(const uint4*)(a.q + (size_t)qc * a.nh * HD + hq * HD + 32 * c + 8 * lg));
}

// Workgroup = one KV head x 16 queries x all their keys (the form without a workspace). Waves 0 .. G-1 are
// the head waves (wave w: query head kvh * G + w), so each staged K/V page serves all G heads of the group;
// waves G and G + 1 stage K and V into a double buffer: while the head waves compute step s from buffer
// s & 1, they write step s + 1 into the other buffer and load step s + 2 into registers, so one barrier per
// step separates the two roles and the head waves hold no staging registers. grid (ceil(P / 16), 1, nkv),
// the longest query blocks first; 64 (G + 2) threads.
// NT: the launch's thread bound (512 up to G = 6: two waves per SIMD, 256 VGPRs; 640 for G = 7, 8)
template <int NT>
__global__ void __launch_bounds__(NT) k_attn_prefill(const PrefillAttnArgs a) {
  __shared__ __align__(16) _Float16 ks[2][KP * PAGE][FK_ROW];
  __shared__ __align__(16) _Float16 vs[2][KP * PAGE][FV_ROW];
  __shared__ int pages[64];
  const int G = a.nh / a.nkv;
  const int qb = gridDim.x - 1 - blockIdx.x, kvh = blockIdx.z;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int nkb = pf_pages(a.pos0, qb, a.P);
  const float sl2 = a.scale * 1.4426950408889634f;       // scores in log2 units
  for (int i = threadIdx.x; i < nkb && i < 64; i += blockDim.x) pages[i] = a.block_table[i];
  __syncthreads();
  // page ids (a step's second page past the range repeats the last: masked on the diagonal step)
  auto pg = [&](int kb) { return kb < 64 ? pages[kb] : a.block_table[kb]; };
  if (wv >= G) {                                         // the staging waves' own loop, same barriers
    const int st = threadIdx.x - 64 * G;
    PfStage r;
    pf_stage_load(r, a, kvh, pg(0), pg(min(1, nkb - 1)), st);
    pf_stage_store(r, ks[0], vs[0], st);
    if (KP < nkb) pf_stage_load(r, a, kvh, pg(KP), pg(min(KP + 1, nkb - 1)), st);
    __syncthreads();
    for (int kb = 0, bf = 0; kb < nkb; kb += KP, bf ^= 1) {
      if (kb + KP < nkb) {                               // uniform
        pf_stage_store(r, ks[bf ^ 1], vs[bf ^ 1], st);
        if (kb + 2 * KP < nkb) pf_stage_load(r, a, kvh, pg(kb + 2 * KP), pg(min(kb + 2 * KP + 1, nkb - 1)), st);
      }
      __syncthreads();
    }
    return;
  }
  const int hq = kvh * G + wv;
  h8 qf[4];
  pf_load_q(qf, a, qb, hq, li, lg);
  float m = -INFINITY, l = 0.f;
  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  const int qpos = a.pos0 + qb * PF_QB + li;
  __syncthreads();
  Q355_PF_PHASE_INIT();
  for (int kb = 0, bf = 0; kb < nkb; kb += KP, bf ^= 1) {
    Q355_PF_PHASE(0);
    // causal mask only where the step reaches past the block's first query (uniform; this includes the step
    // with a repeated page past the range)
    const bool diag = (kb + KP) * PAGE - 1 > a.pos0 + qb * PF_QB;
    pf_consume(ks[bf], vs[bf], qf, kb, qpos, diag, sl2, li, lg, m, l, acc);
    Q355_PF_PHASE(5);
    __syncthreads();                                     // this buffer is free; the next one is staged
  }
  Q355_PF_PHASE_END();
  pf_out(a, qb * PF_QB + li, hq, lg, acc, l);
}

// The persistent form (with a workspace): gridDim.x workgroups of G head waves and PF_STAGERS staging waves,
// each walking its items -- (query block, KV head, key split of PF_SPLIT_PAGES pages) -- as one sequence of
// two-page steps, so the staging waves load across item boundaries and the causal rows are balanced over the
// CUs. Items are numbered split-major, query blocks longest first, then KV head; workgroup w takes item
// r W + w in even rounds r and r W + W - 1 - w in odd ones (W = gridDim.x), at most PF_MAX_ROUNDS.
// A split item writes its unnormalized O, m and l to the workspace with device-coherent stores (the splits
// may run on other XCDs) and goes on to the next item without waiting for them. After its last step each
// head wave waits once for its stores and counts all its split items at once, per (query block, KV head,
// head); the last to arrive merges every split of its head in split order (so the result does not depend on
// arrival order), writes the output and resets its counter.
template <int NT>
__global__ void __launch_bounds__(NT) k_attn_prefill_pers(const PrefillAttnArgs a) {
  __shared__ __align__(16) _Float16 ks[2][KP * PAGE][FK_ROW];
  __shared__ __align__(16) _Float16 vs[2][KP * PAGE][FV_ROW];
  __shared__ int4 items[PF_MAX_ROUNDS];                  // (qb, kvh, kb0 | nkb << 16, nsplit | split << 16)
  __shared__ int4 steps[PF_MAX_ROUNDS * PF_SPLIT_PAGES / KP];   // (item, kb, page kb, page kb + 1 in range)
  const int G = a.nh / a.nkv;
  const int nqb = (a.P + PF_QB - 1) / PF_QB;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const float sl2 = a.scale * 1.4426950408889634f;
  Q355_PF_PHASE_INIT();

  // this workgroup's items, computed by every wave (lane r = round r): the staging waves start on steps 0 and 1
  // and the head waves on their queries before the one barrier of the prologue; wave 0 writes the tables
  int4 it = make_int4(0, 0, 0, 0);
  int ns = 0;
  {
    const int W = gridDim.x, w = blockIdx.x, r = lane;
    int c = r * W + ((r & 1) ? W - 1 - w : w);
    if (c < a.n_items) {
      int sp = 0, q0 = pf_qmin(a.pos0, a.P, 0);
      while (c >= (nqb - q0) * a.nkv) {                  // the split this item belongs to
        c -= (nqb - q0) * a.nkv;
        q0 = pf_qmin(a.pos0, a.P, ++sp);
      }
      const int qb = nqb - 1 - c / a.nkv, kvh = c % a.nkv;
      const int L = pf_pages(a.pos0, qb, a.P);
      const int kb0 = sp * PF_SPLIT_PAGES, nkb = min(L, kb0 + PF_SPLIT_PAGES);
      it = make_int4(qb, kvh, kb0 | (nkb << 16), ((L - 1) / PF_SPLIT_PAGES + 1) | (sp << 16));
      ns = (nkb - kb0 + KP - 1) / KP;
    }
  }
  int incl = ns;                                         // inclusive prefix of the step counts
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  const int nst = __shfl(incl, 63), nit = __popcll(__ballot(ns > 0));
  auto item = [&](int r) {                               // item r's fields, from lane r
    return make_int4(__shfl(it.x, r), __shfl(it.y, r), __shfl(it.z, r), __shfl(it.w, r));
  };
  if (wv == 0) {
    // the steps (item, kb, page ids of kb and kb + 1, the second past the range a repeat: masked on the
    // diagonal step), all page-id loads of a lane in flight together
    items[lane] = it;
    const int kb0 = it.z & 0xffff, nkb = it.z >> 16;
    for (int k = 0; k < ns; ++k) {
      const int kb = kb0 + KP * k;
      steps[incl - ns + k] = make_int4(lane, kb, a.block_table[kb], a.block_table[min(kb + 1, nkb - 1)]);
    }
  }
  if (wv >= G) {                                         // staging waves: same barriers as the head waves
    const int st = threadIdx.x - 64 * G;
    PfStage r;
    // steps 0 and 1 from the items directly (step 1: item 0's second step, or item 1's first)
    const int4 i0 = item(0);
    const int kb00 = i0.z & 0xffff, nkb0 = i0.z >> 16;
    pf_stage_load(r, a, i0.y, a.block_table[kb00], a.block_table[min(kb00 + 1, nkb0 - 1)], st);
    pf_stage_store(r, ks[0], vs[0], st);
    if (nst > 1) {
      const bool same = kb00 + KP < nkb0;
      const int4 i1 = same ? i0 : item(1);
      const int kb = same ? kb00 + KP : (i1.z & 0xffff), nkb = i1.z >> 16;
      pf_stage_load(r, a, i1.y, a.block_table[kb], a.block_table[min(kb + 1, nkb - 1)], st);
    }
    __syncthreads();
    for (int g = 0; g < nst; ++g) {
      Q355_PF_PHASE(0);
      if (g + 1 < nst) {
        pf_stage_store(r, ks[(g + 1) & 1], vs[(g + 1) & 1], st);
        Q355_PF_PHASE(2);
        if (g + 2 < nst) pf_stage_load(r, a, items[steps[g + 2].x].y, steps[g + 2].z, steps[g + 2].w, st);
      }
      Q355_PF_PHASE(3);
      __syncthreads();
    }
    Q355_PF_PHASE_END();
    return;
  }

  h8 qf[4], qn[4];                                       // this item's queries and the next item's
  {
    const int4 i0 = item(0), i1 = item(1);
    pf_load_q(qf, a, i0.x, i0.y * G + wv, li, lg);
    if (nit > 1) pf_load_q(qn, a, i1.x, i1.y * G + wv, li, lg);
  }
  float m = -INFINITY, l = 0.f;
  f4 acc[8];
  __syncthreads();                                       // the tables and step 0's stage are ready
  Q355_PF_PHASE(3);
  for (int g = 0; g < nst; ++g) {
    Q355_PF_PHASE(0);
    const int4 st = steps[g];
    const int4 it = items[st.x];
    const int qb = it.x, kvh = it.y, kb0 = it.z & 0xffff, nkb = it.z >> 16;
    if (st.y == kb0) {                                   // the item's first step
      if (st.x > 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[c] = qn[c];
        if (st.x + 1 < nit) pf_load_q(qn, a, items[st.x + 1].x, items[st.x + 1].y * G + wv, li, lg);
      }
      m = -INFINITY;
      l = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const bool diag = (st.y + KP) * PAGE - 1 > a.pos0 + qb * PF_QB;
    pf_consume(ks[g & 1], vs[g & 1], qf, st.y, a.pos0 + qb * PF_QB + li, diag, sl2, li, lg, m, l, acc);
    Q355_PF_PHASE(5);
    if (st.y + KP >= nkb) {                              // the item's last step
      const int nsplit = it.w & 0xffff, sp = it.w >> 16;
      const int hq = kvh * G + wv;
      if (nsplit == 1) {
        pf_out(a, qb * PF_QB + li, hq, lg, acc, l);
      } else {
        // this (query block, KV head)'s partials: [max_splits][G][8][64] float4 and (m, l, -, -) [max_splits][G][16]
        const size_t row = (size_t)qb * a.nkv + kvh;
        const int per = a.max_splits * G;
        const Coh16 PO((const float4*)a.ws + row * per * 512, (unsigned)per * 512 * 16);
        const Coh16 PM((const float4*)a.ws + (size_t)nqb * a.nkv * per * 512 + row * per * 16, (unsigned)per * 16 * 16);
        const unsigned own = (unsigned)(sp * G + wv);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) PO.st16(((own * 512) + dt * 64 + lane) * 16, __builtin_bit_cast(int4, acc[dt]));
        if (lg == 0) PM.st16((own * 16 + li) * 16, __builtin_bit_cast(int4, make_float4(m, l, 0.f, 0.f)));
      }
    }
    Q355_PF_PHASE(1);
    __syncthreads();                                     // this buffer is free; the next one is staged
  }
  // arrivals of this wave's split items, all at once (lane r: item r) after one wait for its partial stores;
  // the last split of a head to arrive merges every split of it in split order and writes the output
  __builtin_amdgcn_s_waitcnt(0);                         // this wave's coherent stores have completed
  int* cnt0 = (int*)(a.ws + pf_ws_floats(nqb, a.nkv, G, a.max_splits) - (size_t)nqb * a.nkv * G);
  bool merge = false;
  if (lane < nit) {
    const int4 it = items[lane];
    const int nsplit = it.w & 0xffff;
    if (nsplit > 1) {
      int* cnt = cnt0 + ((size_t)it.x * a.nkv + it.y) * G + wv;
      merge = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
      if (merge) stc(cnt, 0);                            // every split has arrived: ready for the next call
    }
  }
  for (unsigned long long mb = __ballot(merge); mb; mb &= mb - 1) {
    const int4 it = items[__builtin_ctzll(mb)];
    const int qb = it.x, kvh = it.y, nsplit = it.w & 0xffff;
    const size_t row = (size_t)qb * a.nkv + kvh;
    const int per = a.max_splits * G;
    const Coh16 PO((const float4*)a.ws + row * per * 512, (unsigned)per * 512 * 16);
    const Coh16 PM((const float4*)a.ws + (size_t)nqb * a.nkv * per * 512 + row * per * 16, (unsigned)per * 16 * 16);
    // running-max merge in split order, two splits' loads in flight at a time
    float M = -INFINITY, lt = 0.f;
    f4 o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = f4{0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < nsplit; b0 += 2) {
      int4 v[2][8];
      float4 ml[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const unsigned sl = (unsigned)(min(b0 + u, nsplit - 1) * G + wv);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) v[u][dt] = PO.ld((sl * 512 + dt * 64 + lane) * 16);
        ml[u] = __builtin_bit_cast(float4, PM.ld((sl * 16 + li) * 16));
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (b0 + u >= nsplit) break;                     // uniform
        const float mn = fmaxf(M, ml[u].x);              // split 0 holds key 0: finite
        const float fo = __builtin_amdgcn_exp2f(M - mn), f = __builtin_amdgcn_exp2f(ml[u].x - mn);
        lt = lt * fo + f * ml[u].y;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = o[dt] * fo + f * __builtin_bit_cast(f4, v[u][dt]);
        M = mn;
      }
    }
    pf_out(a, qb * PF_QB + li, kvh * G + wv, lg, o, lt);
  }
  Q355_PF_PHASE(4);
  Q355_PF_PHASE_END();
}

}  // namespace q355
