// Persistent whole-step decode (batch 1) for gfx950: one launch per token, 256 workgroups (one per CU).
//
// Replaces the reference's decode megakernel (mega_source, lab/qwen_mega.py:43-361) and the 143-node
// graph of the same step (embed, 28 x (qkv, attention, O, gate_up, down), head, finish). The arithmetic
// is the batch-1 GEMV path's (f64 accumulation, int64 2^-48 fixed-point residual, single f64 -> fp16
// rounding of q/K/V), so the tokens follow the same oracle.
//
// Phases of one layer and their dependencies:
//   QKV   WG 8 + t, t < 128: tile t (16 rows) of the 2048 QKV rows; RMSNorm of h + Q8_1 + dots + bias +
//         RoPE; q and the new k/v rows -> device-coherent scratch; k/v also -> the paged cache (later tokens).
//         needs all of h (a full barrier after the previous DOWN).
//   ATTN  task (kv head g, page c, query head) on WG 136 + task; f64 partial (o, max, sum) per (head,
//         page). Waits for its 24 QKV producers (q of its head, k and v of its group).
//   O     WG w < 192: tile w % 96, heads 6 (w / 96) .. +5: merge their partials + Q8_1 + dots, add into h
//         (int64 atomics). Waits for every ATTN task.
//   GU    4-5 gate/up tiles per WG 8..255: RMSNorm of h + Q8_1 + dots + SwiGLU -> m (coherent scratch).
//         needs all of h (a full barrier after O).
//   DOWN  3 (tile, 35-block K slice) tasks per WG: Q8_1 of the m slice + dots, add into h. Waits only
//         for the GU workgroups that produced the slice.
// then the tied head (final RMSNorm, 9496 tiles over all WGs, argmax partials), a barrier, and WG 0
// picks the token (lowest index on ties) and advances pos.
//
// Every weight load of a phase is issued before the phase waits for its inputs, so HBM latency overlaps
// the synchronisation. Cross-workgroup data is written with device-scope (write-through) stores or
// atomics and read with device-scope loads; a workgroup publishes a phase by waiting for its own stores
// to be acknowledged and then storing its sequence number into its flag. No L2 writeback/invalidate is
// needed. Every wait is bounded (spin_limit wall-clock ticks): on expiry the error word is set and the
// kernel runs to completion with invalid results, so a launch always terminates.
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

// Optional timing hooks (defined by instrumented builds only; empty in the library).
#ifndef Q355_MEGA_MARK
#define Q355_MEGA_MARK(layer, k)
#endif

constexpr int MG_NWG = 256;          // workgroups (must all be resident: one per CU)
constexpr int MG_NTH = 256;          // threads per workgroup
constexpr int MG_REP = 32;           // replicas of the barrier release word
constexpr int MG_FS = 16;            // unsigneds between flags (64 B)
constexpr int MG_H = 1536, MG_NH = 12, MG_NKV = 2, MG_FFN = 8960, MG_NQKV = 2048;
constexpr int MG_AHPT = 1;                          // query heads per attention task
constexpr int MG_ATPG = 6 / MG_AHPT;                // attention tasks per (kv group, page)
constexpr int MG_GU_TILES = 2 * MG_FFN / 16;        // 1120
constexpr int MG_DOWN_SLICES = 8, MG_DOWN_SB = MG_FFN / 32 / MG_DOWN_SLICES;   // 35 blocks per slice

struct MegaLayer {
  const uint8_t* qkv_qs; const __half* qkv_d; const float* qkv_b; const float* ln1;
  const uint8_t* o_qs; const __half* o_d; const float* ln2;
  const uint8_t* gu_qs; const __half* gu_d;
  const uint8_t* down_qs; const __half* down_d;
  __half* kc; __half* vc;
};

// Workspace layout (bytes), zeroed once by the caller; the sync words must persist across launches.
struct MegaWs {
  unsigned* flags;   // [MG_NWG * MG_FS]
  unsigned* go;      // [MG_REP * MG_FS]
  unsigned* ctl;     // [0] epoch base, [16] error word
  float* q;          // [NH * HD]
  __half* kvnew;     // [2][NKV * HD] the new token's k and v rows (fp16, as the cache holds them)
  double* part;      // [NH][max_chunks][HD + 2]
  float* m;          // [FFN]
  float* amax;       // [MG_NWG]
  int* aidx;         // [MG_NWG]
  long long* accD;   // [2][H] down-projection sums of layer i in slot i % 2 (int64 atomics); folded into the
                     // residual by the O phase of layer i + 1 (or at the end of the launch) and cleared there
};

struct MegaArgs {
  const MegaLayer* layers;
  int L;
  const uint8_t* emb_qs; const __half* emb_d; const float* norm; int V;
  const float* rope_cos; const float* rope_sin;
  const int* block_table; int max_chunks;
  double eps, scale;
  int* tok; int* pos; long long* h; float* logits;
  char* ws; long long spin_limit;
};

__host__ __device__ inline size_t mega_ws_bytes(int max_chunks, int L) {
  return (size_t)MG_NWG * MG_FS * 4 + (size_t)MG_REP * MG_FS * 4 + 256 + (size_t)2 * MG_H * 8 +
         (size_t)MG_NH * max_chunks * (HD + 2) * 8 + (size_t)MG_NH * HD * 4 + (size_t)2 * MG_NKV * HD * 4 +
         (size_t)MG_FFN * 4 + (size_t)MG_NWG * 8;
}

// every offset is a multiple of 8 (the f64 / int64 regions first)
__device__ __forceinline__ MegaWs mega_ws(char* p, int max_chunks, int L) {
  MegaWs w;
  w.flags = (unsigned*)p; p += (size_t)MG_NWG * MG_FS * 4;
  w.go = (unsigned*)p; p += (size_t)MG_REP * MG_FS * 4;
  w.ctl = (unsigned*)p; p += 256;
  w.accD = (long long*)p; p += (size_t)2 * MG_H * 8;
  w.part = (double*)p; p += (size_t)MG_NH * max_chunks * (HD + 2) * 8;
  w.q = (float*)p; p += (size_t)MG_NH * HD * 4;
  w.kvnew = (__half*)p; p += (size_t)2 * MG_NKV * HD * 4;
  w.m = (float*)p; p += (size_t)MG_FFN * 4;
  w.amax = (float*)p; p += (size_t)MG_NWG * 4;
  w.aidx = (int*)p;
  return w;
}

// device-scope (cross-workgroup coherent) loads and stores

__device__ __forceinline__ bool seq_reached(unsigned v, unsigned seq) { return (int)(v - seq) >= 0; }

// ---------------------------------------------------------------------------------------------
// Synchronisation.
struct MgSync {
  unsigned* flags; unsigned* go; unsigned* err; long long limit;

  // this workgroup's device-scope stores/atomics are acknowledged, then its flag = seq
  __device__ __forceinline__ void publish(unsigned seq) const {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) stc(flags + blockIdx.x * MG_FS, seq);
  }
  __device__ __forceinline__ bool failed() const { return ldc(err) != 0u; }
  __device__ __forceinline__ void fail() const { stc(err, 1u); }

  // wave 0 polls the flags of workgroups id(0..n-1) until all reach seq; then the workgroup proceeds. (Keeping
  // several rounds of polls in flight, staggered, measured slower: a flag takes ~1 us to be seen either way.)
  template <typename F>
  __device__ __forceinline__ void wait(int n, F id, unsigned seq) const {
    if (threadIdx.x < 64) {
      const long long t0 = wall_clock64();
      while (true) {
        const unsigned e = ldc(err);                     // in flight with the flags: one round trip per poll
        bool ok = true;
        for (int i = threadIdx.x; i < n; i += 64) ok &= seq_reached(ldc(flags + id(i) * MG_FS), seq);
        if (__all(ok)) break;
        if (e != 0u || wall_clock64() - t0 > limit) { if (threadIdx.x == 0) fail(); break; }
      }
    }
    __syncthreads();
  }

  // full barrier, in two halves so that weight loads can be issued in between: arrive() publishes; finish()
  // has workgroups 0..7 each gather the flags of the 32 workgroups w = x (mod 8) (the ones the dispatcher
  // places on XCD x) and release word x; every workgroup then polls the 8 release words. (A single gatherer
  // polling 256 flags measured 2.6 us per barrier, this form 1.8 us.)
  __device__ __forceinline__ void arrive(unsigned seq) const { publish(seq); }
  __device__ __forceinline__ void finish(unsigned seq) const {
    const int lane = threadIdx.x & 63;
    if (blockIdx.x < 8 && threadIdx.x < 64) {
      const long long t0 = wall_clock64();
      while (true) {
        const unsigned e = ldc(err);
        bool ok = true;
        for (int i = (int)blockIdx.x + 8 * lane; i < MG_NWG; i += 512) ok &= seq_reached(ldc(flags + i * MG_FS), seq);
        if (__all(ok)) break;
        if (e != 0u || wall_clock64() - t0 > limit) { if (lane == 0) fail(); break; }
      }
      if (lane == 0) stc(go + blockIdx.x * MG_FS, seq);
    }
    if (threadIdx.x < 64) {
      const long long t0 = wall_clock64();
      while (true) {
        const unsigned e = ldc(err);
        const bool ok = lane >= 8 || seq_reached(ldc(go + lane * MG_FS), seq);
        if (__all(ok)) break;
        if (e != 0u || wall_clock64() - t0 > limit) { if (lane == 0) fail(); break; }
      }
    }
    __syncthreads();
  }
  __device__ __forceinline__ void barrier(unsigned seq) const {
    arrive(seq);
    finish(seq);
  }
};

// ---------------------------------------------------------------------------------------------
// GEMV pieces. Lane (k-lane kl = wave * 4 + lane / 16, row r = lane % 16) takes blocks b0 + kl + 16 i of
// each of up to NT tiles; tiles past `nt` and blocks past b1 are loaded clamped with their scale zeroed.
template <int NT, int KPL>
struct MgW {
  uint4 w[NT][KPL];
  unsigned dh[NT][KPL];
};

template <int NT, int KPL>
__device__ __forceinline__ void mg_wload(MgW<NT, KPL>& W, const uint8_t* qs8, const __half* d, int nb,
                                         const int (&tile)[NT], const int (&b0)[NT], const int (&b1)[NT]) {
  const uint4* __restrict__ qs = (const uint4*)qs8;
  const unsigned short* __restrict__ dd = (const unsigned short*)d;
  const int lane = threadIdx.x & 63, kl = (threadIdx.x >> 6) * 4 + (lane >> 4), r = lane & 15;
#pragma unroll
  for (int i = 0; i < KPL; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int b = min(b0[t] + kl + 16 * i, b1[t] - 1);
      const size_t idx = ((size_t)tile[t] * nb + b) * 16 + r;
      W.w[t][i] = ld_stream16(qs + idx);
      W.dh[t][i] = ld_stream2(dd + idx);
    }
  __asm__ __volatile__("" ::: "memory");
#pragma unroll
  for (int i = 0; i < KPL; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) W.dh[t][i] = (b0[t] + kl + 16 * i < b1[t]) ? W.dh[t][i] : 0u;
}

// LDS activation operand over absolute K blocks: xq bytes, d (float), sum q (int)
struct MgX {
  int8_t* q;
  float* d;
  int* s;
};

__device__ __forceinline__ void mg_stage8(const MgX& x, int g, const float (&v)[8]) {
  float df;
  int sq;
  const uint2 pk = q8_1_x8(v, df, sq);
  *(uint2*)(x.q + 8 * g) = pk;
  if ((g & 3) == 0) {
    x.d[g >> 2] = df;
    x.s[g >> 2] = sq;
  }
}

// dots of the NT tiles, then the row values (f64) into rv[NT][16] (LDS) via part (LDS)
template <int NT, int KPL>
__device__ __forceinline__ void mg_dots(const MgW<NT, KPL>& W, const MgX& x, const int (&b0)[NT], const int (&b1)[NT],
                                        double (*part)[NT][16], double (*rv)[16]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, kl = wv * 4 + (lane >> 4), r = lane & 15;
  double acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.0;
#pragma unroll
  for (int i = 0; i < KPL; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int b = min(b0[t] + kl + 16 * i, b1[t] - 1);
      const int4* xp = (const int4*)(x.q + (size_t)b * 32);
      const int4 xa = xp[0], xb = xp[1];
      const int xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
      const int dot = q4_block_dot(W.w[t][i], xv);
      const double sc = (double)__half2float(__ushort_as_half((unsigned short)W.dh[t][i])) * (double)x.d[b];
      acc[t] = fma(sc, (double)(dot - 8 * x.s[b]), acc[t]);
    }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    double v = acc[t];
    v = xsum32_d(xsum16_d(v));
    if (lane < 16) part[wv][t][r] = v;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < NT * 16; e += MG_NTH) {
    const int t = e >> 4, rr = e & 15;
    rv[t][rr] = ((part[0][t][rr] + part[1][t][rr]) + part[2][t][rr]) + part[3][t][rr];
  }
  __syncthreads();
}

// RMSNorm of h (1536 values, from the coherent residual or computed by `get`) * w -> Q8_1 into x.
template <typename G>
__device__ __forceinline__ void mg_rms_stage(G get, const float* __restrict__ w, double eps, const MgX& x,
                                             double* red) {
  const int g = threadIdx.x;                  // 8 values per thread, 192 threads active
  const bool act = g < MG_H / 8;
  double hv[8];
  get.load8(act ? g : 0, hv);
  double ss = 0.0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    hv[u] = act ? hv[u] : 0.0;
    ss = fma(hv[u], hv[u], ss);
  }
  float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
  if (act) {
    w0 = ((const float4*)w)[2 * g];
    w1 = ((const float4*)w)[2 * g + 1];
  }
  ss = wave_sum_d(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const double rs = 1.0 / sqrt((((red[0] + red[1]) + red[2]) + red[3]) / (double)MG_H + eps);
  const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  float v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = (float)(hv[u] * rs * (double)wv[u]);
  if (g < 256) {            // every lane takes part in the quad reductions; only active ones store
    float df;
    int sq;
    const uint2 pk = q8_1_x8(v, df, sq);
    if (act) {
      *(uint2*)(x.q + 8 * g) = pk;
      if ((g & 3) == 0) { x.d[g >> 2] = df; x.s[g >> 2] = sq; }
    }
  }
  __syncthreads();
}

// h value i of the current token: from the embedding row (layer 0) or the coherent residual stream
struct HFromEmbed {
  const uint8_t* qs; const __half* d; int tok; int nb;
  __device__ __forceinline__ double operator()(int i) const {
    const int b = i >> 5, e = i & 31;
    const size_t tb = ((size_t)(tok >> 4) * nb + b) * 16 + (tok & 15);
    const uint8_t byte = qs[tb * 16 + (e & 15)];
    const int q = (e < 16 ? (byte & 15) : (byte >> 4)) - 8;
    const double v = (double)__half2float(d[tb]) * (double)q;
    return from_fix(to_fix(v));
  }
  __device__ __forceinline__ void load8(int g, double (&hv)[8]) const {
#pragma unroll
    for (int u = 0; u < 8; ++u) hv[u] = (*this)(8 * g + u);
  }
};
// residual entering layer i > 0: h (with the O sums of layer i - 1 folded in) + the down sums of layer i - 1
struct HSum2 {
  const long long *h, *acc;
  __device__ __forceinline__ long long fix(int i) const { return ldc(h + i) + ldc(acc + i); }
  __device__ __forceinline__ double operator()(int i) const { return from_fix(fix(i)); }
  // values 8 g .. 8 g + 7 with 16-byte device-scope loads (all issued before the first use)
  __device__ __forceinline__ void load8(int g, double (&hv)[8]) const {
    const Coh16 H(h, MG_H * 8), A(acc, MG_H * 8);
    int4 x[4], y[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) { x[u] = H.ld(64 * g + 16 * u); y[u] = A.ld(64 * g + 16 * u); }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long x0 = ((long long)(unsigned)x[u].y << 32) | (unsigned)x[u].x, x1 = ((long long)(unsigned)x[u].w << 32) | (unsigned)x[u].z;
      const long long y0 = ((long long)(unsigned)y[u].y << 32) | (unsigned)y[u].x, y1 = ((long long)(unsigned)y[u].w << 32) | (unsigned)y[u].z;
      hv[2 * u] = from_fix(x0 + y0);
      hv[2 * u + 1] = from_fix(x1 + y1);
    }
  }
};
// residual after the O projection of layer i: h
struct HOne {
  const long long* h;
  __device__ __forceinline__ double operator()(int i) const { return from_fix(ldc(h + i)); }
  __device__ __forceinline__ void load8(int g, double (&hv)[8]) const {
    const Coh16 H(h, MG_H * 8);
    int4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = H.ld(64 * g + 16 * u);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      hv[2 * u] = from_fix(((long long)(unsigned)x[u].y << 32) | (unsigned)x[u].x);
      hv[2 * u + 1] = from_fix(((long long)(unsigned)x[u].w << 32) | (unsigned)x[u].z);
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Attention task: kv group g, page c, query heads 6g + hq .. + MG_AHPT - 1 (one head per task: the f64
// score and P.V chains of one wave are latency-bound, so fewer heads per task shorten the phase). Wave w takes positions
// 16w .. 16w + 15 of the page: lane (p = lane / 4, quarter dq = lane % 4) scores position 16w + p over
// dims 32dq .. 32dq + 31 (f64, exact fp16 products), lanes of a position sum their quarters; the page
// maximum is exchanged through LDS so every wave's e^(s - M) shares M, and lane l accumulates dims 2l, 2l+1
// of P.V over the wave's 16 positions. The 4 waves' sums are added in fixed order into one partial
// (o[128], M, l) per (head, page). K/V come straight from the cache into registers; the new token's row
// comes from the coherent scratch.
struct MgAttnRegs {
  u32x4 k4[4];       // this lane's quarter of its position's K row
  unsigned v2[16];   // dims 2 lane, 2 lane + 1 of the wave's 16 V rows
};

// the task's K/V page rows from the cache (positions before this token: written by earlier launches), issued
// before the task waits for this token's q / k / v
__device__ __forceinline__ void mg_attn_load(MgAttnRegs& R, const MegaArgs& a, const MegaLayer& Ly, int g, int c) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int p = lane >> 2, dq = lane & 3;
  const int pg = a.block_table[c];
  const int row = 16 * wv + p;
  const __half* kbase = Ly.kc + ((size_t)pg * MG_NKV + g) * PAGE * HD;
  const __half* vbase = Ly.vc + ((size_t)pg * MG_NKV + g) * PAGE * HD;
#pragma unroll
  for (int i = 0; i < 4; ++i) R.k4[i] = ((const u32x4*)(kbase + (size_t)row * HD + 32 * dq))[i];
#pragma unroll
  for (int r = 0; r < 16; ++r) R.v2[r] = ((const unsigned*)(vbase + (size_t)(16 * wv + r) * HD))[lane];
}

__device__ __forceinline__ void mg_attn_task(const MegaArgs& a, const MegaLayer& Ly, const MegaWs& ws, int g, int c,
                                             int hq, int pos, char* lds, MgAttnRegs& R) {
  constexpr int NQ = MG_AHPT;
  double* qd = (double*)lds;                     // [NQ][HD] queries (f64)
  double* red_m = qd + NQ * HD;                  // [NQ][4]
  double* red_l = red_m + 4 * NQ;                // [NQ][4]
  double* red_o = red_l + 4 * NQ;                // [4][NQ][HD]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int p = lane >> 2, dq = lane & 3;
  const int row = 16 * wv + p, gp = c * PAGE + row;
  const bool valid = gp <= pos;
  u32x4 (&k4)[4] = R.k4;
  unsigned (&v2)[16] = R.v2;
  Q355_MEGA_MARK(31, 1);
  for (int e = threadIdx.x; e < NQ * HD; e += MG_NTH)
    qd[e] = (double)ldc(ws.q + (6 * g + hq) * HD + e);
  // the new token's row (written in this launch) from the coherent scratch
  const int inew = pos - c * PAGE;
  if (inew >= 16 * wv && inew < 16 * wv + 16) {
    const Coh16 KVN(ws.kvnew, 2 * MG_NKV * HD * 2);
    if (row == inew) {
#pragma unroll
      for (int i = 0; i < 4; ++i) k4[i] = __builtin_bit_cast(u32x4, KVN.ld((g * HD + 32 * dq + 8 * i) * 2));
    }
    const unsigned nv = KVN.ld4((MG_NKV * HD + g * HD + 2 * lane) * 2);
#pragma unroll
    for (int r = 0; r < 16; ++r) v2[r] = (16 * wv + r == inew) ? nv : v2[r];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) v2[r] = (c * PAGE + 16 * wv + r <= pos) ? v2[r] : 0u;   // rows past the context
  __syncthreads();
  Q355_MEGA_MARK(31, 2);

  double ev[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const double* qh = qd + h * HD + 32 * dq;
    double sp[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const __half2* k2 = (const __half2*)&k4[i];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 kf = __half22float2(k2[u]);
        sp[u] = fma(qh[8 * i + 2 * u], (double)kf.x, sp[u]);
        sp[u] = fma(qh[8 * i + 2 * u + 1], (double)kf.y, sp[u]);
      }
    }
    double sc = (sp[0] + sp[1]) + (sp[2] + sp[3]);
    sc += dpp_d<DPP_XOR1>(sc);                          // the 4 quarters of a position (one quad)
    sc += dpp_d<DPP_XOR2>(sc);
    sc = valid ? sc * a.scale : -INFINITY;
    const double mw = wave_max_d(sc);                   // each position appears 4 times: harmless for max
    if (lane == 0) red_m[h * 4 + wv] = mw;
    ev[h] = sc;
    Q355_MEGA_MARK(31, 8 + h);
  }
  __syncthreads();
  Q355_MEGA_MARK(31, 3);
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const double M = fmax(fmax(red_m[h * 4], red_m[h * 4 + 1]), fmax(red_m[h * 4 + 2], red_m[h * 4 + 3]));
    const double e = valid ? exp(ev[h] - M) : 0.0;
    const double lw = wave_sum_d(dq == 0 ? e : 0.0);    // one copy of each position
    const int2 ei = *reinterpret_cast<const int2*>(&e);
    double o0 = 0.0, o1 = 0.0, o2 = 0.0, o3 = 0.0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      int2 bi;
      bi.x = __builtin_amdgcn_readlane(ei.x, 4 * r);
      bi.y = __builtin_amdgcn_readlane(ei.y, 4 * r);
      const double er = *reinterpret_cast<const double*>(&bi);
      const float2 vf = __half22float2(*reinterpret_cast<const __half2*>(&v2[r]));
      if (r & 1) { o2 = fma(er, (double)vf.x, o2); o3 = fma(er, (double)vf.y, o3); }
      else { o0 = fma(er, (double)vf.x, o0); o1 = fma(er, (double)vf.y, o1); }
    }
    red_o[(wv * NQ + h) * HD + 2 * lane] = o0 + o2;
    red_o[(wv * NQ + h) * HD + 2 * lane + 1] = o1 + o3;
    if (lane == 0) red_l[h * 4 + wv] = lw;
  }
  __syncthreads();
  Q355_MEGA_MARK(31, 4);
  for (int e = threadIdx.x; e < NQ * HD; e += MG_NTH) {
    const int h = e / HD, d = e % HD;
    const double o = ((red_o[(0 * NQ + h) * HD + d] + red_o[(1 * NQ + h) * HD + d]) + red_o[(2 * NQ + h) * HD + d]) +
                     red_o[(3 * NQ + h) * HD + d];
    double* P = ws.part + ((size_t)(6 * g + hq + h) * a.max_chunks + c) * (HD + 2);
    stc(P + d, o);
    if (d == 0) {
      const double M = fmax(fmax(red_m[h * 4], red_m[h * 4 + 1]), fmax(red_m[h * 4 + 2], red_m[h * 4 + 3]));
      const double l = ((red_l[h * 4] + red_l[h * 4 + 1]) + red_l[h * 4 + 2]) + red_l[h * 4 + 3];
      stc(P + HD, M);
      stc(P + HD + 1, l);
    }
  }
  Q355_MEGA_MARK(31, 5);
  __syncthreads();                                       // LDS reused by the next task
}

// merge of one head's page partials (one wave, coherent loads), as attn_merge_head
__device__ __forceinline__ void mg_merge_head(const double* P, int nch, double* out) {
  const int lane = threadIdx.x & 63;
  const Coh16 PC(P, nch * (HD + 2) * 8);
  const double* pc = P + (size_t)min(lane, nch - 1) * (HD + 2);
  const double mc = ldc(pc + HD), lc = ldc(pc + HD + 1);
  const double M = wave_max_d(lane < nch ? mc : -INFINITY);
  const double w = lane < nch ? exp(mc - M) : 0.0;
  const double L = wave_sum_d(w * (lane < nch ? lc : 0.0));
  const int2 wi = *reinterpret_cast<const int2*>(&w);
  double o0 = 0.0, o1 = 0.0;
  for (int c0 = 0; c0 < nch; c0 += 8) {
    double v0[8], v1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {                     // dims 2 lane, 2 lane + 1: one 16-byte load (rows are
      const int4 t = PC.ld(((min(c0 + u, nch - 1) * (HD + 2)) + 2 * lane) * 8);   // 1040 B apart)
      v0[u] = __builtin_bit_cast(double, make_int2(t.x, t.y));
      v1[u] = __builtin_bit_cast(double, make_int2(t.z, t.w));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int2 bi;
      bi.x = __builtin_amdgcn_readlane(wi.x, c0 + u);
      bi.y = __builtin_amdgcn_readlane(wi.y, c0 + u);
      const double wc = *reinterpret_cast<const double*>(&bi);
      o0 = fma(wc, v0[u], o0);
      o1 = fma(wc, v1[u], o1);
    }
  }
  out[2 * lane] = o0 / L;
  out[2 * lane + 1] = o1 / L;
}

// merge of the 6 heads of one kv group when they have at most 8 page partials, every load issued at once (one
// memory round trip): thread t < 48 takes (head t / 8, chunk t % 8) and forms w_c = e^(m_c - M) and L (the
// max and the pairwise sum over its 8 lanes, chunks past nch as zero: the same tree as mg_merge_head's 64-lane
// sum) into LDS; then thread t < 192 takes head t / 32, dims 4 (t % 32) .. + 3: o = sequential fmas in chunk
// order, o / L -- mg_merge_head's arithmetic.
__device__ __forceinline__ void mg_merge6_short(const double* P0, int max_chunks, int nch, double (*ob)[HD],
                                                double (*wsh)[9]) {
  const int h = threadIdx.x >> 5, dq = threadIdx.x & 31;
  int4 ml, va[8], vb[8];
  const Coh16 PC(P0, 6 * max_chunks * (HD + 2) * 8);     // the 6 heads' partials, one uniform base
  if (threadIdx.x < 48) {                                // (m, l) first: the weights start while the values arrive
    const unsigned hc = (unsigned)(threadIdx.x >> 3) * max_chunks + min((int)threadIdx.x & 7, nch - 1);
    ml = PC.ld((hc * (HD + 2) + HD) * 8);
  }
  if (threadIdx.x < 192) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const unsigned c = ((unsigned)h * max_chunks + min(u, nch - 1)) * (HD + 2);
      va[u] = PC.ld((c + 4 * dq) * 8);
      vb[u] = PC.ld((c + 4 * dq + 2) * 8);
    }
  }
  __asm__ __volatile__("" ::: "memory");                 // the value loads stay issued here
  if (threadIdx.x < 48) {
    const int hh = threadIdx.x >> 3, c = threadIdx.x & 7;
    const double m = c < nch ? __builtin_bit_cast(double, make_int2(ml.x, ml.y)) : -INFINITY;
    double M = fmax(m, dpp_d<DPP_XOR1>(m));              // max and sum over the 8 lanes of a head
    M = fmax(M, dpp_d<DPP_XOR2>(M));
    M = fmax(M, dpp_d<DPP_HALF_MIRROR>(M));
    const double w = c < nch ? exp(m - M) : 0.0;
    double t = w * (c < nch ? __builtin_bit_cast(double, make_int2(ml.z, ml.w)) : 0.0);
    t += dpp_d<DPP_XOR1>(t);
    t += dpp_d<DPP_XOR2>(t);
    t += dpp_d<DPP_HALF_MIRROR>(t);
    wsh[hh][c] = w;
    if (c == 0) wsh[hh][8] = t;
  }
  Q355_MEGA_MARK(32, 1);
  __syncthreads();
  Q355_MEGA_MARK(32, 2);
  if (threadIdx.x < 192) {
    double o[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const double w = wsh[h][u];
      o[0] = fma(w, __builtin_bit_cast(double, make_int2(va[u].x, va[u].y)), o[0]);
      o[1] = fma(w, __builtin_bit_cast(double, make_int2(va[u].z, va[u].w)), o[1]);
      o[2] = fma(w, __builtin_bit_cast(double, make_int2(vb[u].x, vb[u].y)), o[2]);
      o[3] = fma(w, __builtin_bit_cast(double, make_int2(vb[u].z, vb[u].w)), o[3]);
    }
    const double L = wsh[h][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) ob[h][4 * dq + i] = o[i] / L;
  }
}

// ---------------------------------------------------------------------------------------------
// which workgroup runs which task
// Workgroups 0..7 gather the barrier flags; their gather loops would wait for any weight loads in flight (the
// vector memory counter is in order), so they take no QKV or gate/up tiles: QKV tile t runs on workgroup
// MG_GATH + t, the gate/up tiles spread over workgroups MG_GATH..255 (at most 5 each either way), attention
// task i on workgroup MG_GATH + 128 + i.
constexpr int MG_GATH = 8;
constexpr int MG_QKV_WG0 = MG_GATH, MG_ATT_WG0 = MG_GATH + MG_NQKV / 16;
__device__ __forceinline__ int gu_tile0(int w) {
  return w < MG_GATH ? 0 : (MG_GU_TILES * (w - MG_GATH)) / (MG_NWG - MG_GATH);
}
__device__ __forceinline__ int gu_owner(int t) {      // the workgroup whose tile range holds gate/up tile t
  int w = MG_GATH + (t * (MG_NWG - MG_GATH)) / MG_GU_TILES;
  while (w + 1 < MG_NWG && gu_tile0(w + 1) <= t) ++w;
  while (gu_tile0(w) > t) --w;
  return w;
}
__device__ __forceinline__ int attn_wg(int idx) { return (MG_ATT_WG0 + idx) % MG_NWG; }

// head chunk ck of this workgroup's tile range [t0, t1): tiles t0 + 8 ck .. (clamped to t1 - 1)
__device__ __forceinline__ void mg_head_load(MgW<8, 3>& W, const MegaArgs& a, int t0, int t1, int ck) {
  int tl[8];
  const int b0[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int b1[8] = {MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32};
#pragma unroll
  for (int t = 0; t < 8; ++t) tl[t] = min(t0 + 8 * ck + t, t1 - 1);
  mg_wload(W, a.emb_qs, a.emb_d, MG_H / 32, tl, b0, b1);
}

__device__ __forceinline__ void mg_head_chunk(const MgW<8, 3>& W, const MegaArgs& a, const MgX& x, const int (&b0)[8],
                                              const int (&b1)[8], double* part_s, double (*rv)[16], int t0, int t1,
                                              int ck, float& best, int& bidx) {
  mg_dots(W, x, b0, b1, reinterpret_cast<double(*)[8][16]>(part_s), rv);
  const int tb = t0 + 8 * ck, nt = min(8, t1 - tb);
  if (threadIdx.x < 64) {
    for (int rr = threadIdx.x; rr < nt * 16; rr += 64) {      // rows in increasing order per lane
      const float v = (float)rv[rr >> 4][rr & 15];
      const int row = tb * 16 + rr;
      a.logits[row] = v;
      if (v > best) { best = v; bidx = row; }
    }
  }
}

__global__ void __launch_bounds__(MG_NTH) k_mega_decode(const MegaArgs a) {
  extern __shared__ __align__(16) char lds[];
  __shared__ double part_s[4 * 8 * 16];
  __shared__ double rv[8][16];
  __shared__ double red[4];
  __shared__ double ob[6][HD];
  const MegaWs ws = mega_ws(a.ws, a.max_chunks, a.L);
  const MgSync sy{ws.flags, ws.go, ws.ctl + 16, a.spin_limit};
  const unsigned base = ldc(ws.ctl);
  unsigned seq = base;
  const int w = blockIdx.x;
  const int tok = *a.tok, pos = *a.pos;
  if (pos < 0 || pos >= a.max_chunks * PAGE || tok < 0 || tok >= a.V) {   // uniform: every workgroup leaves
    if (w == 0 && threadIdx.x == 0) sy.fail();
    return;
  }
  const int nch = pos / PAGE + 1;
  // attention slots: slot = hq * P8 + (page pc = g * nch + c), P8 = the page count rounded up to 8, so the tasks
  // that stage one K/V page run on workgroups 136 + slot of one XCD (x mod 8) and share its L2
  const int P8 = (MG_NKV * nch + 7) & ~7;
  const int n_slot = MG_ATPG * P8;
  const int n_attn_wg = n_slot < MG_NWG ? n_slot : MG_NWG;
  MgX x;
  x.q = (int8_t*)lds;                                  // K blocks of the widest operand (down: 280)
  x.d = (float*)(lds + MG_FFN);
  x.s = (int*)(lds + MG_FFN + (MG_FFN / 32) * 4);
  const HFromEmbed emb{a.emb_qs, a.emb_d, tok, MG_H / 32};

  // weights of the next QKV / gate-up phase are loaded between a barrier's arrive and finish
  MgW<1, 3> Wq;
  const int qt = w - MG_QKV_WG0;                       // QKV tile of this workgroup (valid for 0..127)
  const bool is_qkv = qt >= 0 && qt < MG_NQKV / 16;
  const int qkv_b0[1] = {0}, qkv_b1[1] = {MG_H / 32}, qkv_tl[1] = {is_qkv ? qt : 0};
  if (is_qkv) mg_wload(Wq, a.layers[0].qkv_qs, a.layers[0].qkv_d, MG_H / 32, qkv_tl, qkv_b0, qkv_b1);
  // O weights (workgroups w < 192: tile w % 96, K slice w / 96), loaded well before the O phase: at the start
  // of the layer on the gathering workgroups, after the QKV flag, or before the attention task's K/V
  MgW<1, 2> Wo;
  const int otl[1] = {w % 96}, ob0[1] = {24 * (w / 96)}, ob1[1] = {24 * (w / 96) + 24};

  // the residual stream lives in a.h (int64 fixed point): layer 0's O phase starts it from the embedding row
  // (written here by the owners of its 96 tiles, before their first flag), O sums are added into it, and the
  // down sums of layer i collect in accD slot i % 2 until layer i + 1's O phase folds them in
  long long* const hres = a.h;
  if (w < MG_H / 16 && threadIdx.x < 16) stc(hres + w * 16 + threadIdx.x, to_fix(emb(w * 16 + threadIdx.x)));

  for (int layer = 0; layer < a.L; ++layer) {
    const MegaLayer Ly = a.layers[layer];
    long long* const accPrev = ws.accD + (size_t)((layer + 1) & 1) * MG_H;   // down sums of layer - 1
    long long* const accCur = ws.accD + (size_t)(layer & 1) * MG_H;
    const HSum2 prev{hres, accPrev};
    // ---- QKV ----
    const unsigned s_qkv = ++seq;
    if (w < MG_QKV_WG0) mg_wload(Wo, Ly.o_qs, Ly.o_d, MG_H / 32, otl, ob0, ob1);
    if (is_qkv) {
      // epilogue operands (bias pair, RoPE angle, page) loaded before the normalisation
      const int r = threadIdx.x & 15, row = qt * 16 + r;
      const float bias = Ly.qkv_b[row], bias2 = Ly.qkv_b[row ^ 1];
      const int e2 = row % HD, ci = e2 >> 1;
      const float rc = a.rope_cos[(size_t)pos * (HD / 2) + ci], rs = a.rope_sin[(size_t)pos * (HD / 2) + ci];
      const int pg = a.block_table[pos / PAGE];
      if (layer == 0) mg_rms_stage(emb, Ly.ln1, a.eps, x, red);
      else mg_rms_stage(prev, Ly.ln1, a.eps, x, red);
      Q355_MEGA_MARK(layer, 9);
      mg_dots(Wq, x, qkv_b0, qkv_b1, reinterpret_cast<double(*)[1][16]>(part_s), rv);
      Q355_MEGA_MARK(layer, 10);
      if (threadIdx.x < 16) {
        const Coh16 KVN(ws.kvnew, 2 * MG_NKV * HD * 2);
        const double v = rv[0][r] + (double)bias;
        const int nq = MG_NH * HD, nk = MG_NKV * HD;
        if (row < nq + nk) {
          const double v2 = rv[0][r ^ 1] + (double)bias2;
          const int hi = e2 & 1;
          const double c = rc, sn = rs;
          const double lo_v = hi ? v2 : v, hi_v = hi ? v : v2;
          const double out = hi ? (hi_v * c + lo_v * sn) : (lo_v * c - hi_v * sn);
          const int dim = ci + (HD / 2) * hi;
          const __half hv = half_rn(out);
          if (row < nq) {
            stc(ws.q + (row / HD) * HD + dim, __half2float(hv));
          } else {
            const int kvh = (row - nq) / HD;
            Ly.kc[(((size_t)pg * MG_NKV + kvh) * PAGE + pos % PAGE) * HD + dim] = hv;
            KVN.st2((kvh * HD + dim) * 2, __half_as_ushort(hv));
          }
        } else {
          const int rvv = row - nq - nk, kvh = rvv / HD, dim = rvv % HD;
          const __half hv = half_rn(v);
          Ly.vc[(((size_t)pg * MG_NKV + kvh) * PAGE + pos % PAGE) * HD + dim] = hv;
          KVN.st2((MG_NKV * HD + kvh * HD + dim) * 2, __half_as_ushort(hv));
        }
      }
    }
    Q355_MEGA_MARK(layer, 0);
    sy.publish(s_qkv);
    if (is_qkv) mg_wload(Wo, Ly.o_qs, Ly.o_d, MG_H / 32, otl, ob0, ob1);   // (QKV workgroups 8..135 are O ones)

    // ---- attention: task idx on workgroup MG_ATT_WG0 + idx; its K/V page is loaded before it waits for its
    // q, k and v producers ----
    const unsigned s_attn = ++seq;
    for (int idx = (w - MG_ATT_WG0 + MG_NWG) % MG_NWG; idx < n_slot; idx += MG_NWG) {
      if (w < 192 && idx < MG_NWG - MG_ATT_WG0) mg_wload(Wo, Ly.o_qs, Ly.o_d, MG_H / 32, otl, ob0, ob1);
      const int pc = idx % P8, hq = (idx / P8) * MG_AHPT;
      if (pc >= MG_NKV * nch) continue;              // padding slot (uniform per workgroup)
      const int g = pc / nch, c = pc % nch;
      MgAttnRegs AR;
      mg_attn_load(AR, a, Ly, g, c);
      Q355_MEGA_MARK(31, 7);
      // its 24 producers: the 8 q tiles of head 6 g + hq and the 8 k and 8 v tiles of group g
      const int hq0 = (6 * g + hq) * (HD / 16), kt0 = MG_NH * (HD / 16) + g * (HD / 16);
      sy.wait(3 * (HD / 16), [hq0, kt0](int i) {
        return MG_QKV_WG0 + (i < 8 ? hq0 + i : (i < 16 ? kt0 + i - 8 : kt0 + MG_NKV * (HD / 16) + i - 16));
      }, s_qkv);
      Q355_MEGA_MARK(31, 0);
      mg_attn_task(a, Ly, ws, g, c, hq, pos, lds, AR);
    }
    if (w >= MG_ATT_WG0 && w < 192 && w - MG_ATT_WG0 >= n_slot)   // O workgroups without an attention slot
      mg_wload(Wo, Ly.o_qs, Ly.o_d, MG_H / 32, otl, ob0, ob1);
    Q355_MEGA_MARK(layer, 1);
    sy.publish(s_attn);

    // ---- O projection (+ merge) into the residual; slice-0 workgroups fold in the previous layer's down sums ----
    const unsigned s_o = ++seq;
    if (w < 192) {
      const int tile = otl[0], sl = w / 96;
      const MgW<1, 2>& W = Wo;
      const int(&b0)[1] = ob0;
      const int(&b1)[1] = ob1;
      // every attention task (not only this slice's): once all are done, every QKV workgroup is done (each
      // produced some task's q, k or v), so nobody reads this layer's QKV-phase residual any more
      sy.wait(n_attn_wg, [](int i) { return attn_wg(i); }, s_attn);
      Q355_MEGA_MARK(layer, 2);
      if (nch <= 8) {
        mg_merge6_short(ws.part + (size_t)(6 * sl) * a.max_chunks * (HD + 2), a.max_chunks, nch, ob,
                        reinterpret_cast<double(*)[9]>(part_s));
      } else {
        const int wv = threadIdx.x >> 6;
        for (int hh = wv; hh < 6; hh += 4)
          mg_merge_head(ws.part + (size_t)(6 * sl + hh) * a.max_chunks * (HD + 2), nch, ob[hh]);
      }
      Q355_MEGA_MARK(layer, 15);
      __syncthreads();
      if (threadIdx.x < 96) {                            // 768 values, 8 per thread, quads whole
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = (float)ob[0][8 * threadIdx.x + u];
        mg_stage8(x, 24 * sl * 4 + threadIdx.x, v);
      }
      __syncthreads();
      mg_dots(W, x, b0, b1, reinterpret_cast<double(*)[1][16]>(part_s), rv);
      if (threadIdx.x < 16) {
        const int row = tile * 16 + threadIdx.x;
        long long add = to_fix(rv[0][threadIdx.x]);
        if (sl == 0 && layer > 0) {
          add += ldc(accPrev + row);
          stc(accPrev + row, 0LL);
        }
        atomicAdd((unsigned long long*)(hres + row), (unsigned long long)add);
      }
    }
    Q355_MEGA_MARK(layer, 3);
    sy.arrive(s_o);
    const int gt0 = gu_tile0(w), gnt = gu_tile0(w + 1) - gt0;
    MgW<5, 3> Wg;
    int gtl[5], gb0[5], gb1[5];
#pragma unroll
    for (int t = 0; t < 5; ++t) { gtl[t] = gt0 + min(t, max(gnt - 1, 0)); gb0[t] = 0; gb1[t] = MG_H / 32; }
    if (gnt > 0) mg_wload(Wg, Ly.gu_qs, Ly.gu_d, MG_H / 32, gtl, gb0, gb1);
    sy.finish(s_o);
    Q355_MEGA_MARK(layer, 4);

    // ---- gate/up + SwiGLU ----
    const unsigned s_gu = ++seq;
    if (gnt > 0) {                                       // (the gathering workgroups have no tiles)
      const int t0 = gt0, nt = gnt;
      mg_rms_stage(HOne{hres}, Ly.ln2, a.eps, x, red);
      Q355_MEGA_MARK(layer, 11);
      mg_dots(Wg, x, gb0, gb1, reinterpret_cast<double(*)[5][16]>(part_s), rv);
      Q355_MEGA_MARK(layer, 12);
      for (int e = threadIdx.x; e < nt * 8; e += MG_NTH) {
        const int t = e >> 3, k = e & 7;
        const double gg = rv[t][2 * k], uu = rv[t][2 * k + 1];
        stc(ws.m + (t0 + t) * 8 + k, (float)(gg / (1.0 + exp(-gg)) * uu));
      }
    }
    Q355_MEGA_MARK(layer, 5);
#ifdef Q355_MEGA_PROBE
    __builtin_amdgcn_s_waitcnt(0);
    Q355_MEGA_MARK(33, 0);
#endif
    sy.publish(s_gu);

    // ---- down: into this layer's accD slot ----
    const unsigned s_down = ++seq;
    {
      MgW<3, 3> W;
      int tl[3], b0[3], b1[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const int task = w + MG_NWG * k;
        tl[k] = task % 96;
        b0[k] = (task / 96) * MG_DOWN_SB;
        b1[k] = b0[k] + MG_DOWN_SB;
      }
      mg_wload(W, Ly.down_qs, Ly.down_d, MG_FFN / 32, tl, b0, b1);
      // the m values of the three slices come from gate/up tiles 4 b0 .. 4 b1 - 1 (8 m values per tile): one
      // wait over the producers of all three (consecutive owners per slice)
      int lo[3], n[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        lo[k] = gu_owner(4 * b0[k]);
        n[k] = gu_owner(4 * b1[k] - 1) - lo[k] + 1;
      }
      sy.wait(n[0] + n[1] + n[2], [&](int i) { return i < n[0] ? lo[0] + i : (i < n[0] + n[1] ? lo[1] + i - n[0] : lo[2] + i - n[0] - n[1]); },
              s_gu);
      Q355_MEGA_MARK(layer, 6);
      const Coh16 M(ws.m, MG_FFN * 4);
      for (int task = threadIdx.x; task < 3 * MG_DOWN_SB * 4; task += MG_NTH) {
        const int k = task / (MG_DOWN_SB * 4);
        const int g = ((w + MG_NWG * k) / 96) * MG_DOWN_SB * 4 + task % (MG_DOWN_SB * 4);
        const int4 m0 = M.ld(32 * g), m1 = M.ld(32 * g + 16);
        const float v[8] = {__int_as_float(m0.x), __int_as_float(m0.y), __int_as_float(m0.z), __int_as_float(m0.w),
                            __int_as_float(m1.x), __int_as_float(m1.y), __int_as_float(m1.z), __int_as_float(m1.w)};
        mg_stage8(x, g, v);
      }
      __syncthreads();
      Q355_MEGA_MARK(layer, 13);
      mg_dots(W, x, b0, b1, reinterpret_cast<double(*)[3][16]>(part_s), rv);
      Q355_MEGA_MARK(layer, 14);
      if (threadIdx.x < 48) {
        const int k = threadIdx.x >> 4, r = threadIdx.x & 15;
        const int tile = (w + MG_NWG * k) % 96;
        atomicAdd((unsigned long long*)(accCur + tile * 16 + r), (unsigned long long)to_fix(rv[k][r]));
      }
    }
    Q355_MEGA_MARK(layer, 7);
    sy.arrive(s_down);
    if (is_qkv && layer + 1 < a.L)
      mg_wload(Wq, a.layers[layer + 1].qkv_qs, a.layers[layer + 1].qkv_d, MG_H / 32, qkv_tl, qkv_b0, qkv_b1);
    sy.finish(s_down);
    Q355_MEGA_MARK(layer, 8);
  }
  Q355_MEGA_MARK(a.L, 0);

  long long* const accLast = ws.accD + (size_t)((a.L - 1) & 1) * MG_H;
  const HSum2 fin{hres, accLast};
  if (!a.logits) {
    // no head in this launch (the caller runs its own, e.g. a Q6_K output matrix): after the last barrier nobody
    // reads the residual any more; workgroup 0 folds in the last down sums, clears their slot and moves the
    // sequence base on. tok and pos are left to the caller's head and finish.
    if (w == 0) {
      for (int i = threadIdx.x; i < MG_H; i += MG_NTH) {
        a.h[i] = fin.fix(i);
        stc(accLast + i, 0LL);
      }
      if (threadIdx.x == 0) stc(ws.ctl, base + 4096u);
    }
    return;
  }

  // ---- tied head: final RMSNorm, logits, argmax partial per workgroup (8-tile chunks, double-buffered) ----
  {
    const int ntiles = a.V / 16;
    const int t0 = (int)(((long long)ntiles * w) / MG_NWG), t1 = (int)(((long long)ntiles * (w + 1)) / MG_NWG);
    const int nck = (t1 - t0 + 7) / 8;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    MgW<8, 3> WA, WB;
    const int hb0[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int hb1[8] = {MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32, MG_H / 32};
    mg_head_load(WA, a, t0, t1, 0);
    mg_rms_stage(fin, a.norm, a.eps, x, red);
    for (int k = 0; k < nck; k += 2) {
      mg_head_load(WB, a, t0, t1, min(k + 1, nck - 1));     // clamped: unconditional
      mg_head_chunk(WA, a, x, hb0, hb1, part_s, rv, t0, t1, k, best, bidx);
      mg_head_load(WA, a, t0, t1, min(k + 2, nck - 1));
      if (k + 1 < nck) mg_head_chunk(WB, a, x, hb0, hb1, part_s, rv, t0, t1, k + 1, best, bidx);
    }
    if (threadIdx.x < 64) {
      wave_argmax(best, bidx);
      if (threadIdx.x == 0) { stc(ws.amax + w, best); stc(ws.aidx + w, bidx); }
    }
  }
  Q355_MEGA_MARK(a.L, 1);
  const unsigned s_head = ++seq;
  sy.publish(s_head);
  if (w == 0) {
    sy.wait(MG_NWG, [](int i) { return i; }, s_head);
    // the final residual (for the caller): fold in the last layer's down sums and clear their slot
    for (int i = threadIdx.x; i < MG_H; i += MG_NTH) {
      a.h[i] = fin.fix(i);
      stc(accLast + i, 0LL);
    }
    if (threadIdx.x < 64) {
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      for (int i = threadIdx.x; i < MG_NWG; i += 64) {
        const float v = ldc(ws.amax + i);
        const int id = ldc(ws.aidx + i);
        if (v > best || (v == best && id < bidx)) { best = v; bidx = id; }
      }
      wave_argmax(best, bidx);
      if (threadIdx.x == 0) {
        *a.tok = bidx;
        *a.pos = pos + 1;
        stc(ws.ctl, base + 4096u);                      // sequence numbers of the next launch start above
      }
    }
  }
}

}  // namespace q355
