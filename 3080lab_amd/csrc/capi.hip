// C ABI of libqwen355.so: argument validation on the host, launch geometry, template dispatch.
#include <cstdio>
#include <cstring>
#include <cstdarg>
#include <mutex>

#include "../../include/qwen355.h"
#include "common.h"
#include "q355_kernels.h"

namespace q355 {
__global__ void k_quant_q8_1(const float*, int8_t*, half2*, long);
__global__ void k_rmsnorm_q8_1(const float*, const float*, int8_t*, half2*, int, float);
__global__ void k_embed_q4_0(const uint8_t*, const __half*, int, int, const int*, long long*);
__global__ void k_finish(const float*, const int*, int, int*, int*);
__global__ void k_blockdots(const uint8_t*, int, int, const int8_t*, int, int*);
template <int G>
__global__ void k_attn_decode(const AttnArgs);
__global__ void k_attn_merge(const AttnArgs);
__global__ void k_attn_merge_split(const AttnArgs);
constexpr int ATTN_KW = 64;   // keys per wave of k_attn_decode_mfma (32 measured slower: 12.9 vs 12.1 us at B = 8)
__global__ void k_rmsnorm_fix_q8_1(const long long*, const float*, int8_t*, half2*, int, double);
__global__ void k_qkv_finish(GemvArgs, long long*);
}  // namespace q355

using namespace q355;

static thread_local char g_err[512] = "";

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

static int launched(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return Q355_OK;
}

#define REQUIRE(cond, ...) do { if (!(cond)) return fail(Q355_EINVAL, __VA_ARGS__); } while (0)

extern "C" const char* q355_last_error(void) { return g_err; }
extern "C" const char* q355_version(void) { return "qwen355 0.1 gfx950"; }

// ------------------------------------------------------------------------------------------------
// GEMV dispatch over (T, NT, NW, KPL, prologue, epilogue); grid = (N/16/NT tiles, KS K-slices).
template <int PRO, int EPI, int NT, int NW, int KPL, int WF = WF_Q4_0>
static int launch_gemv(const GemvArgs& a, int KS, hipStream_t s) {
  const int tiles = a.N / 16, nb = a.K / 32;
  if (tiles % NT) return fail(Q355_EINVAL, "gemv: N/16=%d not a multiple of %d tiles per workgroup", tiles, NT);
  const int per = (nb + KS - 1) / KS;
  if (per > 4 * NW * KPL) return fail(Q355_EINVAL, "gemv: K=%d slice of %d blocks exceeds %d", a.K, per, 4 * NW * KPL);
  const dim3 grid(tiles / NT, KS);
  size_t lds = (size_t)a.T * a.K + (size_t)a.T * nb * 8;
  if (PRO == PRO_ATTN) lds += 8 + (size_t)a.nh * HD * 8;  // merged heads of one token; 8: f64 alignment
  switch (a.T) {
    case 1: hipLaunchKernelGGL((k_gemv<1, NT, NW, KPL, PRO, EPI, WF>), grid, dim3(NW * 64), lds, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<2, NT, NW, KPL, PRO, EPI, WF>), grid, dim3(NW * 64), lds, s, a); break;
    case 3: hipLaunchKernelGGL((k_gemv<3, NT, NW, KPL, PRO, EPI, WF>), grid, dim3(NW * 64), lds, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemv<4, NT, NW, KPL, PRO, EPI, WF>), grid, dim3(NW * 64), lds, s, a); break;
    default: return fail(Q355_EINVAL, "gemv: T=%d outside 1..4", a.T);
  }
  return launched("gemv");
}

// Generic shapes without K split: K <= 1536 -> 4 waves x 3 blocks per lane; K <= 9216 -> 8 waves x 9.
template <int PRO, int EPI>
static int launch_gemv_generic(const GemvArgs& a, hipStream_t s) {
  const int tiles = a.N / 16;
  const bool nt4 = tiles % 4 == 0 && tiles / 4 >= 512;
  if (a.K <= 1536) {
    return nt4 ? launch_gemv<PRO, EPI, 4, 4, 3>(a, 1, s) : launch_gemv<PRO, EPI, 1, 4, 3>(a, 1, s);
  }
  return nt4 ? launch_gemv<PRO, EPI, 4, 8, 9>(a, 1, s) : launch_gemv<PRO, EPI, 1, 8, 9>(a, 1, s);
}

static int check_mat(const char* what, const void* qs, const void* d, int N, int K) {
  REQUIRE(qs && d, "%s: null weight pointer", what);
  REQUIRE(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", what, N);
  REQUIRE(K > 0 && K % 32 == 0 && K <= 9216, "%s: K=%d must be a multiple of 32 and <= 9216", what, K);
  return Q355_OK;
}

extern "C" int q355_quant_q8_1(const float* x, int8_t* xq, void* xds, int T, int K, void* stream) {
  REQUIRE(x && xq && xds, "quant_q8_1: null pointer");
  REQUIRE(T > 0 && K > 0 && K % 32 == 0, "quant_q8_1: T=%d K=%d (K %% 32 == 0)", T, K);
  long nblk = (long)T * (K / 32);
  long threads = nblk * 32;
  hipLaunchKernelGGL(k_quant_q8_1, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, xq,
                     (half2*)xds, nblk);
  return launched("quant_q8_1");
}

extern "C" int q355_rmsnorm_q8_1(const float* h, const float* w, int8_t* xq, void* xds, int T, int H, float eps,
                                 void* stream) {
  REQUIRE(h && w && xq && xds, "rmsnorm_q8_1: null pointer");
  REQUIRE(T > 0 && H > 0 && H % 32 == 0 && H <= 2048, "rmsnorm_q8_1: T=%d H=%d (H %% 32 == 0, H <= 2048)", T, H);
  hipLaunchKernelGGL(k_rmsnorm_q8_1, dim3(T), dim3(256), 0, (hipStream_t)stream, h, w, xq, (half2*)xds, H, eps);
  return launched("rmsnorm_q8_1");
}

extern "C" int q355_gemv_q4_0_q8_1(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq,
                                   const void* xds, int T, float* y, const float* bias, int epi, void* stream) {
  if (int e = check_mat("gemv_q4_0_q8_1", qs, d, N, K)) return e;
  REQUIRE(xq && xds && y, "gemv_q4_0_q8_1: null pointer");
  REQUIRE(T >= 1 && T <= 4, "gemv_q4_0_q8_1: T=%d outside 1..4", T);
  REQUIRE(epi >= 0 && epi <= 2, "gemv_q4_0_q8_1: epi=%d (0 store, 1 resid, 2 bias)", epi);
  REQUIRE(epi != 2 || bias, "gemv_q4_0_q8_1: bias epilogue needs bias");
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.xq = xq; a.xds = (const half2*)xds; a.y = y; a.aux = bias;
  hipStream_t s = (hipStream_t)stream;
  switch (epi) {
    case 0: return launch_gemv_generic<PRO_Q8, EPI_STORE>(a, s);
    case 1: return launch_gemv_generic<PRO_Q8, EPI_RESID>(a, s);
    default: return launch_gemv_generic<PRO_Q8, EPI_BIAS>(a, s);
  }
}

template <int T, int EPI>
static void launch_gemv_bf16(const uint8_t* qs, const void* d, int N, int K, const void* x, float* y,
                             const float* bias, hipStream_t s) {
  const size_t lds = (size_t)T * K * 2;
  if (K <= 16 * 3 * 32)
    hipLaunchKernelGGL((k_gemv_bf16<T, 3, EPI>), dim3(N / 16), dim3(256), lds, s, qs, (const __half*)d, N, K,
                       (const unsigned short*)x, y, bias);
  else
    hipLaunchKernelGGL((k_gemv_bf16<T, 18, EPI>), dim3(N / 16), dim3(256), lds, s, qs, (const __half*)d, N, K,
                       (const unsigned short*)x, y, bias);
}

template <int EPI>
static int gemv_bf16_t(const uint8_t* qs, const void* d, int N, int K, const void* x, int T, float* y,
                       const float* bias, hipStream_t s) {
  switch (T) {
    case 1: launch_gemv_bf16<1, EPI>(qs, d, N, K, x, y, bias, s); break;
    case 2: launch_gemv_bf16<2, EPI>(qs, d, N, K, x, y, bias, s); break;
    case 3: launch_gemv_bf16<3, EPI>(qs, d, N, K, x, y, bias, s); break;
    default: launch_gemv_bf16<4, EPI>(qs, d, N, K, x, y, bias, s); break;
  }
  return launched("gemv_q4_0_bf16");
}

extern "C" int q355_gemv_q4_0_bf16(const uint8_t* qs, const void* d, int N, int K, const void* x, int T, float* y,
                                   const float* bias, int epi, void* stream) {
  if (int e = check_mat("gemv_q4_0_bf16", qs, d, N, K)) return e;
  REQUIRE(x && y, "gemv_q4_0_bf16: null pointer");
  REQUIRE(T >= 1 && T <= 4, "gemv_q4_0_bf16: T=%d outside 1..4", T);
  REQUIRE(K <= 9216, "gemv_q4_0_bf16: K=%d > 9216", K);
  REQUIRE(epi >= 0 && epi <= 2, "gemv_q4_0_bf16: epi=%d (0 store, 1 resid, 2 bias)", epi);
  REQUIRE(epi != 2 || bias, "gemv_q4_0_bf16: bias epilogue needs bias");
  hipStream_t s = (hipStream_t)stream;
  switch (epi) {
    case 0: return gemv_bf16_t<EPI_STORE>(qs, d, N, K, x, T, y, bias, s);
    case 1: return gemv_bf16_t<EPI_RESID>(qs, d, N, K, x, T, y, bias, s);
    default: return gemv_bf16_t<EPI_BIAS>(qs, d, N, K, x, T, y, bias, s);
  }
}

extern "C" int q355_gemv_blockdots(const uint8_t* qs, int N, int K, const int8_t* xq, int T, int32_t* out,
                                   void* stream) {
  REQUIRE(qs && xq && out, "gemv_blockdots: null pointer");
  REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0 && T > 0, "gemv_blockdots: N=%d K=%d T=%d", N, K, T);
  hipLaunchKernelGGL(k_blockdots, dim3(1024), dim3(256), 0, (hipStream_t)stream, qs, N, K, xq, T, out);
  return launched("gemv_blockdots");
}

extern "C" int q355_qkv_rope_kv(const uint8_t* qs, const void* d, int K, const int64_t* h, const float* nw, double eps,
                                const float* bias, const float* rope_cos, const float* rope_sin, const int32_t* pos,
                                const int32_t* block_table, int bt_stride, int seq_stride, void* kcache,
                                void* vcache, void* qout, int nh, int nkv, int T, void* stream) {
  const int N = (nh + 2 * nkv) * HD;
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 8, "qkv_rope_kv: nh=%d nkv=%d", nh, nkv);
  if (int e = check_mat("qkv_rope_kv", qs, d, N, K)) return e;
  REQUIRE(K <= 1536, "qkv_rope_kv: K=%d > 1536 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "qkv_rope_kv: null pointer");
  REQUIRE(T >= 1 && T <= 4, "qkv_rope_kv: T=%d outside 1..4", T);
  REQUIRE(bt_stride > 0 && (seq_stride == 0 || seq_stride == 1), "qkv_rope_kv: bt_stride=%d seq_stride=%d",
          bt_stride, seq_stride);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.hfix = (const long long*)h; a.nw = nw; a.eps = eps; a.aux = bias;
  a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.nh = nh; a.nkv = nkv;
  return launch_gemv<PRO_RMS, EPI_QKV, 1, 4, 3>(a, 1, (hipStream_t)stream);
}

// Layer 0's QKV product with the embedding in its prologue: h = the tied Q4_0 embedding row of tok[j] (the
// values q355_embed_q4_0 writes, computed by every workgroup), RMSNorm etc. as q355_qkv_rope_kv; h_out
// receives the row (the residual stream of the step). One launch (and one graph node) instead of two.
extern "C" int q355_qkv_rope_kv_embed(const uint8_t* qs, const void* d, int K, const uint8_t* emb_qs,
                                      const void* emb_d, int V, const int32_t* tok, int64_t* h_out, const float* nw,
                                      double eps, const float* bias, const float* rope_cos, const float* rope_sin,
                                      const int32_t* pos, const int32_t* block_table, int bt_stride, int seq_stride,
                                      void* kcache, void* vcache, void* qout, int nh, int nkv, int T, void* stream) {
  const int N = (nh + 2 * nkv) * HD;
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 8, "qkv_rope_kv_embed: nh=%d nkv=%d", nh, nkv);
  if (int e = check_mat("qkv_rope_kv_embed", qs, d, N, K)) return e;
  if (int e = check_mat("qkv_rope_kv_embed (embedding)", emb_qs, emb_d, V, K)) return e;
  REQUIRE(K <= 1536, "qkv_rope_kv_embed: K=%d > 1536 (fused RMSNorm prologue)", K);
  REQUIRE(tok && h_out && nw && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "qkv_rope_kv_embed: null pointer");
  REQUIRE(T >= 1 && T <= 4, "qkv_rope_kv_embed: T=%d outside 1..4", T);
  REQUIRE(bt_stride > 0 && (seq_stride == 0 || seq_stride == 1), "qkv_rope_kv_embed: bt_stride=%d seq_stride=%d",
          bt_stride, seq_stride);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.emb_qs = emb_qs; a.emb_d = (const __half*)emb_d; a.emb_v = V; a.tok = tok; a.hout = (long long*)h_out;
  a.nw = nw; a.eps = eps; a.aux = bias;
  a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.nh = nh; a.nkv = nkv;
  return launch_gemv<PRO_EMB, EPI_QKV, 1, 4, 3>(a, 1, (hipStream_t)stream);
}

extern "C" int q355_ffn_gate_up(const uint8_t* qs, const void* d, int N2, int K, const int64_t* h, const float* nw,
                                double eps, float* m, int T, void* stream) {
  if (int e = check_mat("ffn_gate_up", qs, d, N2, K)) return e;
  REQUIRE(K <= 1536, "ffn_gate_up: K=%d > 1536 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && m, "ffn_gate_up: null pointer");
  REQUIRE(T >= 1 && T <= 4, "ffn_gate_up: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N2; a.K = K; a.T = T;
  a.hfix = (const long long*)h; a.nw = nw; a.eps = eps; a.y = m;
  return launch_gemv<PRO_RMS, EPI_SWIGLU, 5, 4, 3>(a, 1, (hipStream_t)stream);
}

extern "C" int q355_ffn_down(const uint8_t* qs, const void* d, int N, int K, const float* m, int64_t* h, int T,
                             void* stream) {
  if (int e = check_mat("ffn_down", qs, d, N, K)) return e;
  REQUIRE(m && h, "ffn_down: null pointer");
  REQUIRE(T >= 1 && T <= 4, "ffn_down: T=%d outside 1..4", T);
  REQUIRE(K % 128 == 0 && K <= 9216, "ffn_down: K=%d must be a multiple of 128, <= 9216", K);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.xf = m; a.yfix = (long long*)h;
  // 2 K slices of <= 144 blocks: 8 waves = 32 k-lanes x 5 blocks per lane (192 workgroups for N = 1536): 4.32 us
  // per layer against 4.60 with 4 slices of 4 waves (graph-timed)
  return launch_gemv<PRO_F32, EPI_RESID_FIX, 1, 8, 5>(a, 2, (hipStream_t)stream);
}

extern "C" int q355_head_nparts(int V) { return V / 128; }

extern "C" int q355_head_logits(const uint8_t* qs, const void* d, int V, int K, const int64_t* h, const float* nw,
                                double eps, float* logits, float* pmax, int32_t* pidx, int T, void* stream) {
  if (int e = check_mat("head_logits", qs, d, V, K)) return e;
  REQUIRE(V % 128 == 0, "head_logits: V=%d must be a multiple of 128", V);
  REQUIRE(K <= 1536, "head_logits: K=%d > 1536 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && logits && pmax && pidx, "head_logits: null pointer");
  REQUIRE(T >= 1 && T <= 4, "head_logits: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = V; a.K = K; a.T = T;
  a.hfix = (const long long*)h; a.nw = nw; a.eps = eps; a.y = logits; a.pmax = pmax; a.pidx = pidx;
  return launch_gemv<PRO_RMS, EPI_LOGITS, 8, 4, 3>(a, 1, (hipStream_t)stream);
}

static int check_q6k(const char* what, const void* lo, const void* hi, const void* sc, const void* d, int N, int K) {
  REQUIRE(lo && hi && sc && d, "%s: null weight pointer", what);
  REQUIRE(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", what, N);
  REQUIRE(K > 0 && K % 256 == 0, "%s: K=%d must be a positive multiple of 256 (Q6_K super-blocks)", what, K);
  return Q355_OK;
}

extern "C" int q355_head_logits_q6k(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int V, int K,
                                    const int64_t* h, const float* nw, double eps, float* logits, float* pmax,
                                    int32_t* pidx, int T, void* stream) {
  if (int e = check_q6k("head_logits_q6k", lo, hi, sc, d, V, K)) return e;
  REQUIRE(V % 128 == 0, "head_logits_q6k: V=%d must be a multiple of 128", V);
  REQUIRE(K <= 1536, "head_logits_q6k: K=%d > 1536 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && logits && pmax && pidx, "head_logits_q6k: null pointer");
  REQUIRE(T >= 1 && T <= 4, "head_logits_q6k: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = lo; a.qhi = hi; a.qsc = (const uint8_t*)sc; a.d = (const __half*)d; a.N = V; a.K = K; a.T = T;
  a.hfix = (const long long*)h; a.nw = nw; a.eps = eps; a.y = logits; a.pmax = pmax; a.pidx = pidx;
  return launch_gemv<PRO_RMS, EPI_LOGITS, 8, 4, 3, WF_Q6_K>(a, 1, (hipStream_t)stream);
}

extern "C" int q355_gemv_q6_k_q8_1(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int N, int K,
                                   const int8_t* xq, const void* xds, int T, float* y, void* stream) {
  if (int e = check_q6k("gemv_q6_k_q8_1", lo, hi, sc, d, N, K)) return e;
  REQUIRE(xq && xds && y, "gemv_q6_k_q8_1: null pointer");
  REQUIRE(T >= 1 && T <= 4, "gemv_q6_k_q8_1: T=%d outside 1..4", T);
  REQUIRE(K <= 1536, "gemv_q6_k_q8_1: K=%d > 1536", K);
  GemvArgs a = {};
  a.qs = lo; a.qhi = hi; a.qsc = (const uint8_t*)sc; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.xq = xq; a.xds = (const half2*)xds; a.y = y;
  return launch_gemv<PRO_Q8, EPI_STORE, 1, 4, 3, WF_Q6_K>(a, 1, (hipStream_t)stream);
}

extern "C" int q355_finish(const float* pmax, const int32_t* pidx, int nparts, int32_t* tok, int32_t* pos, int T,
                           void* stream) {
  REQUIRE(pmax && pidx && tok && pos, "finish: null pointer");
  REQUIRE(nparts > 0 && T > 0, "finish: nparts=%d T=%d", nparts, T);
  hipLaunchKernelGGL(k_finish, dim3(T), dim3(256), 0, (hipStream_t)stream, pmax, pidx, nparts, tok, pos);
  return launched("finish");
}

extern "C" int q355_embed_q4_0(const uint8_t* qs, const void* d, int V, int H, const int32_t* tok, int64_t* h, int T,
                               void* stream) {
  if (int e = check_mat("embed_q4_0", qs, d, V, H)) return e;
  REQUIRE(tok && h && T > 0, "embed_q4_0: null pointer or T=%d", T);
  hipLaunchKernelGGL(k_embed_q4_0, dim3(T), dim3(64), 0, (hipStream_t)stream, qs, (const __half*)d, V, H, tok,
                     (long long*)h);
  return launched("embed_q4_0");
}

extern "C" int q355_attn_decode(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                double scale, double* part, int8_t* oq, void* ods, float* o32, int T, int fp32,
                                void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && part, "attn_decode: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0, "attn_decode: nh=%d nkv=%d", nh, nkv);
  REQUIRE(nh / nkv == 6 || nh / nkv == 4 || nh / nkv == 8, "attn_decode: GQA group %d (4, 6 or 8 supported)", nh / nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64, "attn_decode: max_chunks=%d bt_stride=%d",
          max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 65535, "attn_decode: T=%d", T);
  REQUIRE((oq == nullptr) == (ods == nullptr), "attn_decode: oq and ods go together");
  REQUIRE(oq || !o32, "attn_decode: o32 needs the merge outputs oq/ods");
  REQUIRE(oq || !fp32, "attn_decode: fp32 = 1 merges in the same launch: oq/ods required");
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part;
  a.oq = oq; a.ods = (half2*)ods; a.o32 = o32;
  hipStream_t s = (hipStream_t)stream;
  if (fp32) {                                           // attention (4-page merge inside) + split merge
    hipLaunchKernelGGL(k_attn_decode_mfma<ATTN_KW>, dim3(nkv * ((max_chunks + 3) / 4), T), dim3(4 * 64 / ATTN_KW * 64), 0, s, a);
    if (int e = launched("attn_decode")) return e;
    hipLaunchKernelGGL(k_attn_merge_split, dim3(nkv, T), dim3(256), 0, s, a);
    return launched("attn_merge_split");
  } else {
    // one query head per workgroup, 4 waves of 16 positions each; the workgroups of a KV head's group each
    // stage its K/V page (from L2 after the first). Measured at position 256 (graph of 28 launches): 4 waves
    // 4.16 us, 8 waves 4.18, 16 waves 4.64, 2 waves 4.95
    const dim3 grid(nh * ((max_chunks + 7) & ~7), T);   // chunk slots padded to 8: one XCD per page
    switch (nh / nkv) {
      case 4: hipLaunchKernelGGL((k_attn_decode<4, double, 4, 4>), grid, dim3(256), 0, s, a); break;
      case 6: hipLaunchKernelGGL((k_attn_decode<6, double, 4, 6>), grid, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((k_attn_decode<8, double, 4, 8>), grid, dim3(256), 0, s, a); break;
    }
  }
  if (int e = launched("attn_decode")) return e;
  if (!oq) return Q355_OK;
  hipLaunchKernelGGL(k_attn_merge, dim3(T, nh), dim3(64), 0, s, a);
  return launched("attn_merge");
}

// ------------------------------------------------------------------------------------------------
// Allocation-free batched decode attention (q355_attn_decode with fp32 = 1): the split partials live in a
// file-scope device array. Each GPU holds its own copy at its own address, looked up once per device with
// hipGetSymbolAddress; host code uses only that address, never the array's name. Calls that overlap on one
// GPU share the array and race; the kernels need no initial contents (each token's merge reads only the
// splits its own attention workgroups wrote in the same call).
static constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_BYTES / sizeof(float)];
static constexpr int NOALLOC_MAX_DEVICES = 64;
static float* g_scratch[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_for_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "attn_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, "attn_decode_noalloc: device %d >= %d", dev, NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : Q355_EINVAL, "attn_decode_noalloc: hipGetSymbolAddress: %s",
                  hipGetErrorString(e));
    g_scratch[dev] = (float*)p;
  }
  *out = g_scratch[dev];
  return Q355_OK;
}

extern "C" int64_t q355_attn_decode_noalloc_max_bytes(void) { return (int64_t)NOALLOC_SCRATCH_BYTES; }

extern "C" int q355_attn_decode_noalloc(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                        const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                        double scale, int8_t* oq, void* ods, float* o32, int T, void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && oq && ods, "attn_decode_noalloc: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16, "attn_decode_noalloc: nh=%d nkv=%d", nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64,
          "attn_decode_noalloc: max_chunks=%d bt_stride=%d", max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 65535, "attn_decode_noalloc: T=%d", T);
  // split partials: [T][nkv][ceil(max_chunks / 4)][G] (o[128], M, L) fp32
  const size_t need = (size_t)T * nh * ((max_chunks + 3) / 4) * (HD + 2) * sizeof(float);
  REQUIRE(need <= NOALLOC_SCRATCH_BYTES,
          "attn_decode_noalloc: T=%d nh=%d max_chunks=%d need %zu bytes of split partials, the fixed scratch holds %zu",
          T, nh, max_chunks, need, NOALLOC_SCRATCH_BYTES);
  float* ws = nullptr;
  if (int e = scratch_for_current_device(&ws)) return e;
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = (double*)ws;
  a.oq = oq; a.ods = (half2*)ods; a.o32 = o32;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_attn_decode_mfma<ATTN_KW>, dim3(nkv * ((max_chunks + 3) / 4), T), dim3(4 * 64 / ATTN_KW * 64), 0,
                     s, a);
  if (int e = launched("attn_decode_noalloc")) return e;
  hipLaunchKernelGGL(k_attn_merge_split, dim3(nkv, T), dim3(256), 0, s, a);
  return launched("attn_decode_noalloc merge");
}

extern "C" int q355_attn_decode_f16(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                    const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                    double scale, double* part, void* oh, int T, void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && part && oh, "attn_decode_f16: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16, "attn_decode_f16: nh=%d nkv=%d", nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64, "attn_decode_f16: max_chunks=%d bt_stride=%d",
          max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 65535, "attn_decode_f16: T=%d", T);
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part; a.oh = (__half*)oh;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_attn_decode_mfma<ATTN_KW>, dim3(nkv * ((max_chunks + 3) / 4), T), dim3(4 * 64 / ATTN_KW * 64), 0, s, a);
  if (int e = launched("attn_decode_f16")) return e;
  hipLaunchKernelGGL(k_attn_merge_split, dim3(nkv, T), dim3(256), 0, s, a);
  return launched("attn_merge_split");
}

extern "C" int q355_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                                 const int32_t* pos, int nh, int64_t* h, int T, void* stream) {
  const int K = nh * HD;
  if (int e = check_mat("attn_o_resid", qs, d, N, K)) return e;
  REQUIRE(part && pos && h, "attn_o_resid: null pointer");
  REQUIRE(K <= 1536 && nh % 3 == 0, "attn_o_resid: nh=%d must be a multiple of 3 with nh*128 <= 1536", nh);
  REQUIRE(max_chunks > 0 && max_chunks <= 64, "attn_o_resid: max_chunks=%d", max_chunks);
  REQUIRE(T >= 1 && T <= 4, "attn_o_resid: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.attn_part = part; a.attn_max_chunks = max_chunks; a.pos = pos; a.nh = nh; a.yfix = (long long*)h;
  // 3 K slices of nh/3 heads (16 blocks for nh = 12): 16 k-lanes x 1 block per lane
  // two 16-row tiles per workgroup (144 workgroups): 4.1 us per layer against 4.57 with one (graph-timed)
  if ((N / 16) % 2 == 0) return launch_gemv<PRO_ATTN, EPI_RESID_FIX, 2, 4, 1>(a, 3, (hipStream_t)stream);
  return launch_gemv<PRO_ATTN, EPI_RESID_FIX, 1, 4, 1>(a, 3, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------------------
// MFMA path (batched decode, prefill)

extern "C" int q355_rmsnorm_fix_q8_1(const int64_t* h, const float* w, int8_t* xq, void* xds, int T, int H, double eps,
                                     void* stream) {
  REQUIRE(h && w && xq && xds, "rmsnorm_fix_q8_1: null pointer");
  REQUIRE(T > 0 && H > 0 && H % 32 == 0 && H <= 2048, "rmsnorm_fix_q8_1: T=%d H=%d (H %% 32 == 0, <= 2048)", T, H);
  hipLaunchKernelGGL(k_rmsnorm_fix_q8_1, dim3(T), dim3(256), 0, (hipStream_t)stream, (const long long*)h, w, xq,
                     (half2*)xds, H, eps);
  return launched("rmsnorm_fix_q8_1");
}

template <int TG, int KPW, int EPI>
static int launch_mmq_reg(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  if constexpr (TG == 1) {
    if (a.T <= 8) {                                     // half-column form (k_mmq_r HALF)
      hipLaunchKernelGGL((k_mmq_reg<TG, 4, 4, KPW, EPI, false, true>), grid, dim3(256), lds, s, a);
      return launched("mmq");
    }
  }
  hipLaunchKernelGGL((k_mmq_reg<TG, 4, 4, KPW, EPI>), grid, dim3(256), lds, s, a);
  return launched("mmq");
}

template <int TG, int EPI>
static int launch_mmq(GemvArgs a, int KS, hipStream_t s) {
  constexpr int NT = 4, NW = 4, TT = 16 * TG;
  constexpr size_t LDS_MAX = 65536;
  const int nb = a.K / 32, per = (nb + KS - 1) / KS;
  const dim3 grid(a.N / (16 * NT), KS, (a.T + TT - 1) / TT);
  const size_t pb = (size_t)NW * NT * TT * 16 * sizeof(MmqAcc<TG>);     // wave partials
  if (per <= NW * 5) {
    // narrow K slices (decode): the whole slice's nibbles in registers (KPW blocks per wave), its activations
    // and scales in LDS; wider slices run faster through the pipelined kernel below
    const size_t xb = (size_t)TT * (per * 32 + 16) + (size_t)TT * per * 8 + (size_t)NT * per * 32;
    const size_t lds = xb > pb ? xb : pb;
    if (lds <= 160 * 1024) {                          // gfx950: 160 KB of LDS per workgroup
      if (per <= NW * 1) return launch_mmq_reg<TG, 1, EPI>(a, grid, lds, s);
      if (per <= NW * 2) return launch_mmq_reg<TG, 2, EPI>(a, grid, lds, s);
      return launch_mmq_reg<TG, 5, EPI>(a, grid, lds, s);
    }
  }
  // activation chunk: TT rows of (32 B per block + 16 B pad) + 8 B (d, sum) per block, within 64 KB
  const int ch_max = (int)((LDS_MAX - (size_t)TT * 16) / ((size_t)TT * 40));
  const int nchunks = (per + ch_max - 1) / ch_max;
  a.mmq_chunk = (per + nchunks - 1) / nchunks;
  const size_t xb = (size_t)TT * (a.mmq_chunk * 32 + 16) + (size_t)TT * a.mmq_chunk * 8;
  const size_t lds = xb > pb ? xb : pb;
  if (lds > LDS_MAX) return fail(Q355_EINVAL, "mmq: %zu B of LDS for %d tokens", lds, TT);
  hipLaunchKernelGGL((k_mmq<TG, NT, NW, EPI>), grid, dim3(NW * 64), lds, s, a);
  return launched("mmq");
}

// Prefill sizes (STORE, RESID_FIX, SWIGLU_Q8, QKV with at least one 128 x 64 tile per CU): the LDS-tiled
// kernel, workgroups of 128 rows x 64 tokens (2 x 2 waves of 64 x 32; 165 VGPRs: three per CU). One K slice: each output
// has exactly one writer, so RESID_FIX is a plain read-add-write. Measured at P = 2048: gate_up 247.6 us with
// 128-token workgroups (two per CU) against 223.5 us with 64-token ones.
template <int EPI>
static int launch_mmq_big(GemvArgs a, hipStream_t s) {
  const int rt = a.N / 128, tt2 = (a.T + 63) / 64;
  if (rt * tt2 >= 768) {                           // three or more 64-token workgroups per CU
    constexpr size_t lds2 = 2 * LdsTile<2, 2, 2, TILE_CB>::BUF;
    hipLaunchKernelGGL((k_mmq_tile<2, 2, 2, EPI>), dim3(rt, 1, tt2), dim3(256), lds2, s, a);
  } else {
    // 32-token workgroups: twice the workgroups for grids that give CUs fewer than three 64-token ones, or
    // an uneven number (N = 1536: 384 of them): measured at P = 2048, down 166.6 -> 150.6 us, qkv (512 ->
    // 1024 workgroups) 49.9 -> 42.5 us; 64-row workgroups of 2 waves instead: down 186 us
    constexpr size_t lds1 = 2 * LdsTile<2, 2, 1, TILE_CB>::BUF;
    hipLaunchKernelGGL((k_mmq_tile<2, 2, 1, EPI>), dim3(rt, 1, (a.T + 31) / 32), dim3(256), lds1, s, a);
  }
  return launched("mmq");
}

// LOGITS over a large vocabulary (N % 128 == 0) for up to 64 tokens: the LDS-tiled kernel with all tokens
// in one workgroup, so each weight is read once (128 rows x 16 / 32 / 64 tokens per workgroup).
static int launch_mmq_logits_tile(const GemvArgs& a, hipStream_t s) {
  const dim3 grid(a.N / 128, 1, 1);
  if (a.T <= 16) {
    constexpr size_t lds = 2 * LdsTile<2, 1, 1, TILE_CB>::BUF;
    hipLaunchKernelGGL((k_mmq_tile<2, 1, 1, EPI_LOGITS>), grid, dim3(128), lds, s, a);
  } else if (a.T <= 32) {
    constexpr size_t lds = 2 * LdsTile<2, 2, 1, TILE_CB>::BUF;
    hipLaunchKernelGGL((k_mmq_tile<2, 2, 1, EPI_LOGITS>), grid, dim3(256), lds, s, a);
  } else {
    constexpr size_t lds = 2 * LdsTile<2, 2, 2, TILE_CB>::BUF;
    hipLaunchKernelGGL((k_mmq_tile<2, 2, 2, EPI_LOGITS>), grid, dim3(256), lds, s, a);
  }
  return launched("mmq");
}

// Register-resident decode-batch kernel (T <= 32). SWIGLU (fp32 out) with N % 80 == 0 and K <= 1536:
// 80-row workgroups of 16 waves x 3 blocks (8 x 6 at 32 tokens; 224 for gate_up, one per CU). RESID_FIX from fp32 activations
// (XF32): 64-row workgroups, K split 32 blocks per slice (16 waves x 2 up to 16 tokens, else 8 x 4) or <= 16
// (4 waves x 4).
// Returns -1 outside these classes.
// Up to 8 tokens (TG = 1) the kernels run in their half-column form (k_mmq_r HALF).
template <int TG, int NT, int NW, int KPW, int EPI, bool XF32>
static void launch_mmq_r(const GemvArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (TG == 1) {
    if (a.T <= 8) {
      hipLaunchKernelGGL((k_mmq_r<TG, NT, NW, KPW, EPI, XF32, true>), grid, dim3(NW * 64), 0, s, a);
      return;
    }
  }
  hipLaunchKernelGGL((k_mmq_r<TG, NT, NW, KPW, EPI, XF32>), grid, dim3(NW * 64), 0, s, a);
}

template <int TG, int EPI, bool XF32>
static int launch_mmq_r_tg(const GemvArgs& a, hipStream_t s) {
  const int nb = a.K / 32;
  if constexpr (EPI == EPI_SWIGLU && !XF32) {
    if (a.N % 80 || a.N / 80 > 256 || nb > 8 * 6) return -1;
    // up to 16 tokens 16 waves x 3 blocks (8 x 6: 9.66 against 8.34 us at B = 8); 32 tokens keep 8 waves (the
    // 16-wave partials would need 160 KB of LDS)
    if constexpr (TG == 1) launch_mmq_r<TG, 5, 16, 3, EPI, XF32>(a, dim3(a.N / 80), s);
    else launch_mmq_r<TG, 5, 8, 6, EPI, XF32>(a, dim3(a.N / 80), s);
    return launched("mmq");
  }
  if constexpr (EPI == EPI_QKV && !XF32) {
    // one writer per output (no K split): 16-row workgroups of 16 waves x 3 blocks (8 waves x 6: 5.77 / 9.80 us
    // at B = 8 / 32 against 5.20 / 8.94), bias + RoPE + K/V write in the epilogue (a RoPE pair sits in
    // adjacent rows of one tile)
    if (a.N % 16 || nb > 16 * 3) return -1;
    launch_mmq_r<TG, 1, 16, 3, EPI, XF32>(a, dim3(a.N / 16), s);
    return launched("mmq");
  }
  if constexpr (EPI == EPI_RESID_FIX && XF32) {
    if (a.N % 64) return -1;
    if (nb >= 64) {
      const int KS = (nb + 31) / 32;
      if constexpr (TG == 1) launch_mmq_r<TG, 4, 16, 2, EPI, XF32>(a, dim3(a.N / 64, KS), s);
      else launch_mmq_r<TG, 4, 8, 4, EPI, XF32>(a, dim3(a.N / 64, KS), s);
      return launched("mmq");
    }
    int KS = 1;
    while ((a.N / 64) * KS < 256 && nb / (KS + 1) >= 4) ++KS;
    if ((nb + KS - 1) / KS > 16) return -1;
    launch_mmq_r<TG, 4, 4, 4, EPI, XF32>(a, dim3(a.N / 64, KS), s);
    return launched("mmq");
  }
  return -1;
}

template <int EPI>
static int launch_mmq_tg(const GemvArgs& a, int KS, hipStream_t s) {
  if constexpr (EPI == EPI_SWIGLU) {
    if (a.T <= 32) {
      const int r = a.T <= 16 ? launch_mmq_r_tg<1, EPI, false>(a, s) : launch_mmq_r_tg<2, EPI, false>(a, s);
      if (r >= 0) return r;
    }
  }
  if constexpr (EPI == EPI_LOGITS)
    if (a.N % 128 == 0 && a.N >= 128 * 256 && a.T <= 64) return launch_mmq_logits_tile(a, s);
  // prefill sizes: the LDS-tiled kernel; from 512 tokens on always, so a prompt split into chunks of >= 512
  // tokens computes every row with the same kernel (and the same summation order) as one chunk
  if constexpr (EPI == EPI_STORE || EPI == EPI_RESID_FIX || EPI == EPI_SWIGLU_Q8)
    if (a.N % 128 == 0 && (a.T >= 512 || (a.N / 128) * ((a.T + 63) / 64) >= 256)) return launch_mmq_big<EPI>(a, s);
  // up to 64 tokens (decode batches): 16-token workgroups, several per CU, hide each other's latencies;
  // prefill sizes: 32- or 64-token workgroups reuse every staged weight block 2 or 4 times
  if (a.T <= 64) return launch_mmq<1, EPI>(a, KS, s);
  return a.T < 256 ? launch_mmq<2, EPI>(a, KS, s) : launch_mmq<4, EPI>(a, KS, s);
}

extern "C" int q355_mmq_q4_0_q8_1(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq, const void* xds,
                                  int T, int epi, float* y, int64_t* yfix, int8_t* oq, void* ods, float* pmax,
                                  int32_t* pidx, void* stream) {
  if (int e = check_mat("mmq_q4_0_q8_1", qs, d, N, K)) return e;
  REQUIRE(xq && xds, "mmq_q4_0_q8_1: null activation pointer");
  REQUIRE(T >= 1 && T <= 65535 * 32, "mmq_q4_0_q8_1: T=%d", T);
  REQUIRE(N % 64 == 0, "mmq_q4_0_q8_1: N=%d must be a multiple of 64", N);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xq = xq; a.xds = (const half2*)xds;
  hipStream_t s = (hipStream_t)stream;
  const int nb = K / 32, groups = N / 64;
  switch (epi) {
    case 0:
      REQUIRE(y, "mmq_q4_0_q8_1: store needs y");
      a.y = y;
      return launch_mmq_tg<EPI_STORE>(a, 1, s);
    case 6: {
      REQUIRE(yfix, "mmq_q4_0_q8_1: resid_fix needs yfix");
      a.yfix = (long long*)yfix;
      int KS = T >= 256 ? 1 : 384 / groups;           // prefill sizes have parallelism enough
      KS = KS < 1 ? 1 : (KS > nb / 4 ? nb / 4 : KS);
      if (KS < 1) KS = 1;
      return launch_mmq_tg<EPI_RESID_FIX>(a, KS, s);
    }
    case 4:
      REQUIRE(y, "mmq_q4_0_q8_1: swiglu needs y");
      a.y = y;
      return launch_mmq_tg<EPI_SWIGLU>(a, 1, s);
    case 7:
      REQUIRE(oq && ods, "mmq_q4_0_q8_1: swiglu_q8 needs oq/ods");
      a.oq = oq; a.ods = (half2*)ods;
      return launch_mmq_tg<EPI_SWIGLU_Q8>(a, 1, s);
    case 5:
      REQUIRE(pmax && pidx, "mmq_q4_0_q8_1: logits needs pmax, pidx (y optional)");
      a.y = y; a.pmax = pmax; a.pidx = pidx;
      return launch_mmq_tg<EPI_LOGITS>(a, 1, s);
    default:
      return fail(Q355_EINVAL, "mmq_q4_0_q8_1: epi=%d (0 store, 4 swiglu, 5 logits, 6 resid_fix, 7 swiglu_q8)", epi);
  }
}

// Batched decode, int8 path: attention without its merge launch, then the O projection whose activation
// staging merges the split partials (and quantizes to Q8_1) per head.
extern "C" int q355_attn_decode_partials(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                         const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                         double scale, double* part, int8_t* oq, void* ods, int T, void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && part && oq && ods, "attn_decode_partials: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16, "attn_decode_partials: nh=%d nkv=%d", nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64, "attn_decode_partials: max_chunks=%d", max_chunks);
  REQUIRE(T > 0 && T <= 65535, "attn_decode_partials: T=%d", T);
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part; a.oq = oq; a.ods = (half2*)ods;
  hipLaunchKernelGGL(k_attn_decode_mfma<ATTN_KW>, dim3(nkv * ((max_chunks + 3) / 4), T), dim3(4 * 64 / ATTN_KW * 64), 0,
                     (hipStream_t)stream, a);
  return launched("attn_decode_partials");
}

// Batched decode attention of the int8 path in f64 (k_attn_batch_f64, 4 pages per split) + the f64 split merge
// -> Q8_1 oq/ods (and fp32 o32 if asked). q64: the f64 queries the QKV epilogue writes.
constexpr int ATTN64_SPG = 2;                         // pages per split (4 waves per page)
constexpr int ATTN64_FUSED_MERGE_T = 16;              // work-list launches of up to this many tokens merge in-kernel

template <int G>
static int launch_attn_f64(const AttnArgs& a, int T, hipStream_t s) {
  const int nsp = (a.max_chunks + ATTN64_SPG - 1) / ATTN64_SPG;
  if (a.arrivals)                                       // up to 16 tokens: few workgroups, latency first
    hipLaunchKernelGGL((k_attn_batch_f64<G, ATTN64_SPG, true>), dim3(a.nkv * nsp, T), dim3(ATTN64_SPG * 256), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn_batch_f64<G, ATTN64_SPG>), dim3(a.nkv * nsp, T), dim3(ATTN64_SPG * 256), 0, s, a);
  if (int e = launched("attn_decode_f64")) return e;
  if (nsp == 1 || a.arrivals) return Q355_OK;          // every token fits one split, or merged by its last split
  hipLaunchKernelGGL((k_attn_merge_f64<G, ATTN64_SPG>), dim3(a.nkv, T), dim3(G * 64), 0, s, a);
  return launched("attn_merge_f64");
}

static int attn_decode_f64(const double* q64, const void* kcache, const void* vcache, const int32_t* pos,
                           const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks, double scale,
                           double* part, int8_t* oq, void* ods, float* o32, int T, const void* work, void* stream) {
  REQUIRE(q64 && kcache && vcache && pos && block_table && part && oq && ods, "attn_decode_f64: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0, "attn_decode_f64: nh=%d nkv=%d", nh, nkv);
  REQUIRE(nh / nkv == 6 || nh / nkv == 4 || nh / nkv == 8, "attn_decode_f64: GQA group %d (4, 6 or 8 supported)",
          nh / nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64, "attn_decode_f64: max_chunks=%d bt_stride=%d",
          max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 65535, "attn_decode_f64: T=%d", T);
  AttnArgs a = {};
  a.q64 = q64; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part; a.oq = oq; a.ods = (half2*)ods; a.o32 = o32;
  a.work = (const int4*)work;
  // the arrival counters follow the items in the work buffer. Up to 16 tokens the last split of each (token, KV
  // head) merges it (B = 8: 1.567 -> 1.533 ms per step); at 32 the merging workgroups' 4-split load rounds
  // outlast the separate merge launch (2.39 -> 2.44 ms), so that keeps it
  if (work && T <= ATTN64_FUSED_MERGE_T)
    a.arrivals = (int*)((char*)work + (size_t)16 * a.nkv * ((max_chunks + ATTN64_SPG - 1) / ATTN64_SPG) * T);
  hipStream_t s = (hipStream_t)stream;
  switch (nh / nkv) {
    case 4: return launch_attn_f64<4>(a, T, s);
    case 6: return launch_attn_f64<6>(a, T, s);
    default: return launch_attn_f64<8>(a, T, s);
  }
}

extern "C" int q355_attn_decode_f64(const double* q64, const void* kcache, const void* vcache, const int32_t* pos,
                                    const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                    double scale, double* part, int8_t* oq, void* ods, float* o32, int T,
                                    void* stream) {
  return attn_decode_f64(q64, kcache, vcache, pos, block_table, bt_stride, nh, nkv, max_chunks, scale, part, oq, ods,
                         o32, T, nullptr, stream);
}

// The step's live-item list of q355_attn_decode_f64_wl: 16 B per item, nkv * ceil(max_chunks / 2) * T items,
// then one int arrival counter per (token, KV head).
extern "C" int64_t q355_attn_f64_worklist_bytes(int T, int nkv, int max_chunks) {
  return (int64_t)16 * nkv * ((max_chunks + ATTN64_SPG - 1) / ATTN64_SPG) * T + (int64_t)4 * T * nkv;
}

extern "C" int q355_attn_f64_worklist(const int32_t* pos, const int32_t* block_table, int bt_stride, int nkv,
                                      int max_chunks, int T, void* work, void* stream) {
  REQUIRE(pos && block_table && work, "attn_f64_worklist: null pointer");
  REQUIRE(nkv > 0 && nkv <= 255 && max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64,
          "attn_f64_worklist: nkv=%d max_chunks=%d bt_stride=%d", nkv, max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 64, "attn_f64_worklist: T=%d (1..64)", T);
  const int cap = nkv * ((max_chunks + ATTN64_SPG - 1) / ATTN64_SPG) * T;
  hipLaunchKernelGGL(k_attn_worklist<ATTN64_SPG>, dim3(1), dim3(64), 0, (hipStream_t)stream, pos, block_table,
                     bt_stride, T, nkv, max_chunks, (int4*)work, cap);
  return launched("attn_f64_worklist");
}

// q355_attn_decode_f64 over the step's live-item list (q355_attn_f64_worklist, built from the same pos,
// block_table, nkv, max_chunks and T after the positions were last changed): bit-identical outputs.
extern "C" int q355_attn_decode_f64_wl(const double* q64, const void* kcache, const void* vcache, const int32_t* pos,
                                       const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                       double scale, double* part, int8_t* oq, void* ods, float* o32, int T,
                                       const void* work, void* stream) {
  REQUIRE(work, "attn_decode_f64_wl: null work list");
  REQUIRE(T <= 64, "attn_decode_f64_wl: T=%d (the work list holds up to 64 tokens)", T);
  return attn_decode_f64(q64, kcache, vcache, pos, block_table, bt_stride, nh, nkv, max_chunks, scale, part, oq, ods,
                         o32, T, work, stream);
}

extern "C" int q355_attn_decode_partials_f16(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                             const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                             double scale, double* part, void* oh, int T, void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && part && oh, "attn_decode_partials_f16: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16, "attn_decode_partials_f16: nh=%d nkv=%d", nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride && max_chunks <= 64, "attn_decode_partials_f16: max_chunks=%d",
          max_chunks);
  REQUIRE(T > 0 && T <= 65535, "attn_decode_partials_f16: T=%d", T);
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part; a.oh = (__half*)oh;
  hipLaunchKernelGGL(k_attn_decode_mfma<ATTN_KW>, dim3(nkv * ((max_chunks + 3) / 4), T), dim3(4 * 64 / ATTN_KW * 64), 0,
                     (hipStream_t)stream, a);
  return launched("attn_decode_partials_f16");
}

extern "C" int q355_gemm_f16_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                                          const int32_t* pos, int nh, int nkv, const void* oh, int64_t* h, int T,
                                          void* stream) {
  const int K = nh * HD;
  if (int e = check_mat("gemm_f16_attn_o_resid", qs, d, N, K)) return e;
  REQUIRE(part && pos && oh && h, "gemm_f16_attn_o_resid: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16 && N % 64 == 0, "gemm_f16_attn_o_resid: N=%d nh=%d nkv=%d",
          N, nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= 64 && T >= 1 && T <= 16, "gemm_f16_attn_o_resid: max_chunks=%d T=%d (T <= 16)",
          max_chunks, T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xh = (const __half*)oh;
  a.attn_part = part; a.attn_max_chunks = max_chunks; a.pos = pos; a.nh = nh; a.nkv = nkv; a.yfix = (long long*)h;
  hipLaunchKernelGGL(k_gemm_f16_attn_o, dim3(N / 64, nh), dim3(256), 0, (hipStream_t)stream, a);
  return launched("gemm_f16_attn_o_resid");
}

extern "C" int q355_mmq_attn_o_resid(const uint8_t* qs, const void* d, int N, const double* part, int max_chunks,
                                     const int32_t* pos, int nh, int nkv, const int8_t* xq, const void* xds,
                                     int64_t* h, int T, void* stream) {
  const int K = nh * HD;
  if (int e = check_mat("mmq_attn_o_resid", qs, d, N, K)) return e;
  REQUIRE(part && pos && xq && xds && h, "mmq_attn_o_resid: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && N % 64 == 0, "mmq_attn_o_resid: N=%d nh=%d nkv=%d", N, nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= 64 && T >= 1 && T <= 65535 * 16, "mmq_attn_o_resid: max_chunks=%d T=%d",
          max_chunks, T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xq = xq; a.xds = (const half2*)xds;
  a.attn_part = part; a.attn_max_chunks = max_chunks; a.pos = pos; a.nh = nh; a.nkv = nkv; a.yfix = (long long*)h;
  // one K slice per head (4 blocks), 16 tokens per workgroup
  constexpr int TT = 16, NT = 4, NW = 4, per = 4;
  const size_t xb = (size_t)TT * (per * 32 + 16) + (size_t)TT * per * 8 + (size_t)NT * per * 32;
  const size_t pb = (size_t)NW * NT * TT * 16 * sizeof(MmqAcc<1>);
  hipLaunchKernelGGL((k_mmq_reg<1, NT, NW, 1, EPI_RESID_FIX, true>), dim3(N / 64, nh, (T + TT - 1) / TT), dim3(256),
                     xb > pb ? xb : pb, (hipStream_t)stream, a);
  return launched("mmq_attn_o_resid");
}

extern "C" int q355_mmq_nparts(int N) { return N / 64; }

extern "C" int q355_mmq_q6k_logits(const uint8_t* lo, const uint8_t* hi, const int8_t* sc, const void* d, int V, int K,
                                   const int8_t* xq, const void* xds, int T, float* y, float* pmax, int32_t* pidx,
                                   void* stream) {
  REQUIRE(lo && hi && sc && d && xq && xds && pmax && pidx, "mmq_q6k_logits: null pointer");
  REQUIRE(V > 0 && V % 64 == 0, "mmq_q6k_logits: V=%d must be a positive multiple of 64", V);
  REQUIRE(K > 0 && K % 256 == 0 && K <= 1536, "mmq_q6k_logits: K=%d must be a multiple of 256 and <= 1536", K);
  REQUIRE(T >= 1 && T <= 32, "mmq_q6k_logits: T=%d outside 1..32", T);
  GemvArgs a = {};
  a.qs = lo; a.qhi = hi; a.qsc = (const uint8_t*)sc; a.d = (const __half*)d; a.N = V; a.K = K; a.T = T;
  a.xq = xq; a.xds = (const half2*)xds; a.y = y; a.pmax = pmax; a.pidx = pidx;
  const int TT = T <= 16 ? 16 : 32;
  const size_t lds = (size_t)TT * (K + Q6M_XPAD) + (size_t)TT * (K / 32) * sizeof(float);
  if (T <= 16)
    hipLaunchKernelGGL(k_mmq_q6k_logits<1>, dim3(V / 64), dim3(Q6M_WAVES * 64), lds, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(k_mmq_q6k_logits<2>, dim3(V / 64), dim3(Q6M_WAVES * 64), lds, (hipStream_t)stream, a);
  return launched("mmq_q6k_logits");
}

extern "C" int q355_mmq_q4_0_f32(const uint8_t* qs, const void* d, int N, int K, const float* xf, int T,
                                 int64_t* yfix, void* stream) {
  if (int e = check_mat("mmq_q4_0_f32", qs, d, N, K)) return e;
  REQUIRE(xf && yfix, "mmq_q4_0_f32: null pointer");
  REQUIRE(T >= 1 && T <= 32, "mmq_q4_0_f32: T=%d (decode batches, <= 32)", T);
  REQUIRE(N % 64 == 0, "mmq_q4_0_f32: N=%d must be a multiple of 64", N);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xf = xf; a.yfix = (long long*)yfix;
  hipStream_t s = (hipStream_t)stream;
  const int r = T <= 16 ? launch_mmq_r_tg<1, EPI_RESID_FIX, true>(a, s) : launch_mmq_r_tg<2, EPI_RESID_FIX, true>(a, s);
  if (r < 0) return fail(Q355_EINVAL, "mmq_q4_0_f32: K=%d outside the supported slices", K);
  return r;
}

// ------------------------------------------------------------------------------------------------
// fp16-activation batched decode path.
template <int TG, int EPI>
static int launch_gemm_f16(GemvArgs a, int KS, hipStream_t s) {
  constexpr int NT = 4, NW = 4, TT = 16 * TG;
  constexpr size_t LDS_MAX = 65536;
  const int nb = a.K / 32, per = (nb + KS - 1) / KS;
  const size_t pb = (size_t)NW * NT * TT * 16 * 4;
  const int ch_max = (int)(LDS_MAX / ((size_t)TT * 2) - 8) / 32;
  const int nchunks = (per + ch_max - 1) / ch_max;
  a.mmq_chunk = (per + nchunks - 1) / nchunks;
  const size_t xb = (size_t)TT * (a.mmq_chunk * 32 + 8) * 2;
  const size_t lds = xb > pb ? xb : pb;
  const dim3 grid(a.N / (16 * NT), KS, (a.T + TT - 1) / TT);
  hipLaunchKernelGGL((k_gemm_f16<TG, NT, NW, EPI>), grid, dim3(NW * 64), lds, s, a);
  return launched("gemm_f16");
}

// Register-resident variant for T <= 32: one launch per shape class. SWIGLU_F16 and the other single-slice
// epilogues: 80-row workgroups (N % 80 == 0; 224 for gate_up, one per CU; 16 waves x 3 blocks up to 16 tokens,
// measured 8.4 against 9.0 us at B = 8) or 64-row ones, 8 waves x 6 blocks over K <= 1536. RESID_FIX: 64-row workgroups of 4 waves, K split until ~256 workgroups.
// Returns -1 when the shape falls outside these classes.
template <int TG, int EPI>
static int launch_gemm_f16r_tg(const GemvArgs& a, hipStream_t s) {
  const int nb = a.K / 32;
  if constexpr (EPI == EPI_QKV) {                    // no K split: 16-row workgroups, finish in the epilogue
    if (a.N % 16 || nb > 16 * 3) return -1;
    hipLaunchKernelGGL((k_gemm_f16r<TG, 1, 16, 3, EPI>), dim3(a.N / 16), dim3(1024), 0, s, a);
    return launched("gemm_f16");
  } else {
    if (EPI == EPI_RESID_FIX) {
      if (a.N % 64) return -1;
      if (nb >= 64) {                                  // long K (down): 16 waves x 2 blocks per slice (8 x 4 at 32 tokens)
        const int KS = (nb + 31) / 32;
        if constexpr (TG == 1) hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 16, 2, EPI>), dim3(a.N / 64, KS), dim3(1024), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 8, 4, EPI>), dim3(a.N / 64, KS), dim3(512), 0, s, a);
        return launched("gemm_f16");
      }
      int KS = 1;
      while ((a.N / 64) * KS < 256 && nb / (KS + 1) >= 4) ++KS;
      while ((nb + KS - 1) / KS > 4 * 8) ++KS;
      const int per = (nb + KS - 1) / KS;
      const dim3 grid(a.N / 64, KS);
      if (per <= 4 * 2) hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 4, 2, EPI>), grid, dim3(256), 0, s, a);
      else if (per <= 4 * 4) hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 4, 4, EPI>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 4, 8, EPI>), grid, dim3(256), 0, s, a);
      return launched("gemm_f16");
    }
    if (nb > 8 * 6) return -1;
    if (a.N % 80 == 0 && a.N / 80 <= 256) {
      if constexpr (TG == 1) hipLaunchKernelGGL((k_gemm_f16r<TG, 5, 16, 3, EPI>), dim3(a.N / 80), dim3(1024), 0, s, a);
      else hipLaunchKernelGGL((k_gemm_f16r<TG, 5, 8, 6, EPI>), dim3(a.N / 80), dim3(512), 0, s, a);
    } else {
      if (a.N % 64) return -1;
      hipLaunchKernelGGL((k_gemm_f16r<TG, 4, 8, 6, EPI>), dim3(a.N / 64), dim3(512), 0, s, a);
    }
    return launched("gemm_f16");
  }
}

template <int EPI>
static int launch_gemm_f16_tg(const GemvArgs& a, int KS, hipStream_t s) {
  if (a.T <= 32) {
    const int r = a.T <= 16 ? launch_gemm_f16r_tg<1, EPI>(a, s) : launch_gemm_f16r_tg<2, EPI>(a, s);
    if (r >= 0) return r;
  }
  return a.T <= 16 ? launch_gemm_f16<1, EPI>(a, KS, s) : launch_gemm_f16<2, EPI>(a, KS, s);
}

extern "C" int q355_gemm_q4_0_f16(const uint8_t* qs, const void* d, int N, int K, const void* xh, int T, int epi,
                                  float* y, int64_t* yfix, void* yh, float* pmax, int32_t* pidx, void* stream) {
  if (int e = check_mat("gemm_q4_0_f16", qs, d, N, K)) return e;
  REQUIRE(xh, "gemm_q4_0_f16: null activation pointer");
  REQUIRE(T >= 1 && T <= 65535 * 32, "gemm_q4_0_f16: T=%d", T);
  REQUIRE(N % 64 == 0, "gemm_q4_0_f16: N=%d must be a multiple of 64", N);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xh = (const __half*)xh;
  hipStream_t s = (hipStream_t)stream;
  const int nb = K / 32, groups = N / 64;
  switch (epi) {
    case 0:
      REQUIRE(y, "gemm_q4_0_f16: store needs y");
      a.y = y;
      return launch_gemm_f16_tg<EPI_STORE>(a, 1, s);
    case 5:
      REQUIRE(pmax && pidx, "gemm_q4_0_f16: logits needs pmax, pidx (y optional)");
      a.y = y; a.pmax = pmax; a.pidx = pidx;
      return launch_gemm_f16_tg<EPI_LOGITS>(a, 1, s);
    case 6: {
      REQUIRE(yfix, "gemm_q4_0_f16: resid_fix needs yfix");
      a.yfix = (long long*)yfix;
      int KS = 384 / groups;
      KS = KS < 1 ? 1 : (KS > nb / 4 ? nb / 4 : KS);
      if (KS < 1) KS = 1;
      return launch_gemm_f16_tg<EPI_RESID_FIX>(a, KS, s);
    }
    case 8:
      REQUIRE(yh, "gemm_q4_0_f16: swiglu_f16 needs yh");
      a.yh = (__half*)yh;
      return launch_gemm_f16_tg<EPI_SWIGLU_F16>(a, 1, s);
    default:
      return fail(Q355_EINVAL, "gemm_q4_0_f16: epi=%d (0 store, 5 logits, 6 resid_fix, 8 swiglu_f16)", epi);
  }
}

// QKV of the fp16 batched path (T <= 32) with bias, RoPE and the K/V write in the product's epilogue.
extern "C" int q355_gemm_f16_qkv_rope(const uint8_t* qs, const void* d, int N, int K, const void* xh, int T,
                                     const float* bias, const float* rope_cos, const float* rope_sin,
                                     const int32_t* pos, const int32_t* block_table, int bt_stride, int seq_stride,
                                     void* kcache, void* vcache, void* qout, int nh, int nkv, void* stream) {
  if (int e = check_mat("gemm_f16_qkv_rope", qs, d, N, K)) return e;
  REQUIRE(xh && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "gemm_f16_qkv_rope: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && N == (nh + 2 * nkv) * HD, "gemm_f16_qkv_rope: N=%d must be (nh + 2 nkv) * 128", N);
  REQUIRE(T >= 1 && T <= 32 && K <= 1536 && bt_stride > 0 && (seq_stride == 0 || seq_stride == 1),
          "gemm_f16_qkv_rope: T=%d K=%d bt_stride=%d seq_stride=%d (T <= 32, K <= 1536)", T, K, bt_stride, seq_stride);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xh = (const __half*)xh;
  a.aux = bias; a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.nh = nh; a.nkv = nkv;
  const int r = T <= 16 ? launch_gemm_f16r_tg<1, EPI_QKV>(a, (hipStream_t)stream)
                        : launch_gemm_f16r_tg<2, EPI_QKV>(a, (hipStream_t)stream);
  return r >= 0 ? r : fail(Q355_EINVAL, "gemm_f16_qkv_rope: unsupported shape N=%d K=%d", N, K);
}

extern "C" int q355_rmsnorm_fix_f16(const int64_t* h, const float* w, void* xh, int T, int H, double eps,
                                    void* stream) {
  REQUIRE(h && w && xh, "rmsnorm_fix_f16: null pointer");
  REQUIRE(T >= 1 && H % 8 == 0 && H / 8 <= 256, "rmsnorm_fix_f16: T=%d H=%d", T, H);
  hipLaunchKernelGGL(k_rmsnorm_fix_f16, dim3(T), dim3(256), 0, (hipStream_t)stream, (const long long*)h, w,
                     (__half*)xh, H, eps);
  return launched("rmsnorm_fix_f16");
}

extern "C" int q355_qkv_finish(int64_t* acc, const float* bias, const float* rope_cos, const float* rope_sin,
                               const int32_t* pos, const int32_t* block_table, int bt_stride, int seq_stride,
                               void* kcache, void* vcache, void* qout, int nh, int nkv, int T, void* stream) {
  REQUIRE(acc && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "qkv_finish: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && T > 0 && bt_stride > 0 && (seq_stride == 0 || seq_stride == 1),
          "qkv_finish: nh=%d nkv=%d T=%d bt_stride=%d seq_stride=%d", nh, nkv, T, bt_stride, seq_stride);
  GemvArgs a = {};
  a.aux = bias; a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.nh = nh; a.nkv = nkv;
  hipLaunchKernelGGL(k_qkv_finish, dim3(T), dim3(256), 0, (hipStream_t)stream, a, (long long*)acc);
  return launched("qkv_finish");
}

// QKV product with the finish fused into its epilogue: every output has one writer (no K split), so no int64
// accumulator and no second launch. Decode batches (T <= 32, K <= 1536) run the register-resident kernel,
// larger T the LDS-tiled one.
extern "C" int q355_mmq_qkv_rope(const uint8_t* qs, const void* d, int N, int K, const int8_t* xq, const void* xds,
                                 int T, const float* bias, const float* rope_cos, const float* rope_sin,
                                 const int32_t* pos, const int32_t* block_table, int bt_stride, int seq_stride,
                                 void* kcache, void* vcache, void* qout, double* q64, int nh, int nkv,
                                 void* stream) {
  if (int e = check_mat("mmq_qkv_rope", qs, d, N, K)) return e;
  REQUIRE(xq && xds && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "mmq_qkv_rope: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && N == (nh + 2 * nkv) * HD && N % 128 == 0,
          "mmq_qkv_rope: N=%d must be (nh + 2 nkv) * 128 = %d and a multiple of 128", N, (nh + 2 * nkv) * HD);
  REQUIRE(T >= 1 && T <= 65535 * 64 && bt_stride > 0 && (seq_stride == 0 || seq_stride == 1),
          "mmq_qkv_rope: T=%d bt_stride=%d seq_stride=%d", T, bt_stride, seq_stride);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T; a.xq = xq; a.xds = (const half2*)xds;
  a.aux = bias; a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.qout64 = q64;
  a.nh = nh; a.nkv = nkv;
  if (T <= 32) {                                     // decode batches: register-resident, all tokens per workgroup
    const int r = T <= 16 ? launch_mmq_r_tg<1, EPI_QKV, false>(a, (hipStream_t)stream)
                          : launch_mmq_r_tg<2, EPI_QKV, false>(a, (hipStream_t)stream);
    if (r >= 0) return r;
  }
  return launch_mmq_big<EPI_QKV>(a, (hipStream_t)stream);
}

extern "C" int64_t q355_attn_prefill_ws_bytes(int P, int max_ctx, int nh, int nkv) {
  if (P < 1 || max_ctx < P || nh < 1 || nkv < 1 || nh % nkv) return -1;
  return (int64_t)(pf_ws_floats((P + PF_QB - 1) / PF_QB, nkv, nh / nkv, pf_max_splits(0, max_ctx)) * sizeof(float));
}

// compute units of the current device (the persistent prefill attention's workgroups), cached per device
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 256;
  return cus[dev];
}

static int attn_prefill(const void* q, const void* kcache, const void* vcache, const int32_t* block_table, int pos0,
                        int P, int nh, int nkv, float scale, float* out, int8_t* oq, void* ods, void* ws,
                        int64_t ws_bytes, hipStream_t stream) {
  REQUIRE(q && kcache && vcache && block_table && (out || (oq && ods)), "attn_prefill: null pointer");
  REQUIRE(P >= 1 && pos0 >= 0, "attn_prefill: P=%d pos0=%d", P, pos0);
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv >= 4 && nh / nkv <= 8 && nkv <= 65535,
          "attn_prefill: nh=%d nkv=%d (4 to 8 query heads per KV head)", nh, nkv);
  PrefillAttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.block_table = block_table; a.pos0 = pos0; a.P = P; a.nh = nh; a.nkv = nkv; a.scale = scale; a.out = out;
  a.oq = oq; a.ods = (half2*)ods;
  const int G = nh / nkv, nqb = (P + PF_QB - 1) / PF_QB;
  const dim3 block(64 * (G + PF_STAGERS));
  if (ws) {
    // the persistent form: items balanced over one workgroup per CU, at most PF_MAX_ROUNDS each; where every
    // row is one item and they fit one round, there is nothing to balance and the per-row kernel starts sooner
    const int items = pf_items(pos0, P, nkv);
    const int W = items < device_cus() ? items : device_cus();
    const bool balance = pf_max_splits(pos0, P) > 1 || items > W;
    if (balance && (items + W - 1) / W <= PF_MAX_ROUNDS) {
      a.max_splits = pf_max_splits(pos0, P);
      const int64_t need = (int64_t)(pf_ws_floats(nqb, nkv, G, a.max_splits) * sizeof(float));
      REQUIRE(ws_bytes >= need, "attn_prefill: workspace of %lld bytes, %lld needed for pos0 + P = %d",
              (long long)ws_bytes, (long long)need, pos0 + P);
      a.ws = (float*)ws;
      a.n_items = items;
      if (block.x <= 512) hipLaunchKernelGGL(k_attn_prefill_pers<512>, dim3(W), block, 0, stream, a);
      else hipLaunchKernelGGL(k_attn_prefill_pers<640>, dim3(W), block, 0, stream, a);
      return launched("attn_prefill");
    }
  }
  // one workgroup per (query block, KV head) with all its keys
  const dim3 grid(nqb, 1, nkv);
  if (block.x <= 512) hipLaunchKernelGGL(k_attn_prefill<512>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(k_attn_prefill<640>, grid, block, 0, stream, a);
  return launched("attn_prefill");
}

extern "C" int q355_attn_prefill(const void* q, const void* kcache, const void* vcache, const int32_t* block_table,
                                 int pos0, int P, int nh, int nkv, float scale, float* out, void* ws,
                                 int64_t ws_bytes, void* stream) {
  REQUIRE(out, "attn_prefill: null output");
  return attn_prefill(q, kcache, vcache, block_table, pos0, P, nh, nkv, scale, out, nullptr, nullptr, ws, ws_bytes,
                      (hipStream_t)stream);
}

extern "C" int q355_attn_prefill_q8_1(const void* q, const void* kcache, const void* vcache,
                                      const int32_t* block_table, int pos0, int P, int nh, int nkv, float scale,
                                      int8_t* oq, void* ods, void* ws, int64_t ws_bytes, void* stream) {
  REQUIRE(oq && ods, "attn_prefill_q8_1: null output");
  return attn_prefill(q, kcache, vcache, block_table, pos0, P, nh, nkv, scale, nullptr, oq, ods, ws, ws_bytes,
                      (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------------------
// Persistent decode step (batch 1).
extern "C" int64_t q355_mega_ws_bytes(int max_chunks, int L) { return (int64_t)mega_ws_bytes(max_chunks, L); }
extern "C" int q355_mega_layer_bytes(void) { return (int)sizeof(MegaLayer); }

static constexpr size_t MEGA_LDS = (size_t)MG_FFN + 2 * (MG_FFN / 32) * 4 > (3 * HD + 24 + 12 * HD) * 8
                                       ? (size_t)MG_FFN + 2 * (MG_FFN / 32) * 4 : (size_t)(3 * HD + 24 + 12 * HD) * 8;

extern "C" int q355_mega_decode(const void* layers, int L, const uint8_t* emb_qs, const void* emb_d, const float* norm,
                                int V, const float* rope_cos, const float* rope_sin, const int32_t* block_table,
                                int max_chunks, double eps, int32_t* tok, int32_t* pos, int64_t* h, float* logits,
                                void* ws, int64_t spin_limit_us, void* stream) {
  REQUIRE(layers && emb_qs && emb_d && norm && rope_cos && rope_sin && block_table && tok && pos && h && ws,
          "mega_decode: null pointer");
  REQUIRE(L >= 1 && L <= 256, "mega_decode: L=%d", L);
  REQUIRE(V > 0 && V % 16 == 0 && V / 16 >= MG_NWG, "mega_decode: V=%d (multiple of 16, >= %d)", V, 16 * MG_NWG);
  REQUIRE(max_chunks >= 1 && max_chunks <= 64, "mega_decode: max_chunks=%d (1..64)", max_chunks);
  REQUIRE(spin_limit_us > 0, "mega_decode: spin_limit_us=%lld", (long long)spin_limit_us);
  // all MG_NWG workgroups must be resident at once (they wait on each other)
  static int checked_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(Q355_EINVAL, "mega_decode: no device");
  if (checked_dev != dev) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_mega_decode, MG_NTH, MEGA_LDS) != hipSuccess)
      return fail(Q355_EINVAL, "mega_decode: device query failed");
    REQUIRE((long)cus * per_cu >= MG_NWG, "mega_decode: %d CUs x %d resident workgroups < %d", cus, per_cu, MG_NWG);
    checked_dev = dev;
  }
  MegaArgs a = {};
  a.layers = (const MegaLayer*)layers; a.L = L;
  a.emb_qs = emb_qs; a.emb_d = (const __half*)emb_d; a.norm = norm; a.V = V;
  a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.block_table = block_table; a.max_chunks = max_chunks;
  a.eps = eps; a.scale = 1.0 / sqrt((double)HD);
  a.tok = tok; a.pos = pos; a.h = (long long*)h; a.logits = logits;
  a.ws = (char*)ws; a.spin_limit = spin_limit_us * 100;      // wall_clock64 runs at 100 MHz
  hipLaunchKernelGGL(k_mega_decode, dim3(MG_NWG), dim3(MG_NTH), MEGA_LDS, (hipStream_t)stream, a);
  return launched("mega_decode");
}

// Measurement only (bench.py): read `bytes` (a multiple of 16) from p once, streaming; no output.
extern "C" int q355_stream_read(const void* p, int64_t bytes, void* stream) {
  REQUIRE(p && bytes > 0 && bytes % 16 == 0, "stream_read: p=%p bytes=%lld", p, (long long)bytes);
  const long n16 = (long)(bytes / 16);
  hipLaunchKernelGGL(k_stream_read, dim3((unsigned)((n16 + 4095) / 4096)), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)p, n16, (unsigned*)nullptr);
  return launched("stream_read");
}
