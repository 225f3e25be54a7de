// C ABI of libqwen355.so: argument validation on the host, launch geometry, template dispatch.
#include <cstdio>
#include <cstring>
#include <cstdarg>

#include "../../include/qwen355.h"
#include "common.h"
#include "q355_kernels.h"

namespace q355 {
__global__ void k_quant_q8_1(const float*, int8_t*, half2*, long);
__global__ void k_rmsnorm_q8_1(const float*, const float*, int8_t*, half2*, int, float);
__global__ void k_embed_q4_0(const uint8_t*, const __half*, int, int, const int*, float*);
__global__ void k_finish(const float*, const int*, int, int*, int*);
__global__ void k_blockdots(const uint8_t*, int, int, const int8_t*, int, int*);
__global__ void k_attn_decode(const AttnArgs);
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
// GEMV dispatch over (T, NT, prologue, epilogue).
template <int PRO, int EPI, int NT>
static int launch_gemv_t(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  switch (a.T) {
    case 1: hipLaunchKernelGGL((k_gemv<1, NT, PRO, EPI>), grid, dim3(256), lds, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<2, NT, PRO, EPI>), grid, dim3(256), lds, s, a); break;
    case 3: hipLaunchKernelGGL((k_gemv<3, NT, PRO, EPI>), grid, dim3(256), lds, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemv<4, NT, PRO, EPI>), grid, dim3(256), lds, s, a); break;
    default: return fail(Q355_EINVAL, "gemv: T=%d outside 1..4", a.T);
  }
  return launched("gemv");
}

template <int PRO, int EPI>
static int launch_gemv_nt(const GemvArgs& a, int NT, int split, hipStream_t s) {
  const int tiles = a.N / 16;
  if (tiles % NT) return fail(Q355_EINVAL, "gemv: N/16=%d not a multiple of NT=%d", tiles, NT);
  dim3 grid(tiles / NT, split);
  size_t lds = (size_t)a.T * a.K + (size_t)a.T * (a.K / 32) * 8;
  switch (NT) {
    case 1: return launch_gemv_t<PRO, EPI, 1>(a, grid, lds, s);
    case 2: return launch_gemv_t<PRO, EPI, 2>(a, grid, lds, s);
    case 4: return launch_gemv_t<PRO, EPI, 4>(a, grid, lds, s);
    default: return fail(Q355_EINVAL, "gemv: NT=%d", NT);
  }
}

// Tiles per workgroup: enough workgroups to cover 256 CUs when the matrix allows it.
static int pick_nt(int N) {
  const int tiles = N / 16;
  if (tiles % 4 == 0 && tiles / 4 >= 512) return 4;
  if (tiles % 2 == 0 && tiles / 2 >= 512) return 2;
  return 1;
}

static int check_mat(const char* what, const void* qs, const void* d, int N, int K) {
  REQUIRE(qs && d, "%s: null weight pointer", what);
  REQUIRE(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", what, N);
  REQUIRE(K > 0 && K % 32 == 0 && K <= 8960, "%s: K=%d must be a multiple of 32 and <= 8960", what, K);
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
                                   const void* xds, int T, float* y, const float* bias, int epi, int split,
                                   void* stream) {
  if (int e = check_mat("gemv_q4_0_q8_1", qs, d, N, K)) return e;
  REQUIRE(xq && xds && y, "gemv_q4_0_q8_1: null pointer");
  REQUIRE(T >= 1 && T <= 4, "gemv_q4_0_q8_1: T=%d outside 1..4", T);
  REQUIRE(epi >= 0 && epi <= 2, "gemv_q4_0_q8_1: epi=%d (0 store, 1 resid, 2 bias)", epi);
  REQUIRE(epi != 2 || bias, "gemv_q4_0_q8_1: bias epilogue needs bias");
  REQUIRE(split >= 1 && split <= K / 32 && (split == 1 || epi == 1),
          "gemv_q4_0_q8_1: split=%d (1..K/32, >1 only with epi 1)", split);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.xq = xq; a.xds = (const half2*)xds; a.y = y; a.aux = bias;
  const int NT = pick_nt(N);
  hipStream_t s = (hipStream_t)stream;
  switch (epi) {
    case 0: return launch_gemv_nt<PRO_Q8, EPI_STORE>(a, NT, 1, s);
    case 1: return launch_gemv_nt<PRO_Q8, EPI_RESID>(a, NT, split, s);
    default: return launch_gemv_nt<PRO_Q8, EPI_BIAS>(a, NT, 1, s);
  }
}

extern "C" int q355_gemv_blockdots(const uint8_t* qs, int N, int K, const int8_t* xq, int T, int32_t* out,
                                   void* stream) {
  REQUIRE(qs && xq && out, "gemv_blockdots: null pointer");
  REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0 && T > 0, "gemv_blockdots: N=%d K=%d T=%d", N, K, T);
  hipLaunchKernelGGL(k_blockdots, dim3(1024), dim3(256), 0, (hipStream_t)stream, qs, N, K, xq, T, out);
  return launched("gemv_blockdots");
}

extern "C" int q355_qkv_rope_kv(const uint8_t* qs, const void* d, int K, const float* h, const float* nw, float eps,
                                const float* bias, const float* rope_cos, const float* rope_sin, const int32_t* pos,
                                const int32_t* block_table, int bt_stride, int seq_stride, void* kcache,
                                void* vcache, void* qout, int nh, int nkv, int T, void* stream) {
  const int N = (nh + 2 * nkv) * HD;
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 8, "qkv_rope_kv: nh=%d nkv=%d", nh, nkv);
  if (int e = check_mat("qkv_rope_kv", qs, d, N, K)) return e;
  REQUIRE(K <= 2048, "qkv_rope_kv: K=%d > 2048 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && bias && rope_cos && rope_sin && pos && block_table && kcache && vcache && qout,
          "qkv_rope_kv: null pointer");
  REQUIRE(T >= 1 && T <= 4, "qkv_rope_kv: T=%d outside 1..4", T);
  REQUIRE(bt_stride > 0 && (seq_stride == 0 || seq_stride == 1), "qkv_rope_kv: bt_stride=%d seq_stride=%d",
          bt_stride, seq_stride);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N; a.K = K; a.T = T;
  a.h = h; a.nw = nw; a.eps = eps; a.aux = bias;
  a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.pos = pos; a.block_table = block_table;
  a.bt_stride = bt_stride; a.seq_stride = seq_stride;
  a.kcache = (__half*)kcache; a.vcache = (__half*)vcache; a.qout = (__half*)qout; a.nh = nh; a.nkv = nkv;
  return launch_gemv_nt<PRO_RMS, EPI_QKV>(a, 1, 1, (hipStream_t)stream);
}

extern "C" int q355_ffn_gate_up(const uint8_t* qs, const void* d, int N2, int K, const float* h, const float* nw,
                                float eps, int8_t* mq, void* mds, int T, void* stream) {
  if (int e = check_mat("ffn_gate_up", qs, d, N2, K)) return e;
  REQUIRE(N2 % 64 == 0, "ffn_gate_up: N2=%d must be a multiple of 64 (32 SwiGLU outputs per block)", N2);
  REQUIRE(K <= 2048, "ffn_gate_up: K=%d > 2048 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && mq && mds, "ffn_gate_up: null pointer");
  REQUIRE(T >= 1 && T <= 4, "ffn_gate_up: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = N2; a.K = K; a.T = T;
  a.h = h; a.nw = nw; a.eps = eps; a.oq = mq; a.ods = (half2*)mds;
  return launch_gemv_nt<PRO_RMS, EPI_SWIGLU_Q8>(a, 4, 1, (hipStream_t)stream);
}

extern "C" int q355_head_nparts(int V) { return V / 64; }

extern "C" int q355_head_logits(const uint8_t* qs, const void* d, int V, int K, const float* h, const float* nw,
                                float eps, float* logits, float* pmax, int32_t* pidx, int T, void* stream) {
  if (int e = check_mat("head_logits", qs, d, V, K)) return e;
  REQUIRE(V % 64 == 0, "head_logits: V=%d must be a multiple of 64", V);
  REQUIRE(K <= 2048, "head_logits: K=%d > 2048 (fused RMSNorm prologue)", K);
  REQUIRE(h && nw && logits && pmax && pidx, "head_logits: null pointer");
  REQUIRE(T >= 1 && T <= 4, "head_logits: T=%d outside 1..4", T);
  GemvArgs a = {};
  a.qs = qs; a.d = (const __half*)d; a.N = V; a.K = K; a.T = T;
  a.h = h; a.nw = nw; a.eps = eps; a.y = logits; a.pmax = pmax; a.pidx = pidx;
  return launch_gemv_nt<PRO_RMS, EPI_LOGITS>(a, 4, 1, (hipStream_t)stream);
}

extern "C" int q355_finish(const float* pmax, const int32_t* pidx, int nparts, int32_t* tok, int32_t* pos, int T,
                           void* stream) {
  REQUIRE(pmax && pidx && tok && pos, "finish: null pointer");
  REQUIRE(nparts > 0 && T > 0, "finish: nparts=%d T=%d", nparts, T);
  hipLaunchKernelGGL(k_finish, dim3(T), dim3(256), 0, (hipStream_t)stream, pmax, pidx, nparts, tok, pos);
  return launched("finish");
}

extern "C" int q355_embed_q4_0(const uint8_t* qs, const void* d, int V, int H, const int32_t* tok, float* h, int T,
                               void* stream) {
  if (int e = check_mat("embed_q4_0", qs, d, V, H)) return e;
  REQUIRE(tok && h && T > 0, "embed_q4_0: null pointer or T=%d", T);
  hipLaunchKernelGGL(k_embed_q4_0, dim3(T), dim3(64), 0, (hipStream_t)stream, qs, (const __half*)d, V, H, tok, h);
  return launched("embed_q4_0");
}

extern "C" int q355_attn_decode(const void* q, const void* kcache, const void* vcache, const int32_t* pos,
                                const int32_t* block_table, int bt_stride, int nh, int nkv, int max_chunks,
                                float scale, float* part, uint32_t* counter, int8_t* oq, void* ods, float* o32, int T,
                                void* stream) {
  REQUIRE(q && kcache && vcache && pos && block_table && part && counter && oq && ods, "attn_decode: null pointer");
  REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && nh / nkv <= 8, "attn_decode: nh=%d nkv=%d", nh, nkv);
  REQUIRE(max_chunks > 0 && max_chunks <= bt_stride, "attn_decode: max_chunks=%d bt_stride=%d", max_chunks, bt_stride);
  REQUIRE(T > 0 && T <= 65535, "attn_decode: T=%d", T);
  AttnArgs a = {};
  a.q = (const __half*)q; a.kcache = (const __half*)kcache; a.vcache = (const __half*)vcache;
  a.pos = pos; a.block_table = block_table; a.bt_stride = bt_stride; a.nh = nh; a.nkv = nkv;
  a.max_chunks = max_chunks; a.scale = scale; a.part = part; a.counter = counter;
  a.oq = oq; a.ods = (half2*)ods; a.o32 = o32;
  hipLaunchKernelGGL(k_attn_decode, dim3(nkv * max_chunks, T), dim3(256), 0, (hipStream_t)stream, a);
  return launched("attn_decode");
}
