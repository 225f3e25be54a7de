// Shared device helpers for the gfx950 (CDNA4) Qwen2.5 Q4_0 hot path.
//
// Device formats (one layout for every kernel of the library):
//   Q4_0 matrix W [N, K] (N % 16 == 0, K % 32 == 0), "16-row tiled planes":
//     qs  uint8 [N/16][K/32][16 rows][16 B]   the GGUF qs bytes of each block, unchanged: byte i holds
//                                             weight i (low nibble) and weight i+16 (high nibble), stored 0..15
//     d   fp16  [N/16][K/32][16 rows]         the GGUF block scale; value = d * (q - 8)
//   For a fixed (tile, block) the 16 rows' nibbles are 256 contiguous bytes, so one wave64 load of
//   16 B per lane (16 rows x 4 consecutive blocks) reads 1 KB contiguous, and the same bytes form the
//   A operand of v_mfma_i32_16x16x32_i8 (lane = row, 8 bytes per k-group).
//   Q8_1 activations X [T, K]:
//     xq  int8  [T][K]
//     xds half2 [T][K/32] = (d, s): d = fp16(amax/127), s = fp16(d * sum q) (llama.cpp block_q8_1 fields;
//                                  the quantizer rule is q8_code's)
//   Kernels use the exact integer block correction dot - 8 * sum(q) (sum recomputed from xq), not s.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <type_traits>

#define Q355_QK 32
#define Q355_WAVE 64

namespace q355 {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal hint: weights are read once per step).
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 ld_stream8(const void* p) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  u32x2 v = __builtin_nontemporal_load((const u32x2*)p);
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ unsigned ld_stream4(const void* p) { return __builtin_nontemporal_load((const unsigned*)p); }
__device__ __forceinline__ unsigned ld_stream2(const void* p) { return __builtin_nontemporal_load((const unsigned short*)p); }

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Exact int32 dot of one Q4_0 block (16 B of GGUF qs, unsigned nibbles 0..15) with 32 int8 values.
__device__ __forceinline__ int q4_block_dot(const uint4 w, const int* x) {
  int acc = 0;
  acc = dot4((int)(w.x & 0x0F0F0F0Fu), x[0], acc);
  acc = dot4((int)(w.y & 0x0F0F0F0Fu), x[1], acc);
  acc = dot4((int)(w.z & 0x0F0F0F0Fu), x[2], acc);
  acc = dot4((int)(w.w & 0x0F0F0F0Fu), x[3], acc);
  acc = dot4((int)((w.x >> 4) & 0x0F0F0F0Fu), x[4], acc);
  acc = dot4((int)((w.y >> 4) & 0x0F0F0F0Fu), x[5], acc);
  acc = dot4((int)((w.z >> 4) & 0x0F0F0F0Fu), x[6], acc);
  acc = dot4((int)((w.w >> 4) & 0x0F0F0F0Fu), x[7], acc);
  return acc;
}

// One 32-weight block of the Q6_K planes against 32 int8 values: v = lo | hi << 4 in 0..63, weight value
// sc[i / 16] * (v - 32); returns sum over the two 16-weight sub-blocks of sc_s * (dot_s - 32 sum x_s)
// (exact int32; the caller scales by the super-block d and the activation d).
// lo byte i holds v_i & 15 (bits 0-3) and v_{i+16} & 15 (bits 4-7); hi byte b holds v_{b+8j} >> 4 at bits 2j.
__device__ __forceinline__ int q6k_block_isum(const uint4 w, const uint2 h, unsigned sc, const int* x) {
  const unsigned M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
  int d0 = 0, d1 = 0, s0 = 0, s1 = 0;
  d0 = dot4((int)((w.x & M4) | ((h.x & M2) << 4)), x[0], d0);
  d0 = dot4((int)((w.y & M4) | ((h.y & M2) << 4)), x[1], d0);
  d0 = dot4((int)((w.z & M4) | (((h.x >> 2) & M2) << 4)), x[2], d0);
  d0 = dot4((int)((w.w & M4) | (((h.y >> 2) & M2) << 4)), x[3], d0);
  d1 = dot4((int)(((w.x >> 4) & M4) | (((h.x >> 4) & M2) << 4)), x[4], d1);
  d1 = dot4((int)(((w.y >> 4) & M4) | (((h.y >> 4) & M2) << 4)), x[5], d1);
  d1 = dot4((int)(((w.z >> 4) & M4) | (((h.x >> 6) & M2) << 4)), x[6], d1);
  d1 = dot4((int)(((w.w >> 4) & M4) | (((h.y >> 6) & M2) << 4)), x[7], d1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s0 = dot4(x[i], 0x01010101, s0);
    s1 = dot4(x[4 + i], 0x01010101, s1);
  }
  const int c0 = (int)(signed char)(sc & 255), c1 = (int)(signed char)((sc >> 8) & 255);
  return c0 * (d0 - 32 * s0) + c1 * (d1 - 32 * s1);
}

__device__ __forceinline__ int sum_i8x32(const int* x) {
  int s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) s = dot4(x[i], 0x01010101, s);
  return s;
}

// DPP lane exchanges (no LDS traffic): quad_perm xor 1 / xor 2, half-row mirror, row mirror.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
constexpr int DPP_ROR8 = 0x128;                     // row_ror:8: lane l of a 16-lane row takes lane l ^ 8's value
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
// Reductions over aligned groups of 4 lanes (every lane of the group gets the result).
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  return fmaxf(v, dpp<DPP_XOR2>(v));
}
__device__ __forceinline__ int quad_isum(int v) {
  v += dpp<DPP_XOR1>(v);
  return v + dpp<DPP_XOR2>(v);
}
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<DPP_XOR1>(v);
  return v + dpp<DPP_XOR2>(v);
}
// v + v(lane ^ 16) and v + v(lane ^ 32) with the gfx950 cross-row lane swaps (v_permlane16_swap /
// v_permlane32_swap) instead of an LDS permute: each lane adds its own value and its partner's, in either
// order, which is the same IEEE sum.
__device__ __forceinline__ float xsum16(float v) {
  const unsigned u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float v) {
  const unsigned u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ double xsum16_d(double v) {
  const int2 x = __builtin_bit_cast(int2, v);
  const auto lo = __builtin_amdgcn_permlane16_swap(x.x, x.x, false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(x.y, x.y, false, false);
  return __builtin_bit_cast(double, make_int2(lo[0], hi[0])) + __builtin_bit_cast(double, make_int2(lo[1], hi[1]));
}
__device__ __forceinline__ double xsum32_d(double v) {
  const int2 x = __builtin_bit_cast(int2, v);
  const auto lo = __builtin_amdgcn_permlane32_swap(x.x, x.x, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap(x.y, x.y, false, false);
  return __builtin_bit_cast(double, make_int2(lo[0], hi[0])) + __builtin_bit_cast(double, make_int2(lo[1], hi[1]));
}
// (value, index) argmax over the 64 lanes, larger value first and the lower index on ties (a total order, so
// the pairing pattern does not matter): DPP steps inside each row of 16, then the two cross-row lane swaps.
// Every lane ends with the result. All 64 lanes must be active.
__device__ __forceinline__ void amax_take(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
template <int CTRL>
__device__ __forceinline__ void amax_dpp(float& v, int& i) {
  amax_take(v, i, dpp<CTRL>(v), dpp<CTRL>(i));
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  amax_dpp<DPP_XOR1>(v, i);
  amax_dpp<DPP_XOR2>(v, i);
  amax_dpp<DPP_HALF_MIRROR>(v, i);
  amax_dpp<DPP_MIRROR>(v, i);
  {
    const unsigned u = __float_as_uint(v);
    const auto rv = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    const bool lo = (__lane_id() & 16) == 0;                     // own value in slot 0 (rows 0, 2), else 1
    amax_take(v, i, __uint_as_float(lo ? rv[1] : rv[0]), (int)(lo ? ri[1] : ri[0]));
  }
  {
    const unsigned u = __float_as_uint(v);
    const auto rv = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    const bool lo = __lane_id() < 32;
    amax_take(v, i, __uint_as_float(lo ? rv[1] : rv[0]), (int)(lo ? ri[1] : ri[0]));
  }
}
// Full wave64 sum: 4 DPP steps inside each row of 16, then two cross-row exchanges.
__device__ __forceinline__ float wave_sum_fast(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_MIRROR>(v);
  v = xsum16(v);
  return xsum32(v);
}

// Q8_1 rule of every quantizer in the library (and of the oracle): the reference's QUANT_Q8
// (lab/qwen_batched.py:1032-1033): d = amax / 127 and q = x / d, both IEEE fp32 divisions, q rounded half to
// even (__float2int_rn), q = 0 when d == 0. |x / d| <= 127 (1 + 2^-23), so no clamp is needed. The block is
// stored in llama.cpp's block_q8_1 form: d as fp16 (the scale every product uses) and s = fp16(d * sum q)
// with the fp32 d (llama.cpp quantize_row_q8_1).
__device__ __forceinline__ float q8_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ int q8_code(float x, float d32) {
  const float dv = d32 != 0.0f ? d32 : 1.0f;   // branch-free: a dead block divides by 1 and selects 0
  const int q = (int)__builtin_rintf(x / dv);
  return d32 != 0.0f ? q : 0;
}
__device__ __forceinline__ __half q8_s16(float d32, int sq) { return __float2half_rn(d32 * (float)sq); }

// f64 -> fp16 with ONE round to nearest even (no intermediate fp32 rounding, which can land exactly on an
// fp16 midpoint and then break the tie the other way).
__device__ __forceinline__ __half half_rn(double v) {
  const _Float16 h = (_Float16)v;
  return *reinterpret_cast<const __half*>(&h);
}

// Q8_1 of 8 consecutive values held by one lane; 4 lanes form a 32-block (lane groups aligned to 4).
// Returns the 8 int8 packed in a uint2; df = the fp16 d as float, sq = the block's sum of q, d32 = the fp32 d.
__device__ __forceinline__ uint2 q8_1_x8(const float (&x)[8], float& df, int& sq, float& d32) {
  float amax = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) amax = fmaxf(amax, fabsf(x[u]));
  amax = quad_max(amax);
  d32 = q8_scale(amax);
  df = __half2float(__float2half_rn(d32));
  int q[8];
  int s = 0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    q[u] = q8_code(x[u], d32);
    s += q[u];
  }
  sq = quad_isum(s);
  uint2 pk;
  pk.x = (q[0] & 255) | ((q[1] & 255) << 8) | ((q[2] & 255) << 16) | ((unsigned)(q[3] & 255) << 24);
  pk.y = (q[4] & 255) | ((q[5] & 255) << 8) | ((q[6] & 255) << 16) | ((unsigned)(q[7] & 255) << 24);
  return pk;
}
__device__ __forceinline__ uint2 q8_1_x8(const float (&x)[8], float& df, int& sq) {
  float d32;
  return q8_1_x8(x, df, sq, d32);
}

// f64 wave reductions (the batch-1 decode path accumulates in f64 so that every Q8_1 quantizer input
// agrees with the f64 oracle to ~1e-14; CDNA4 runs f64 FMA at the fp32 vector rate). DPP steps inside each
// 16-lane row (xor 1, xor 2, half-row mirror, row mirror: every lane of the row ends with the row's result),
// then the four row results are read as scalars and combined in a fixed order: no LDS round trips, and
// every lane gets the bitwise same value. All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  int2 x = *reinterpret_cast<int2*>(&v);
  x.x = __builtin_amdgcn_mov_dpp(x.x, CTRL, 0xF, 0xF, true);
  x.y = __builtin_amdgcn_mov_dpp(x.y, CTRL, 0xF, 0xF, true);
  return *reinterpret_cast<double*>(&x);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  int2 x = *reinterpret_cast<int2*>(&v);
  x.x = __builtin_amdgcn_readlane(x.x, l);
  x.y = __builtin_amdgcn_readlane(x.y, l);
  return *reinterpret_cast<double*>(&x);
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_d<DPP_XOR1>(v);
  v += dpp_d<DPP_XOR2>(v);
  v += dpp_d<DPP_HALF_MIRROR>(v);
  v += dpp_d<DPP_MIRROR>(v);
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
__device__ __forceinline__ double wave_max_d(double v) {
  v = fmax(v, dpp_d<DPP_XOR1>(v));
  v = fmax(v, dpp_d<DPP_XOR2>(v));
  v = fmax(v, dpp_d<DPP_HALF_MIRROR>(v));
  v = fmax(v, dpp_d<DPP_MIRROR>(v));
  return fmax(fmax(readlane_d(v, 0), readlane_d(v, 16)), fmax(readlane_d(v, 32), readlane_d(v, 48)));
}

// Wave64 reductions (xor butterfly over all 64 lanes, or over `width` lanes).
template <int WIDTH = 64>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int WIDTH = 64>
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int WIDTH = 64>
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Reductions over aligned 32-lane groups: four DPP steps inside each 16-lane row, then one exchange
// between the two rows of the group (every lane of the group gets the result).
__device__ __forceinline__ float g32_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp<DPP_MIRROR>(v));
  return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ int g32_isum(int v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_MIRROR>(v);
  return v + __shfl_xor(v, 16, 64);
}

// Q8_1 of one value inside a group of 32 lanes that hold one block (lane group aligned to 32), by the rule
// of q8_code. Returns q; writes (d, s) through `ds` from the group's first lane.
__device__ __forceinline__ int q8_1_lane32(float x, half2* ds, bool leader) {
  const float d32 = q8_scale(g32_max(fabsf(x)));
  const int q = q8_code(x, d32);
  const int sq = g32_isum(q);
  if (leader) *ds = __halves2half2(__float2half_rn(d32), q8_s16(d32, sq));
  return q;
}

// Reductions over the 4 lanes l % 16 + 16 g (the MFMA accumulator column) with gfx950's permlane swaps, no
// LDS round trip: v_permlane16_swap / v_permlane32_swap of a register with itself leave lane l holding
// {x[l], x[l ^ 16]} (resp. {x[l], x[l ^ 32]}) in the two results, in either order, so the max or sum of the
// pair is the xor-partner reduction.
__device__ __forceinline__ float col4_max(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float col4_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int col4_isum(int v) {
  auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = (int)r[0] + (int)r[1];
  r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return (int)r[0] + (int)r[1];
}

// Device-coherent relaxed accesses (agent scope): stores reach the memory every XCD reads and loads bypass
// the non-coherent caches, so workgroups on different XCDs can exchange data without cache maintenance.
template <typename T>
__device__ __forceinline__ T ldc(const T* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <typename T>
__device__ __forceinline__ void stc(T* p, T v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }


// 16-byte device-scope loads (buffer loads with the sc1 policy, as the relaxed agent-scope atomic loads use):
// coherent with other CUs' device-scope stores, four times the width of ldc, ordinary wait-count tracking
// The base address must be the same in every lane of the wave (it is moved to scalar registers; a per-lane
// base would make the compiler loop over the distinct values one load at a time).
struct Coh16 {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ static void* uniform(const void* p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v), hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (void*)(((unsigned long long)hi << 32) | lo);
  }
  __device__ __forceinline__ Coh16(const void* p, unsigned bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(uniform(p), 0, (int)bytes, 0x00020000)) {}
  __device__ __forceinline__ int4 ld(unsigned byte_off) const {
    return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 16));
  }
  __device__ __forceinline__ unsigned ld4(unsigned byte_off) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 16);
  }
  // 2- and 16-byte device-scope stores (the sc1 policy of the relaxed agent-scope atomic stores)
  __device__ __forceinline__ void st2(unsigned byte_off, unsigned short v) const {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, (int)byte_off, 0, 16);
  }
  __device__ __forceinline__ void st16(unsigned byte_off, int4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), r,
                                           (int)byte_off, 0, 16);
  }
};

}  // namespace q355
