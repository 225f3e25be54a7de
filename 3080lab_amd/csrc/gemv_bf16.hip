// Reference-parity mode of the decode GEMV: Q4_0 weights x bf16 activations in fp32 (the arithmetic of the
// reference's gemv_source, lab/qwen_kernels.py:14-113: per 32-block y += d * sum_i fmaf(q_i - 8, x_i), fp32),
// for callers that want the reference's bf16 decode numerics instead of Q8_1 activations.
// Workgroup = one 16-row tile x all K (4 waves x 4 k-lanes = 16 k-lanes, KPL blocks per lane), T <= 4 tokens;
// the activations are staged in LDS as bf16; each lane converts nibbles to float (byte conversions) and runs 32
// fp32 FMAs per block; the 16 k-lane partial sums reduce in a fixed order (lanes, then waves).
#include "common.h"
#include "q355_kernels.h"

namespace q355 {

template <int T, int KPL, int EPI>
__global__ void __launch_bounds__(256) k_gemv_bf16(const uint8_t* __restrict__ qs8, const __half* __restrict__ d,
                                                   int N, int K, const unsigned short* __restrict__ x, float* y,
                                                   const float* bias) {
  extern __shared__ __align__(16) unsigned short xs[];       // [T][K] bf16
  __shared__ float part[4][T][16];
  const int nb = K / 32;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kl = wv * 4 + (lane >> 4);
  const int tile = blockIdx.x;
  const uint4* __restrict__ qs = (const uint4*)qs8;
  const unsigned short* __restrict__ dd = (const unsigned short*)d;
  uint4 w[KPL];
  unsigned dh[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int b = min(kl + 16 * i, nb - 1);
    const size_t idx = ((size_t)tile * nb + b) * 16 + r;
    w[i] = ld_stream16(qs + idx);
    dh[i] = dd[idx];
  }
  __asm__ __volatile__("" ::: "memory");
  for (int e = threadIdx.x; e < T * K / 8; e += 256) ((uint4*)xs)[e] = ((const uint4*)x)[e];
  __syncthreads();
  float acc[T];
#pragma unroll
  for (int j = 0; j < T; ++j) acc[j] = 0.f;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int b = kl + 16 * i;
    if (b < nb) {
      const float dw = __half2float(__ushort_as_half((unsigned short)dh[i]));
      const unsigned wb[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const unsigned short* xb = xs + (size_t)j * K + (size_t)b * 32;
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint4 x0 = *(const uint4*)(xb + 4 * k);            // weights 4k..4k+3 (low nibbles)
          const uint2 x1 = *(const uint2*)(xb + 16 + 4 * k);       // weights 16+4k.. (high nibbles)
          const unsigned xl[2] = {x0.x, x0.y}, xh[2] = {x1.x, x1.y};
          const unsigned lo = wb[k] & 0x0F0F0F0Fu, hi = (wb[k] >> 4) & 0x0F0F0F0Fu;
          // byte -> float (v_cvt_f32_ubyte0..3)
          const float ql[4] = {(float)(lo & 255u), (float)((lo >> 8) & 255u), (float)((lo >> 16) & 255u),
                               (float)(lo >> 24)};
          const float qh[4] = {(float)(hi & 255u), (float)((hi >> 8) & 255u), (float)((hi >> 16) & 255u),
                               (float)(hi >> 24)};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float xlo = __uint_as_float((u & 1 ? xl[u >> 1] & 0xFFFF0000u : xl[u >> 1] << 16));
            const float xhi = __uint_as_float((u & 1 ? xh[u >> 1] & 0xFFFF0000u : xh[u >> 1] << 16));
            s = fmaf(ql[u] - 8.f, xlo, s);
            s = fmaf(qh[u] - 8.f, xhi, s);
          }
        }
        acc[j] = fmaf(dw, s, acc[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < T; ++j) {
    float v = acc[j];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lane < 16) part[wv][j][r] = v;
  }
  __syncthreads();
  if (threadIdx.x < 16 * T) {
    const int j = threadIdx.x >> 4, rr = threadIdx.x & 15, row = tile * 16 + rr;
    const float v = ((part[0][j][rr] + part[1][j][rr]) + part[2][j][rr]) + part[3][j][rr];
    if (EPI == EPI_STORE) y[(size_t)j * N + row] = v;
    else if (EPI == EPI_RESID) y[(size_t)j * N + row] += v;
    else y[(size_t)j * N + row] = v + bias[row];
  }
}

}  // namespace q355
