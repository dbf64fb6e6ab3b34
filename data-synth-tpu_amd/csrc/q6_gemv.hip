// Decode-fused skinny GEMM for packed Q6_K projections: y = x @ decode(W)^T.
//
// Replaces the Pallas kernel packed_q6_k_projection (kaggle/packed_q6/kernel.py:65-148).
// Each wave decodes a 16-row x 256-K unit of the SoA tile straight into MFMA
// A operands (no LDS round trip, no materialised weights) and multiplies it
// with up to 16*NT tokens on v_mfma_f32_16x16x32_bf16 (FP32 accumulation).
// The K blocks of a 16-row group are spread over the waves of one workgroup
// and reduced through LDS in a fixed wave order, so results are deterministic.
#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

// Eight BF16 x values for lane (token row ``xr``) at element ``col`` of a row,
// zero beyond ``k`` (the reference zero-pads x to whole 256-blocks).
__device__ __forceinline__ u32x4 load_x8(const uint16_t* xr, int col, int k, int vec) {
  if (vec && col + 8 <= k) return *reinterpret_cast<const u32x4*>(xr + col);
  u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t e = (col + i < k) ? (uint32_t)xr[col + i] : 0u;
    v[i >> 1] |= e << (16 * (i & 1));
  }
  return v;
}

template <int NT>
__global__ void __launch_bounds__(512) q6_skinny_kernel(const uint16_t* __restrict__ x, int m, int k,
                                                        int64_t ldx, int xvec,
                                                        const uint8_t* __restrict__ data,
                                                        const uint8_t* __restrict__ scales, int n,
                                                        int kb_count, int kw, void* __restrict__ y,
                                                        int ybf16, int64_t ldy) {
  __shared__ float red[8][NT][256];
  const int rgg = blockIdx.x;
  const int tile = rgg >> 2, rg = rgg & 3;
  const int m0 = blockIdx.y * 16 * NT;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int row = rg * 16 + j;

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = wave; kb < kb_count; kb += kw) {
    const int64_t t = (int64_t)tile * kb_count + kb;
    Q6Raw raw;
    q6_load(raw, data + t * kTileBytes, scales + t * 128, row, jA);
    u32x4 xf[NT][8];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int gm = m0 + nt * 16 + j;
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        xf[nt][f] = gm < m ? load_x8(x + (int64_t)gm * ldx, kb * kQK + q6_xfrag_offset(f, jA), k, xvec)
                           : u32x4{0u, 0u, 0u, 0u};
      }
    }
    u32x4 a[8];
    q6_decode_unit(raw, jA, a);
#pragma unroll
    for (int f = 0; f < 8; ++f) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16(a[f], xf[nt][f], acc[nt]);
    }
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][nt][lane * 4 + i] = acc[nt][i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < NT * 256; idx += blockDim.x) {
    const int nt = idx >> 8, e = idx & 255;
    float s = 0.f;
    for (int w = 0; w < kw; ++w) s += red[w][nt][e];
    const int ln = e >> 2, i = e & 3;
    const int gn = tile * kTileRows + rg * 16 + 4 * (ln >> 4) + i;
    const int gm = m0 + nt * 16 + (ln & 15);
    if (gn < n && gm < m) {
      if (ybf16)
        reinterpret_cast<uint16_t*>(y)[(int64_t)gm * ldy + gn] = bf16_bits(s);
      else
        reinterpret_cast<float*>(y)[(int64_t)gm * ldy + gn] = s;
    }
  }
}

}  // namespace q6moe

using namespace q6moe;

extern "C" int q6moe_q6_matmul(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                               const uint8_t* data, const uint8_t* scales, int64_t n, void* y,
                               int y_dtype, int64_t ldy, void* stream) {
  Q6MOE_REQUIRE(x && data && scales && y, "q6_matmul: null pointer");
  Q6MOE_REQUIRE(m >= 1 && k >= 1 && n >= 1, "q6_matmul: x must be a nonempty [M,K] array");
  Q6MOE_REQUIRE(ldx >= k && ldy >= n, "q6_matmul: leading dimensions too small");
  Q6MOE_REQUIRE(m <= (1 << 30) && k <= (1 << 30) && n <= (1 << 30), "q6_matmul: dimension too large");
  Q6MOE_REQUIRE(y_dtype == Q6MOE_F32 || y_dtype == Q6MOE_BF16, "q6_matmul: y dtype must be F32 or BF16");
  Q6MOE_REQUIRE(aligned(data, 16) && aligned(scales, 2) && aligned(x, 2),
                "q6_matmul: data must be 16-byte aligned");
  const int kb = (int)cdiv(k, kQK);
  const int rowgroups = (int)cdiv(n, kTileRows) * 4;
  const int kw = kb < 8 ? kb : 8;
  const int xvec = (ldx % 8 == 0) && aligned(x, 16);
  const int ybf16 = y_dtype == Q6MOE_BF16;
  hipStream_t s = (hipStream_t)stream;
  if (m <= 16) {
    hipLaunchKernelGGL(q6_skinny_kernel<1>, dim3(rowgroups, 1), dim3(64 * kw), 0, s, x, (int)m,
                       (int)k, ldx, xvec, data, scales, (int)n, kb, kw, y, ybf16, ldy);
  } else {
    hipLaunchKernelGGL(q6_skinny_kernel<4>, dim3(rowgroups, (unsigned)cdiv(m, 64)), dim3(64 * kw), 0,
                       s, x, (int)m, (int)k, ldx, xvec, data, scales, (int)n, kb, kw, y, ybf16, ldy);
  }
  return check_launch("q6_skinny_kernel");
}
