// Q6_K / Q5_K / Q4_K / Q8_0 / Q5_1 decode kernels and the on-device GGUF -> SoA repack.
//
//  * q6_soa_decode_kernel  -- whole-matrix decode of the packed SoA planes to
//    BF16 through the unit decoder the matmul kernels use, in its exact-sign
//    form ds * (c - 32) (kaggle/packed_q6/kernel.py:44-62); the matmul form
//    differs only in the sign of exact zeros.
//  * gguf_decode_vec_kernel / gguf_decode_bytes_kernel / gguf_plain_kernel
//    -- dequantize_rows for raw GGUF rows of every type the reference decodes
//    (kaggle/glm53_offload/gguf_quant.py:111-173 and the Q4_0/Q4_1/Q5_0/Q5_1/
//    IQ4_NL decoder of kaggle/qwen38_tpu/quant.py:15-55).
//  * q6_pack_kernel        -- pack_q6's byte permutation
//    (kaggle/packed_q6/layout.py:71-89).
#include <type_traits>

#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

// grid (tiles, KB), block 256 = 4 waves = the 4 row groups of a 64-row tile.
__global__ void __launch_bounds__(256) q6_soa_decode_kernel(const uint8_t* __restrict__ data,
                                                            const uint8_t* __restrict__ scales,
                                                            int n, int k, int kb_count,
                                                            uint16_t* __restrict__ out, int64_t ldo,
                                                            int vec_ok) {
  const int tile = blockIdx.x, kb = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t t = (int64_t)tile * kb_count + kb;
  const int row = wave * 16 + (lane & 15);
  const int jA = lane >> 4;
  Q6Raw raw;
  q6_load(raw, data + t * kTileBytes, scales + t * 128, row, jA);
  u32x4 a[8];
  q6_decode_unit<true>(raw, jA, a);
  const int gn = tile * kTileRows + row;
  if (gn >= n) return;
  uint16_t* orow = out + (int64_t)gn * ldo;
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const int col = kb * kQK + q6_xfrag_offset(f, jA);
    if (vec_ok && col + 8 <= k) {
      *reinterpret_cast<u32x4*>(orow + col) = a[f];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (col + i < k) orow[col + i] = (uint16_t)(a[f][i >> 1] >> (16 * (i & 1)));
      }
    }
  }
}

__device__ __forceinline__ void store_val(void* out, int64_t idx, float v, int bf16) {
  if (bf16)
    reinterpret_cast<uint16_t*>(out)[idx] = bf16_bits(v);
  else
    reinterpret_cast<float*>(out)[idx] = v;
}

__device__ __forceinline__ float rd_half(const uint8_t* p) {
  return half_bits_to_float((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// Block geometry of the quantized GGUF types: values and bytes per block.
template <int QT>
struct BlockFmt;
template <> struct BlockFmt<Q6MOE_Q6_K> { static constexpr int vals = 256, bytes = 210; };
template <> struct BlockFmt<Q6MOE_Q5_K> { static constexpr int vals = 256, bytes = 176; };
template <> struct BlockFmt<Q6MOE_Q4_K> { static constexpr int vals = 256, bytes = 144; };
template <> struct BlockFmt<Q6MOE_Q8_0> { static constexpr int vals = 32, bytes = 34; };
template <> struct BlockFmt<Q6MOE_Q5_1> { static constexpr int vals = 32, bytes = 24; };
template <> struct BlockFmt<Q6MOE_Q5_0> { static constexpr int vals = 32, bytes = 22; };
template <> struct BlockFmt<Q6MOE_Q4_1> { static constexpr int vals = 32, bytes = 20; };
template <> struct BlockFmt<Q6MOE_Q4_0> { static constexpr int vals = 32, bytes = 18; };
template <> struct BlockFmt<Q6MOE_IQ4_NL> { static constexpr int vals = 32, bytes = 18; };

// The 16 IQ4_NL levels (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25,
// 38, 53, 69, 89, 113; kaggle/qwen38_tpu/quant.py:7) as the bytes of four words.
__device__ __forceinline__ int iq4_level(int nib) {
  const uint32_t w = nib < 8 ? (nib < 4 ? 0xBFAD9881u : 0xF6EADDCFu) : (nib < 12 ? 0x26190D01u : 0x71594535u);
  return (int)(int8_t)(w >> (8 * (nib & 3)));
}

// 16 values [part*16, part*16 + 16) of the block at ``b`` (LDS or global).
//  * Q6_K: ds * (code - 32), ds = d * int8 sub-scale (gguf_quant.py:158-173).
//  * Q4_K/Q5_K: fma(d*sc, q, -(dmin*m)) with the 6-bit packed sub-scales and
//    mins; Q5_K's 32 high-bit bytes at 16 (bit j of byte l is bit 4 of
//    sub-block j's position l), then the nibbles (gguf_quant.py:115-157).
//  * Q8_0: d * int8 code (gguf_quant.py:111-114).
//  * 32-value nibble types (kaggle/qwen38_tpu/quant.py:15-55): d (FP16), then
//    m (FP16) for the affine Q4_1/Q5_1, then 32 high bits for Q5_0/Q5_1, then
//    16 bytes whose low nibbles are positions 0-15 and high nibbles 16-31; bit
//    i of the high word is bit 4 of position i. w = d*q + m (affine), d*(q-8)
//    (Q4_0), d*(q-16) (Q5_0), d*level[q] (IQ4_NL). Every product d*q here has
//    at most 18 significant bits, so it is exact in FP32 and the affine sum is
//    one rounding, as in the reference's two-step d*q then +m.
template <int QT>
__device__ __forceinline__ void decode16(const uint8_t* b, int part, float v[16]) {
  if constexpr (QT == Q6MOE_Q6_K) {
    const int p0 = part * 16, h = p0 >> 7, q = (p0 & 127) >> 5, l0 = p0 & 31;
    const float ds = rd_half(b + 208) * (float)(int8_t)b[192 + part];
    const uint8_t* ql = b + h * 64 + (q & 1) * 32 + l0;
    const uint8_t* qh = b + 128 + h * 32 + l0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int lo = (ql[i] >> (4 * (q >> 1))) & 15, hi = (qh[i] >> (2 * q)) & 3;
      v[i] = ds * (float)((lo | (hi << 4)) - 32);
    }
  } else if constexpr (QT == Q6MOE_Q4_K || QT == Q6MOE_Q5_K) {
    const int j = part >> 1, l0 = (part & 1) * 16;  // sub-block, first position
    const float d = rd_half(b), dmin = rd_half(b + 2);
    int sc, mn;
    if (j < 4) {
      sc = b[4 + j] & 63;
      mn = b[8 + j] & 63;
    } else {
      sc = (b[12 + j - 4] & 15) | ((b[4 + j - 4] >> 2) & 48);
      mn = (b[12 + j - 4] >> 4) | ((b[8 + j - 4] >> 2) & 48);
    }
    const float a = d * (float)sc, m = dmin * (float)mn;
    const uint8_t* qs = b + (QT == Q6MOE_Q5_K ? 48 : 16) + (j >> 1) * 32 + l0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int q = (j & 1) ? (qs[i] >> 4) : (qs[i] & 15);
      if constexpr (QT == Q6MOE_Q5_K) q |= ((b[16 + l0 + i] >> j) & 1) << 4;
      v[i] = __builtin_fmaf(a, (float)q, -m);
    }
  } else if constexpr (QT == Q6MOE_Q8_0) {
    const float d = rd_half(b);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = d * (float)(int8_t)b[2 + part * 16 + i];
  } else {
    constexpr bool affine = QT == Q6MOE_Q4_1 || QT == Q6MOE_Q5_1;
    constexpr bool wide = QT == Q6MOE_Q5_0 || QT == Q6MOE_Q5_1;
    constexpr int hi_at = affine ? 4 : 2, lo_at = hi_at + (wide ? 4 : 0);
    const float d = rd_half(b);
    const float m = affine ? rd_half(b + 2) : 0.0f;
    uint32_t qh = 0;
    if constexpr (wide)
      qh = (uint32_t)b[hi_at] | ((uint32_t)b[hi_at + 1] << 8) | ((uint32_t)b[hi_at + 2] << 16) |
           ((uint32_t)b[hi_at + 3] << 24);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int nib = part ? (b[lo_at + i] >> 4) : (b[lo_at + i] & 15);
      const int q = wide ? nib | (int)(((qh >> (part * 16 + i)) & 1u) << 4) : nib;
      if constexpr (QT == Q6MOE_IQ4_NL)
        v[i] = d * (float)iq4_level(nib);
      else if constexpr (affine)
        v[i] = __builtin_fmaf((float)q, d, m);
      else
        v[i] = d * (float)(q - (wide ? 16 : 8));
    }
  }
}

// Stores the 16 values of (row, col) as 16-byte vectors when the target is
// aligned and whole, else value by value (the row's tail).
__device__ __forceinline__ void store16(void* out, int64_t at, int col, int width, const float v[16], int bf16,
                                        int vec_out) {
  if (vec_out && col + 16 <= width && (at & 7) == 0) {
    if (bf16) {
      u32x4 o0, o1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o0[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
        o1[i] = pack_bf16x2(v[8 + 2 * i], v[8 + 2 * i + 1]);
      }
      u32x4* o = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + at);
      o[0] = o0;
      o[1] = o1;
    } else {
      f32x4* o = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + at);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (col + i < width) store_val(out, at + i, v[i], bf16);
  }
}

// Row decode for 4-byte aligned input: a workgroup stages NB consecutive blocks
// (NB * BYTES bytes, a multiple of 4) in LDS with coalesced dword loads, then
// each thread decodes 16 consecutive values of one block.
template <int QT>
__global__ void __launch_bounds__(256)
    gguf_decode_vec_kernel(const uint8_t* __restrict__ raw, int64_t total_blocks, int blocks, int width,
                           void* __restrict__ out, int bf16, int vec_out) {
  constexpr int VALS = BlockFmt<QT>::vals, BYTES = BlockFmt<QT>::bytes;
  constexpr int TPB = VALS / 16, NB = 256 / TPB;  // threads per block, blocks per workgroup
  static_assert((NB * BYTES) % 4 == 0, "whole dwords per workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t st[NB * BYTES];
  const int64_t b0 = (int64_t)blockIdx.x * NB;
  const int nb = total_blocks - b0 < NB ? (int)(total_blocks - b0) : NB;
  const int nbytes = nb * BYTES;
  const uint8_t* src = raw + b0 * BYTES;
  for (int i = threadIdx.x; i * 4 < nbytes; i += 256) {
    if (i * 4 + 4 <= nbytes) {
      *reinterpret_cast<uint32_t*>(st + 4 * i) = *reinterpret_cast<const uint32_t*>(src + 4 * i);
    } else {
      for (int k = 4 * i; k < nbytes; ++k) st[k] = src[k];  // the buffer's last partial dword
    }
  }
  __syncthreads();
  const int bl = threadIdx.x / TPB, part = threadIdx.x % TPB;
  if (bl >= nb) return;
  float v[16];
  decode16<QT>(st + bl * BYTES, part, v);
  const int64_t gb = b0 + bl, row = gb / blocks;
  const int col = (int)(gb - row * blocks) * VALS + part * 16;
  store16(out, row * width + col, col, width, v, bf16, vec_out);
}

// Row decode for input at any byte address: one thread per 16 values, reading
// its block's bytes from global memory.
template <int QT>
__global__ void __launch_bounds__(256)
    gguf_decode_bytes_kernel(const uint8_t* __restrict__ raw, int64_t total_blocks, int blocks, int width,
                             void* __restrict__ out, int bf16, int vec_out) {
  constexpr int VALS = BlockFmt<QT>::vals, BYTES = BlockFmt<QT>::bytes, TPB = VALS / 16;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= total_blocks * TPB) return;
  const int64_t gb = gid / TPB;
  const int part = (int)(gid % TPB);
  float v[16];
  decode16<QT>(raw + gb * BYTES, part, v);
  const int64_t row = gb / blocks;
  const int col = (int)(gb - row * blocks) * VALS + part * 16;
  store16(out, row * width + col, col, width, v, bf16, vec_out);
}

// Unquantized rows (F32, F16, BF16; one value per "block"): the float value,
// then the output rounding. Little-endian element bytes at any alignment.
__global__ void __launch_bounds__(256) gguf_plain_kernel(const uint8_t* __restrict__ raw, int qtype, int64_t n,
                                                         void* __restrict__ out, int bf16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v;
  if (qtype == Q6MOE_GGUF_F32) {
    const uint8_t* p = raw + 4 * i;
    v = __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
  } else {
    const uint8_t* p = raw + 2 * i;
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    v = qtype == Q6MOE_GGUF_F16 ? half_bits_to_float(h) : __uint_as_float(h << 16);
  }
  store_val(out, i, v, bf16);
}

// One thread per (padded row, K block): moves the 208 code/sub-scale bytes into
// the three regions of its tile and the FP16 d into the scale plane.
__global__ void q6_pack_kernel(const uint8_t* __restrict__ raw, int n, int kb_count, int tiles,
                               uint8_t* __restrict__ data, uint8_t* __restrict__ scales,
                               int64_t scale_bytes) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)tiles * kTileRows * kb_count;
  if (gid < total) {
    const int64_t rowg = gid / kb_count;
    const int kb = (int)(gid % kb_count);
    const int tile = (int)(rowg / kTileRows), r = (int)(rowg % kTileRows);
    const int64_t t = (int64_t)tile * kb_count + kb;
    uint8_t* tb = data + t * kTileBytes;
    const bool live = rowg < n;
    const uint8_t* src = raw + (rowg * kb_count + kb) * 210;
    for (int b = 0; b < 128; ++b) tb[kQlOff + r * 128 + b] = live ? src[b] : 0;
    for (int b = 0; b < 64; ++b) tb[kQhOff + r * 64 + b] = live ? src[128 + b] : 0;
    for (int b = 0; b < 16; ++b) tb[kScOff + r * 16 + b] = live ? src[192 + b] : 0;
    scales[(t * kTileRows + r) * 2] = live ? src[208] : 0;
    scales[(t * kTileRows + r) * 2 + 1] = live ? src[209] : 0;
  }
  // zero the 512-byte padding of the scale plane
  const int64_t used = total * 2;
  const int64_t pad = scale_bytes - used;
  if (gid < pad) scales[used + gid] = 0;
}

}  // namespace q6moe

using namespace q6moe;

extern "C" int q6moe_q6_decode(const uint8_t* data, const uint8_t* scales, int64_t n, int64_t k,
                               uint16_t* out, int64_t ldo, void* stream) {
  Q6MOE_REQUIRE(data && scales && out, "q6_decode: null pointer");
  Q6MOE_REQUIRE(n >= 1 && k >= 1 && ldo >= k, "q6_decode: need n >= 1, k >= 1, ldo >= k");
  Q6MOE_REQUIRE(n <= (1 << 30) && k <= (1 << 30), "q6_decode: dimension too large");
  Q6MOE_REQUIRE(aligned(data, 16) && aligned(scales, 2), "q6_decode: data must be 16-byte aligned");
  const int kb = (int)cdiv(k, kQK), tiles = (int)cdiv(n, kTileRows);
  const int vec_ok = (ldo % 8 == 0) && aligned(out, 16);
  hipLaunchKernelGGL(q6_soa_decode_kernel, dim3(tiles, kb), dim3(256), 0, (hipStream_t)stream, data,
                     scales, (int)n, (int)k, kb, out, ldo, vec_ok);
  return check_launch("q6_soa_decode_kernel");
}

extern "C" int q6moe_q6_pack(const uint8_t* raw, int64_t n, int64_t k, uint8_t* data,
                             uint8_t* scales, void* stream) {
  Q6MOE_REQUIRE(raw && data && scales, "q6_pack: null pointer");
  Q6MOE_REQUIRE(n >= 1 && k >= 1 && n <= (1 << 30) && k <= (1 << 30), "q6_pack: bad shape");
  const int kb = (int)cdiv(k, kQK), tiles = (int)cdiv(n, kTileRows);
  const int64_t total = (int64_t)tiles * kTileRows * kb;
  const int64_t scale_bytes = cdiv(total * 2, 512) * 512;
  const int64_t threads = total > scale_bytes - total * 2 ? total : scale_bytes - total * 2;
  hipLaunchKernelGGL(q6_pack_kernel, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0,
                     (hipStream_t)stream, raw, (int)n, kb, tiles, data, scales, scale_bytes);
  return check_launch("q6_pack_kernel");
}

extern "C" int q6moe_gguf_decode(const uint8_t* raw, int qtype, int64_t rows, int64_t width,
                                 void* out, int out_dtype, void* stream) {
  Q6MOE_REQUIRE(raw && out, "gguf_decode: null pointer");
  Q6MOE_REQUIRE(rows >= 1 && width >= 1 && width <= (1 << 30), "gguf_decode: bad shape");
  Q6MOE_REQUIRE(out_dtype == Q6MOE_F32 || out_dtype == Q6MOE_BF16, "gguf_decode: out dtype");
  hipStream_t s = (hipStream_t)stream;
  const int bf16 = out_dtype == Q6MOE_BF16;
  if (qtype == Q6MOE_GGUF_F32 || qtype == Q6MOE_GGUF_F16 || qtype == Q6MOE_GGUF_BF16) {
    const int64_t n = rows * width;
    hipLaunchKernelGGL(gguf_plain_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, raw, qtype, n, out, bf16);
    return check_launch("gguf_plain_kernel");
  }
  const int vec = aligned(out, 16);
  const bool staged = aligned(raw, 4);  // staged through LDS with dword loads
  int rc = Q6MOE_ERR_UNSUPPORTED;
  auto run = [&](auto qt) {
    constexpr int QT = decltype(qt)::value, VALS = BlockFmt<QT>::vals;
    const int blocks = (int)cdiv(width, VALS);
    const int64_t total = rows * blocks;
    if (staged) {
      hipLaunchKernelGGL(gguf_decode_vec_kernel<QT>, dim3((unsigned)cdiv(total, 256 / (VALS / 16))), dim3(256), 0,
                         s, raw, total, blocks, (int)width, out, bf16, vec);
      rc = check_launch("gguf_decode_vec_kernel");
    } else {
      hipLaunchKernelGGL(gguf_decode_bytes_kernel<QT>, dim3((unsigned)cdiv(total * (VALS / 16), 256)), dim3(256),
                         0, s, raw, total, blocks, (int)width, out, bf16, vec);
      rc = check_launch("gguf_decode_bytes_kernel");
    }
  };
  switch (qtype) {
    case Q6MOE_Q6_K: run(std::integral_constant<int, Q6MOE_Q6_K>{}); break;
    case Q6MOE_Q5_K: run(std::integral_constant<int, Q6MOE_Q5_K>{}); break;
    case Q6MOE_Q4_K: run(std::integral_constant<int, Q6MOE_Q4_K>{}); break;
    case Q6MOE_Q8_0: run(std::integral_constant<int, Q6MOE_Q8_0>{}); break;
    case Q6MOE_Q5_1: run(std::integral_constant<int, Q6MOE_Q5_1>{}); break;
    case Q6MOE_Q5_0: run(std::integral_constant<int, Q6MOE_Q5_0>{}); break;
    case Q6MOE_Q4_1: run(std::integral_constant<int, Q6MOE_Q4_1>{}); break;
    case Q6MOE_Q4_0: run(std::integral_constant<int, Q6MOE_Q4_0>{}); break;
    case Q6MOE_IQ4_NL: run(std::integral_constant<int, Q6MOE_IQ4_NL>{}); break;
    default:
      set_error("gguf_decode: unsupported GGUF type (F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, "
                "Q6_K, IQ4_NL)");
      return Q6MOE_ERR_UNSUPPORTED;
  }
  return rc;
}
