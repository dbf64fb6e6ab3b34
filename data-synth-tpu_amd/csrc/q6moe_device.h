// Device-side helpers shared by the q6moe kernels (gfx950 / CDNA4 only).
//
// Number formats follow the reference exactly:
//  * FP16 block scales widen to FP32 exactly (kaggle/packed_q6/kernel.py:27-41).
//  * Q6_K values (d * sc) * code are exact in FP32; Q4_K values round once at
//    the final subtraction (kaggle/glm53_offload/gguf_quant.py:115-173).
//  * BF16 conversion is round-to-nearest-even (kaggle/qwen38_tpu/precision.py:7-17);
//    v_cvt_pk_bf16_f32 implements it in one instruction for two values.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q6moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kQK = 256;              // values per Q6_K / Q4_K block
constexpr int kTileRows = 64;         // SoA output tile (layout.py:15)
constexpr int kTileBytes = 64 * 208;  // 13312 (layout.py:16)
constexpr int kQlOff = 0;             // 64 rows x 128 B
constexpr int kQhOff = 8192;          // 64 rows x 64 B
constexpr int kScOff = 12288;         // 64 rows x 16 B
constexpr int kWave = 64;

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  // v_cvt_f32_f16 widens every finite FP16 pattern (subnormals, signed zero) exactly.
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;  // v_cvt_pk_bf16_f32: RNE
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float bf16_round(float x) {
  return (float)(__bf16)x;
}

__device__ __forceinline__ float bf16_to_float(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__device__ __forceinline__ float ubyte_f(uint32_t w, int b) {
  return (float)((w >> (8 * b)) & 0xffu);  // v_cvt_f32_ubyteN
}

// Four 6-bit Q6_K codes (as unsigned bytes 0..63, value = byte - 32) from one
// ql dword and the matching qh dword. ``hs`` is qh already shifted right by
// 2*q0 so that bits 0-1 of each byte hold the quarter-q0 high bits and bits
// 4-5 the quarter-(q0+2) high bits (gguf_quant.py:159-167).
__device__ __forceinline__ uint32_t q6_codes_lo(uint32_t ql, uint32_t hs) {
  return (ql & 0x0f0f0f0fu) | ((hs << 4) & 0x30303030u);
}
__device__ __forceinline__ uint32_t q6_codes_hi(uint32_t ql, uint32_t hs) {
  return ((ql >> 4) & 0x0f0f0f0fu) | (hs & 0x30303030u);
}

// Eight weights (two code dwords) -> one MFMA bf16x8 operand (4 dwords),
// w = RNE_bf16(ds * (c - 32)) computed as fma(c, ds, -32*ds). Both ds*c and
// ds*32 are exact in FP32, so the value is exact; only the sign of an exact
// zero can differ from ds * (c - 32) (+0 instead of -0), which no sum of
// products can observe. q6_frag_exact keeps the reference's signed zeros.
// The code words are made opaque first: callers pass masked words (K-quant and
// Q5_1 nibbles), and the compiler would otherwise fold each byte's mask into a
// v_bfe_u32 before its conversion instead of one v_cvt_f32_ubyteN per byte.
__device__ __forceinline__ u32x4 q6_frag(uint32_t c0, uint32_t c1, float ds, float nds) {
  asm("" : "+v"(c0), "+v"(c1));
  u32x4 r;
  r[0] = pack_bf16x2(__builtin_fmaf(ubyte_f(c0, 0), ds, nds), __builtin_fmaf(ubyte_f(c0, 1), ds, nds));
  r[1] = pack_bf16x2(__builtin_fmaf(ubyte_f(c0, 2), ds, nds), __builtin_fmaf(ubyte_f(c0, 3), ds, nds));
  r[2] = pack_bf16x2(__builtin_fmaf(ubyte_f(c1, 0), ds, nds), __builtin_fmaf(ubyte_f(c1, 1), ds, nds));
  r[3] = pack_bf16x2(__builtin_fmaf(ubyte_f(c1, 2), ds, nds), __builtin_fmaf(ubyte_f(c1, 3), ds, nds));
  return r;
}

// q6_frag for Q6_K codes with two VALU fewer per four weights: each code byte
// c becomes the FP16 value 1024 + c (bits 0x6400 | c, exact, one v_perm per
// two codes) and v_fma_mix_f32 computes (1024 + c) * ds + n1056 with
// n1056 = -1056 * ds. ds = d * sc has at most 18 significant bits (11-bit FP16
// significand, |sc| <= 128), so n1056 (x 33 * 32) is exact in FP32, and the
// single rounding of the exact ds * (c - 32) returns it unchanged: the value
// and the +0 for c = 32 match q6_frag bit for bit.
__device__ __forceinline__ float h16_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ float h16_hi(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}
__device__ __forceinline__ u32x4 q6_frag_mix(uint32_t c0, uint32_t c1, float ds, float n1056) {
  const uint32_t h0 = __builtin_amdgcn_perm(0x64646464u, c0, 0x04010400u);  // codes 0, 1
  const uint32_t h1 = __builtin_amdgcn_perm(0x64646464u, c0, 0x04030402u);  // codes 2, 3
  const uint32_t h2 = __builtin_amdgcn_perm(0x64646464u, c1, 0x04010400u);
  const uint32_t h3 = __builtin_amdgcn_perm(0x64646464u, c1, 0x04030402u);
  u32x4 r;
  r[0] = pack_bf16x2(__builtin_fmaf(h16_lo(h0), ds, n1056), __builtin_fmaf(h16_hi(h0), ds, n1056));
  r[1] = pack_bf16x2(__builtin_fmaf(h16_lo(h1), ds, n1056), __builtin_fmaf(h16_hi(h1), ds, n1056));
  r[2] = pack_bf16x2(__builtin_fmaf(h16_lo(h2), ds, n1056), __builtin_fmaf(h16_hi(h2), ds, n1056));
  r[3] = pack_bf16x2(__builtin_fmaf(h16_lo(h3), ds, n1056), __builtin_fmaf(h16_hi(h3), ds, n1056));
  return r;
}

// ---------------------------------------------------------------------------
// Bit-planar Q6_K lane layout (the MoE unit tables). A lane holds 64 weights
// as four groups of one 16-wide sub-block each; a group is three 32-bit code
// words w0, w1, w2 laid out so that the FP16 form of every code pair of an
// MFMA operand comes out of one word with one or two v_bitop3 (gfx950's
// three-input bitwise op): about 200 VALU instructions per unit instead of the
// 232 of the byte assembly + v_perm_b32 path of q6_decode_unit.
//   pair k (sub-block positions 2k, 2k+1; low half / high half):
//   k = 0..5  the 6-bit codes at bits [4,10) and [20,26) of word k/2 after a
//             right shift by 6*(k%2), taken as FP16 0x6400 | code << 4, i.e.
//             1024 + 16c, so w = fma(h, ds/16, -96*ds);
//   k = 6, 7  the low nibbles at bits [0,4) and [16,20) of word k-6, the high
//             two bits at bits [2(k-6), 2(k-6)+2) and 16 above in word 2;
//             FP16 0x6400 | code = 1024 + c, so w = fma(h, ds, -1056*ds).
// Both forms give ds*(c-32) exactly (ds has at most 18 significant bits), so
// the BF16 weights equal those of q6_frag_mix bit for bit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t b3_fmt(uint32_t r, uint32_t m, uint32_t k) {
  return __builtin_amdgcn_bitop3_b32(r, m, k, 0xEA);  // (r & m) | k
}
__device__ __forceinline__ uint32_t b3_sel(uint32_t a, uint32_t b, uint32_t m) {
  return __builtin_amdgcn_bitop3_b32(a, b, m, 0xE4);  // (a & m) | (b & ~m)
}
__device__ __forceinline__ uint32_t mix_pair(uint32_t h, float s, float n) {
  return pack_bf16x2(__builtin_fmaf(h16_lo(h), s, n), __builtin_fmaf(h16_hi(h), s, n));
}
// One group: fragment fa = sub-block positions 0..7, fb = 8..15.
__device__ __forceinline__ void q6p_group(uint32_t w0, uint32_t w1, uint32_t w2, float ds, u32x4& fa, u32x4& fb) {
  const uint32_t M4 = 0x03F003F0u, M0 = 0x003F003Fu, MN = 0x000F000Fu, K = 0x64006400u;
  const float s4 = ds * 0.0625f, n4 = -96.f * ds, n0 = -1056.f * ds;
  fa[0] = mix_pair(b3_fmt(w0, M4, K), s4, n4);
  fa[1] = mix_pair(b3_fmt(w0 >> 6, M4, K), s4, n4);
  fa[2] = mix_pair(b3_fmt(w1, M4, K), s4, n4);
  fa[3] = mix_pair(b3_fmt(w1 >> 6, M4, K), s4, n4);
  fb[0] = mix_pair(b3_fmt(w2, M4, K), s4, n4);
  fb[1] = mix_pair(b3_fmt(w2 >> 6, M4, K), s4, n4);
  fb[2] = mix_pair(b3_fmt(b3_sel(w0, w2 << 4, MN), M0, K), ds, n0);
  fb[3] = mix_pair(b3_fmt(b3_sel(w1, w2 << 2, MN), M0, K), ds, n0);
}
// Sub-scale of group g from the lane's scale word (byte g, signed).
__device__ __forceinline__ float q6p_ds(float d, uint32_t scw, int g) {
  return d * (float)(int)(int8_t)(scw >> (8 * g));
}
// The lane's 8 A fragments: fragment 2g+e covers unit positions
// 64g + 16jA + 8e + [0, 8) (the same positions as q6_decode_unit).
__device__ __forceinline__ void q6p_decode(const u32x4& c0, const u32x4& c1, const u32x4& c2, uint32_t scw,
                                           uint32_t dbits, u32x4 a[8]) {
  const float d = half_bits_to_float(dbits);
#pragma unroll
  for (int g = 0; g < 4; ++g) q6p_group(c0[g], c1[g], c2[g], q6p_ds(d, scw, g), a[2 * g], a[2 * g + 1]);
}

__device__ __forceinline__ u32x4 q6_frag_exact(uint32_t c0, uint32_t c1, float ds) {
  u32x4 r;
  r[0] = pack_bf16x2(ds * (ubyte_f(c0, 0) - 32.f), ds * (ubyte_f(c0, 1) - 32.f));
  r[1] = pack_bf16x2(ds * (ubyte_f(c0, 2) - 32.f), ds * (ubyte_f(c0, 3) - 32.f));
  r[2] = pack_bf16x2(ds * (ubyte_f(c1, 0) - 32.f), ds * (ubyte_f(c1, 1) - 32.f));
  r[3] = pack_bf16x2(ds * (ubyte_f(c1, 2) - 32.f), ds * (ubyte_f(c1, 3) - 32.f));
  return r;
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Non-temporal 16-byte load for streamed weight bytes that are read once.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Accurate FP32 sigmoid: where(x >= 0, 1, e) / (1 + e), e = exp(-|x|)
// (kaggle/qwen38_tpu/numerics.py:42-45), with the correctly rounded quotient.
// The divisor d = 1 + e lies in (1, 2] and the numerator in [0, 1], so the
// quotient is formed by the FMA method of Markstein (IBM J. Res. Dev. 34,
// 1990): the hardware reciprocal refined by one Newton step, the product,
// and one correction by the exact FMA residual, without the scaling steps a
// general division needs for extreme exponents. For every BF16 input (the
// only inputs its callers pass) it equals the IEEE quotient of the same e;
// the sigmoid probe's test checks all of them.
__device__ __forceinline__ float sigmoid_acc(float x) {
  const float e = expf(-fabsf(x));
  const float num = x >= 0.f ? 1.f : e;
  const float d = 1.f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  const float r1 = __builtin_fmaf(__builtin_fmaf(-d, r, 1.f), r, r);
  const float q = num * r1;
  return __builtin_fmaf(__builtin_fmaf(-d, q, num), r1, q);
}

// ---------------------------------------------------------------------------
// Q6_K SoA "unit": 16 output rows x one 256-wide K block, decoded by one wave
// straight into eight MFMA A operands.
//
// Lane l handles row (l % 16) of the 16-row group and ql chunks jA = l / 16 and
// jA + 4 (16 bytes each). With q0 = jA >> 1 and e = fragment half, fragment f =
// 2g + e covers block positions
//     p = 128*(g >> 1) + 32*(q0 + 2*(g & 1)) + 16*(jA & 1) + 8*e + [0..7]
// and sub-block jA + 4g. The matching x operand for token j is the 8
// consecutive BF16 values at that position (see q6_xfrag_offset).
// ---------------------------------------------------------------------------
struct Q6Raw {
  u32x4 qlA, qlB;  // ql chunks jA, jA+4 of the row
  u32x4 qhA, qhB;  // qh bytes for h = 0, 1 (same l range)
  u32x4 sc;        // the row's 16 signed sub-scales
  uint32_t d;      // FP16 bits of the block scale
};

__device__ __forceinline__ void q6_load(Q6Raw& r, const uint8_t* tile, const uint8_t* dplane,
                                        int row, int jA) {
  const uint8_t* ql = tile + kQlOff + row * 128 + 16 * jA;
  const uint8_t* qh = tile + kQhOff + row * 64 + 16 * (jA & 1);
  r.qlA = ld16_stream(ql);
  r.qlB = ld16_stream(ql + 64);
  r.qhA = ld16_stream(qh);
  r.qhB = ld16_stream(qh + 32);
  r.sc = ld16_stream(tile + kScOff + row * 16);
  r.d = *reinterpret_cast<const uint16_t*>(dplane + row * 2);
}

// Decode a loaded unit into 8 A fragments (kExact: reference signed zeros).
template <bool kExact = false>
__device__ __forceinline__ void q6_decode_unit(const Q6Raw& r, int jA, u32x4 a[8]) {
  const float d = half_bits_to_float(r.d);
  const int q0 = jA >> 1;
  const int sh = 8 * jA;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int scv = (int)(int8_t)((r.sc[g] >> sh) & 0xff);
    const float ds = d * (float)scv;
    const float n1056 = -1056.f * ds;
    const u32x4& ql = (g >> 1) ? r.qlB : r.qlA;
    const u32x4& qh = (g >> 1) ? r.qhB : r.qhA;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      uint32_t c0, c1;
      const uint32_t h0 = qh[2 * e] >> (2 * q0), h1 = qh[2 * e + 1] >> (2 * q0);
      if (g & 1) {
        c0 = q6_codes_hi(ql[2 * e], h0);
        c1 = q6_codes_hi(ql[2 * e + 1], h1);
      } else {
        c0 = q6_codes_lo(ql[2 * e], h0);
        c1 = q6_codes_lo(ql[2 * e + 1], h1);
      }
      a[2 * g + e] = kExact ? q6_frag_exact(c0, c1, ds) : q6_frag_mix(c0, c1, ds, n1056);
    }
  }
}

// Eight weights w = RNE_bf16(fma(q, a, n)) of small unsigned codes q held as
// FP16 subnormals: a 16-bit half whose bits are q << b (q << b < 1024) is the
// FP16 value q * 2^(b-24), exactly. v_fma_mix_f32 takes it as is with the
// scale s = a * 2^(24-b) (a power-of-two multiple of a, exact; no overflow
// for FP16-derived scales), so h * s = q * a exactly and the single rounding
// is that of fma(q, a, n): the values are bit-identical to q6_frag's, with no
// per-code integer-to-float conversion. ``e`` words hold K positions 0 and 2
// of a four-code group in their low and high halves, ``o`` words positions 1
// and 3.
__device__ __forceinline__ u32x4 sub_frag(uint32_t e0, uint32_t o0, uint32_t e1, uint32_t o1, float s, float n) {
  u32x4 r;
  r[0] = pack_bf16x2(__builtin_fmaf(h16_lo(e0), s, n), __builtin_fmaf(h16_lo(o0), s, n));
  r[1] = pack_bf16x2(__builtin_fmaf(h16_hi(e0), s, n), __builtin_fmaf(h16_hi(o0), s, n));
  r[2] = pack_bf16x2(__builtin_fmaf(h16_lo(e1), s, n), __builtin_fmaf(h16_lo(o1), s, n));
  r[3] = pack_bf16x2(__builtin_fmaf(h16_hi(e1), s, n), __builtin_fmaf(h16_hi(o1), s, n));
  return r;
}

// Q8_0: 8 int8 codes (two words, lowest byte first) times the block scale d;
// each product is exact in FP32 (11-bit d times an 8-bit code), then RNE to
// BF16 (kaggle/glm53_offload/gguf_quant.py:111-114). kOpaque hides the words
// from the compiler, which keeps each code's conversion one v_cvt_f32_i32 with
// a sign-extended byte select where it would otherwise extract byte 0 with a
// separate v_bfe_i32 (the generic kernels' register path); the LDS-staged
// decode-step path selects the one-instruction form by itself.
template <bool kOpaque = false>
__device__ __forceinline__ u32x4 q8_frag(uint32_t w0, uint32_t w1, float d) {
  if constexpr (kOpaque) asm("" : "+v"(w0), "+v"(w1));
  u32x4 r;
  r[0] = pack_bf16x2(d * (float)(int8_t)w0, d * (float)(int8_t)(w0 >> 8));
  r[1] = pack_bf16x2(d * (float)(int8_t)(w0 >> 16), d * (float)(int8_t)(w0 >> 24));
  r[2] = pack_bf16x2(d * (float)(int8_t)w1, d * (float)(int8_t)(w1 >> 8));
  r[3] = pack_bf16x2(d * (float)(int8_t)(w1 >> 16), d * (float)(int8_t)(w1 >> 24));
  return r;
}

// The 8 A fragments of a Q8_0 unit from the lane's 4 code chunks and its 4
// FP16 block scales (chunk g: fragments 2g and 2g+1, scale g).
template <bool kOpaque = false>
__device__ __forceinline__ void q8_decode(const u32x4 (&c)[4], u32x2 dw, u32x4 a[8]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float d = half_bits_to_float((dw[g >> 1] >> (16 * (g & 1))) & 0xffffu);
    a[2 * g] = q8_frag<kOpaque>(c[g][0], c[g][1], d);
    a[2 * g + 1] = q8_frag<kOpaque>(c[g][2], c[g][3], d);
  }
}

// Element offset, inside one 256-wide K block, of the 8 x values that pair
// with fragment f of a lane in k-group jA.
__device__ __forceinline__ int q6_xfrag_offset(int f, int jA) {
  const int g = f >> 1, e = f & 1;
  return 128 * (g >> 1) + 32 * ((jA >> 1) + 2 * (g & 1)) + 16 * (jA & 1) + 8 * e;
}

}  // namespace q6moe
