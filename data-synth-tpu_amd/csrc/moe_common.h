// Shared definitions of the routed-expert kernels (decode and grouped GEMM).
#pragma once
#include <type_traits>

#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

enum { FMT_Q6 = 0, FMT_Q4K = 1, FMT_Q8 = 2, FMT_Q5K = 3, FMT_Q51 = 4 };

// Experts of one layer (one call) that the routing of every path handles:
// the decode kernels' expert bit mask and counts, the grouped routing's
// per-expert counts, bitmaps and scans, and the device router.
constexpr int kMaxExperts = 1024;

// Expert tables of the routed-expert kernels are unit-major: a unit is 16
// output rows x one 256-wide K block, stored exactly as a wave stages it in
// LDS, and an expert's units are ordered [row group][K block] so that a wave
// streaming one row group over K reads one contiguous run. Lane l of the wave
// decoding a unit owns row j = l % 16 and the K positions 64g + 16jA + [0, 16)
// (jA = l / 16, g = 0..3: sub-block 4g + jA).
//   Q6_K unit (3360 B), bit-planar (the same 6 bits per weight, rearranged):
//     codes [0, 3072)    code word g of chunk c (0..2) of lane l at 1024c + 16l + 4g
//                        (bit map in q6moe_device.h, q6p_decode)
//     sc    [3072, 3328) lane l's sub-scales of sub-blocks 4g + jA at 3072 + 4l + g
//     d     [3328, 3360) row j's FP16 scale at 3328 + 2j
//   Q4_K unit (2304 B): chunk c (0..8) of row j's 144-byte block at 16*(16c + j)
//   Q8_0 unit (4352 B: 16 rows x 8 blocks of 34 B, rearranged):
//     codes [0, 4096)    chunk g of lane l at 1024g + 16l: row j's 16 int8 codes at
//                        K positions 64g + 16jA + [0, 16), i.e. codes 16(jA%2) + [0, 16)
//                        of its block 2g + jA/2
//     d     [4096, 4352) FP16 scale of row j's block 2g + h at 4096 + 8(2j + h) + 2g
//   Q5_K unit (2816 B): chunk c (0..10) of row j's 176-byte block at 16*(16c + j)
//   Q5_1 unit (3072 B: 16 rows x 8 blocks of 24 B, rearranged):
//     qs    [0, 2048)    the 16 nibble bytes of row j's block 2g + h at 512g + 256h + 16j
//     aux   [2048, 3072) row j's block 2g + h: high-bit word, FP16 d, FP16 m at
//                        2048 + 64j + 32h + 8g
// (GGUF block formats: kaggle/glm53_offload/gguf_quant.py:111-173,
// kaggle/qwen38_tpu/quant.py:15-55). Rows (and Q8_0 / Q5_1 blocks) past the
// matrix are zero.
constexpr int kQ6Unit = 3360;
constexpr int kQ4Unit = 2304;
constexpr int kQ8Unit = 4352;
constexpr int kQ5KUnit = 2816;
constexpr int kQ51Unit = 3072;

// Calls f(std::integral_constant<int, FMT>) for the runtime format ``fmt``
// (host-side dispatch to the kernels' template instantiations).
template <typename F>
inline void dispatch_format(int fmt, F&& f) {
  switch (fmt) {
    case FMT_Q6: f(std::integral_constant<int, FMT_Q6>{}); break;
    case FMT_Q4K: f(std::integral_constant<int, FMT_Q4K>{}); break;
    case FMT_Q8: f(std::integral_constant<int, FMT_Q8>{}); break;
    case FMT_Q5K: f(std::integral_constant<int, FMT_Q5K>{}); break;
    default: f(std::integral_constant<int, FMT_Q51>{}); break;
  }
}
// Gate/up format (Q6_K, Q4_K, Q5_K or Q8_0) x down format (any).
template <typename F>
inline void dispatch_formats(int fg, int fd, F&& f) {
  dispatch_format(fd, [&](auto d) {
    switch (fg) {
      case FMT_Q6: f(std::integral_constant<int, FMT_Q6>{}, d); break;
      case FMT_Q4K: f(std::integral_constant<int, FMT_Q4K>{}, d); break;
      case FMT_Q5K: f(std::integral_constant<int, FMT_Q5K>{}, d); break;
      default: f(std::integral_constant<int, FMT_Q8>{}, d); break;
    }
  });
}

template <int FMT>
struct UnitBytes;
template <>
struct UnitBytes<0> {
  static constexpr int value = kQ6Unit;
};
template <>
struct UnitBytes<1> {
  static constexpr int value = kQ4Unit;
};
template <>
struct UnitBytes<2> {
  static constexpr int value = kQ8Unit;
};
template <>
struct UnitBytes<3> {
  static constexpr int value = kQ5KUnit;
};
template <>
struct UnitBytes<4> {
  static constexpr int value = kQ51Unit;
};

// One projection's expert table: [rows x k] per expert.
struct Proj {
  const uint8_t* data;  // expert e's units at data + e * dstride
  int64_t dstride;
  int rows, k, kb;
};

// The K block whose second half lies wholly past the matrix (k % 256 in
// (0, 128]), or -1: in 32-value formats its units hold only zero padding there.
__host__ __device__ __forceinline__ int half_block(const Proj& p) {
  return p.k % 256 != 0 && p.k % 256 <= 128 ? p.kb - 1 : -1;
}

template <int FMT>
__device__ __forceinline__ const uint8_t* unit_ptr(const Proj& p, int64_t e, int rgroup, int kb) {
  return p.data + e * p.dstride + ((int64_t)rgroup * p.kb + kb) * UnitBytes<FMT>::value;
}

// Workspace views written by the routing kernel and read by the GEMM kernels.
// A prefill tile: one 16-byte record, read by one scalar load.
struct alignas(16) PfTile {
  int expert, r0, nv, slot;  // expert id, first route position, routes (<= 128), active slot
};

struct MoeWs {
  int* hdr;          // [0] active experts, [1] routes, [2] prefill tiles
  int* active;       // [E] expert id per slot (ascending)
  int* act_off;      // [E+1] first route position of each slot
  PfTile* tile;      // [max tiles] prefill tiles (128 routes of one expert)
  float* ent_r;      // [B*k] merged BF16 route weight of an entry (0: no route)
  int* route_tok;    // [routes] token of each route, grouped by expert, tokens ascending
  float* route_w;    // [routes] its BF16 weight as FP32
  int* tok_pos;      // [B*k] per token: route positions in ascending expert id, -1 padded
  uint16_t* act;     // [B*k, I] BF16 SwiGLU activations
  uint16_t* y;       // [B*k, H] BF16 expert outputs
  uint16_t* sh_act;  // [B, Is]
  uint16_t* sh_y;    // [B, H]
};

// Where a workgroup's tokens come from: routed slots or the dense shared expert.
struct TokenSrc {
  int dense;            // 1: one slot, expert 0, tokens 0..B-1
  int tokens;           // B
  const int* hdr;
  const int* active;
  const int* act_off;
  const int* route_tok; // token of route position (phase 1 input rows)
};

// Decode path (small token counts): routing inputs and published tables.
struct DecRoute {
  const int32_t* ids;
  const uint16_t* wts;
  int B, K, E;
};

struct DecTables {
  int* hdr;          // [0] active experts, [1] routes, [8] call counter, [9] wait gave up (fused kernel)
  int* slot_e;       // [E] expert of slot
  int* slot_t0;      // [E] first route position
  int* slot_cnt;     // [E] routes
  int* tok_n;        // [B] routes of each token
  float* route_w;    // [routes] BF16 route weight as FP32
  int* route_dst;    // [routes] token-major slot b*K + rank (rank = ascending expert id)
};

// The always-on shared expert inside the decode-step launches (tokens <=
// kDecSharedTokens): its gate/up items run in the gate/up launch and its down
// items in the down launch, ahead of the routed ones, one item per 16-token
// pass. is == 0: no shared expert there.
struct DecShared {
  Proj gate, up, down;  // one expert: gate/up [is, H], down [H, is]
  int is;
  uint16_t* act;        // [B, is] SwiGLU activations
  uint16_t* y;          // [B, H] BF16 output
};

struct DecArgs {
  Proj gate, up, down;
  DecRoute R;
  DecTables T;
  DecShared S;
  const uint16_t* x;
  int H, I, max_slots;
  uint16_t* act;
  float* contrib;  // [B*K, H] FP32 f32(y) * f32(r), token-major
  uint64_t* flags; // [max_slots, I/16] per-call tags of the fused decode kernel (NULL: separate launches)
  const uint16_t* sh_y;
  const uint16_t* sh_scale;
  uint16_t* out;
  void* gate_up_start;  // optional hipEvent_t: the gate/up kernel's start (with after_gate_up, its end)
  void* after_gate_up;  // optional hipEvent_t
  void* after_down;     // optional hipEvent_t
};

// The decode-step kernels take the call: tokens, routes and experts within
// their limits, and routes x width (the largest of hidden, intermediate and
// shared intermediate) BF16 values within 32-bit byte offsets.
bool dec_supported(int64_t B, int64_t K, int64_t E, int64_t width);
constexpr int kDecSharedTokens = 64;  // the shared expert joins the decode launches up to this many tokens
int launch_moe_decode(int fmt_gu, int fmt_dn, const DecArgs& A, hipStream_t s);

// Unit-decode probes (q6moe_moe_unpack): the decode kernels' LDS-staged path
// and the prefill kernels' whole-block register path, for the bit-exact tests.
int launch_dec_unpack(int fmt, const Proj& p, int experts, uint16_t* out, hipStream_t s);
bool pf_unpack_supported(int fmt);
int launch_pf_unpack(int fmt, const Proj& p, int experts, uint16_t* out, hipStream_t s);

// Prefill grouped GEMM, tiled on the matrix cores: gate/up (Q6_K, Q8_0 or
// Q4_K; hidden a multiple of 128, intermediate of 64) and down (Q6_K, Q8_0,
// Q5_1 or Q4_K; intermediate a multiple of 128, hidden of 128), each launched
// on its own.
bool pf_gate_up_supported(int fmt, int64_t H, int64_t I);
bool pf_down_supported(int fmt, int64_t H, int64_t I);
int64_t pf_tile_routes();
int launch_moe_prefill_gate_up(int fmt, const Proj& g, const Proj& u, const MoeWs& ws, int max_tiles,
                               const uint16_t* x, int B, int H, int I, hipStream_t s, void* gate_up_start,
                               void* after_gate_up);
int launch_moe_prefill_down(int fmt, const Proj& d, const MoeWs& ws, int max_tiles, int routes, int H, int I,
                            hipStream_t s);

// ---------------------------------------------------------------------------
// Unit decoders: 16 output rows x one 256-wide K block -> 8 MFMA A operands.
// ---------------------------------------------------------------------------
template <int FMT>
struct Unit;

template <>
struct Unit<FMT_Q6> {
  u32x4 c0, c1, c2;  // the lane's code words (bit-planar, group g = word g)
  uint32_t sc;       // the lane's sub-scales: byte g = sub-block 4g + jA
  uint32_t d;        // FP16 bits of the row's block scale
  __device__ __forceinline__ void load(const Proj& p, int64_t e, int rgroup, int kb, int lane) {
    const uint8_t* u = unit_ptr<FMT_Q6>(p, e, rgroup, kb);
    c0 = ld16_stream(u + 16 * lane);
    c1 = ld16_stream(u + 1024 + 16 * lane);
    c2 = ld16_stream(u + 2048 + 16 * lane);
    sc = *reinterpret_cast<const uint32_t*>(u + 3072 + 4 * lane);
    d = *reinterpret_cast<const uint16_t*>(u + 3328 + 2 * (lane & 15));
  }
  __device__ __forceinline__ void decode(u32x4 a[8], int lane) const { q6p_decode(c0, c1, c2, sc, d, a); }
  static __device__ __forceinline__ int xoff(int f, int jA) { return q6_xfrag_offset(f, jA); }
};

// Q4_K unit. Lane (row l%16, chunk jA = l/16) decodes qs bytes [32jA, 32jA+32)
// of its row's block (chunks 1+2jA and 2+2jA): low nibbles are sub-block 2jA
// (positions 64jA + l), high nibbles sub-block 2jA+1 (64jA + 32 + l)
// (kaggle/glm53_offload/gguf_quant.py:115-157). w = fma(q, d*sc, -dmin*m),
// one rounding of the exact value, then RNE to BF16.
template <>
struct Unit<FMT_Q4K> {
  u32x4 hdr, qa, qb;
  __device__ __forceinline__ void load(const Proj& p, int64_t e, int rgroup, int kb, int lane) {
    const uint8_t* u = unit_ptr<FMT_Q4K>(p, e, rgroup, kb);
    const int j = lane & 15, jA = lane >> 4;
    hdr = ld16_stream(u + 16 * j);
    qa = ld16_stream(u + 16 * (16 * (1 + 2 * jA) + j));
    qb = ld16_stream(u + 16 * (16 * (2 + 2 * jA) + j));
  }
  __device__ __forceinline__ void decode(u32x4 a[8], int lane) const {
    const int jA = lane >> 4;
    const float d = half_bits_to_float(hdr[0] & 0xffff);
    const float dmin = half_bits_to_float(hdr[0] >> 16);
    // scale bytes: s = bytes 4..7 (hdr[1]), m = 8..11 (hdr[2]), x = 12..15 (hdr[3])
    float ds[2], dm[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * jA + h;
      int sc, mn;
      if (j < 4) {
        sc = (hdr[1] >> (8 * j)) & 63;
        mn = (hdr[2] >> (8 * j)) & 63;
      } else {
        const int jj = j - 4;
        const uint32_t xb = (hdr[3] >> (8 * jj)) & 0xff;
        sc = (int)((xb & 15) | (((hdr[1] >> (8 * jj)) >> 2) & 48));
        mn = (int)((xb >> 4) | (((hdr[2] >> (8 * jj)) >> 2) & 48));
      }
      ds[h] = d * (float)sc;
      dm[h] = -(dmin * (float)mn);
    }
    // Codes as FP16 subnormals (sub_frag): the low nibbles of bytes 0 and 2
    // of a word sit at bits 0-3 of its halves (q * 2^-24), the high nibbles at
    // bits 4-7 (q * 2^-20); bytes 1 and 3 the same after a shift by 8.
    const float s_lo = ds[0] * 16777216.f, s_hi = ds[1] * 1048576.f;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int hn = f >> 2, bg = f & 3;
      const u32x4& src = bg < 2 ? qa : qb;
      const uint32_t w0 = src[2 * (bg & 1)], w1 = src[2 * (bg & 1) + 1];
      const uint32_t m = hn ? 0x00F000F0u : 0x000F000Fu;
      a[f] = sub_frag(w0 & m, (w0 >> 8) & m, w1 & m, (w1 >> 8) & m, hn ? s_hi : s_lo, dm[hn]);
    }
  }
  static __device__ __forceinline__ int xoff(int f, int jA) {
    return 64 * jA + 32 * (f >> 2) + 8 * (f & 3);
  }
};

// Q8_0 unit: lane (row l%16, k-group jA = l/16) holds codes chunk g (fragments
// 2g, 2g+1) and the four FP16 scales of its blocks 2g + jA/2; w = d * q exact
// in FP32, RNE to BF16 (gguf_quant.py:111-114). Fragment positions are the
// Q6_K ones.
template <>
struct Unit<FMT_Q8> {
  u32x4 c[4];
  u32x2 d;
  __device__ __forceinline__ void load(const Proj& p, int64_t e, int rgroup, int kb, int lane) {
    const uint8_t* u = unit_ptr<FMT_Q8>(p, e, rgroup, kb);
#pragma unroll
    for (int g = 0; g < 4; ++g) c[g] = ld16_stream(u + 1024 * g + 16 * lane);
    d = *reinterpret_cast<const u32x2*>(u + 4096 + 8 * (2 * (lane & 15) + (lane >> 5)));
  }
  __device__ __forceinline__ void decode(u32x4 a[8], int) const { q8_decode<true>(c, d, a); }
  static __device__ __forceinline__ int xoff(int f, int jA) { return q6_xfrag_offset(f, jA); }
};

// The (K-)scale and min of sub-block jsub of a Q4_K / Q5_K header chunk
// (d, dmin, 12 packed 6-bit scale/min bytes; gguf_quant.py:118-135):
// ds = d * sc, dm = -(dmin * m), both exact.
__device__ __forceinline__ void k_scale_min(const u32x4& hdr, int jsub, float& ds, float& dm) {
  const float d = half_bits_to_float(hdr[0] & 0xffff);
  const float dmin = half_bits_to_float(hdr[0] >> 16);
  int sc, mn;
  if (jsub < 4) {
    sc = (hdr[1] >> (8 * jsub)) & 63;
    mn = (hdr[2] >> (8 * jsub)) & 63;
  } else {
    const int jj = jsub - 4;
    const uint32_t xb = (hdr[3] >> (8 * jj)) & 0xff;
    sc = (int)((xb & 15) | (((hdr[1] >> (8 * jj)) >> 2) & 48));
    mn = (int)((xb >> 4) | (((hdr[2] >> (8 * jj)) >> 2) & 48));
  }
  ds = d * (float)sc;
  dm = -(dmin * (float)mn);
}

// Q5_K unit: as Q4_K, with the 32 high-bit bytes (chunks 1-2; bit s of byte l
// is bit 4 of sub-block s at position l) before the nibbles (chunks 3-10).
// Lane (row l%16, jA = l/16) decodes qs bytes [32jA, 32jA+32): low nibbles are
// sub-block 2jA, high nibbles 2jA+1 (kaggle/glm53_offload/gguf_quant.py:137-157).
// w = fma(q, d*sc, -dmin*m): one rounding of the exact value, then RNE to BF16.
template <>
struct Unit<FMT_Q5K> {
  u32x4 hdr, qh0, qh1, qa, qb;
  __device__ __forceinline__ void load(const Proj& p, int64_t e, int rgroup, int kb, int lane) {
    const uint8_t* u = unit_ptr<FMT_Q5K>(p, e, rgroup, kb);
    const int j = lane & 15, jA = lane >> 4;
    hdr = ld16_stream(u + 16 * j);
    qh0 = ld16_stream(u + 16 * (16 + j));
    qh1 = ld16_stream(u + 16 * (32 + j));
    qa = ld16_stream(u + 16 * (16 * (3 + 2 * jA) + j));
    qb = ld16_stream(u + 16 * (16 * (4 + 2 * jA) + j));
  }
  __device__ __forceinline__ void decode(u32x4 a[8], int lane) const {
    const int jA = lane >> 4;
    float ds[2], dm[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) k_scale_min(hdr, 2 * jA + h, ds[h], dm[h]);
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int hn = f >> 2, bg = f & 3, s = 2 * jA + hn;
      const u32x4& src = bg < 2 ? qa : qb;
      const u32x4& qh = bg < 2 ? qh0 : qh1;
      uint32_t c0 = src[2 * (bg & 1)], c1 = src[2 * (bg & 1) + 1];
      c0 = (hn ? c0 >> 4 : c0) & 0x0f0f0f0fu;
      c1 = (hn ? c1 >> 4 : c1) & 0x0f0f0f0fu;
      c0 |= ((qh[2 * (bg & 1)] >> s) & 0x01010101u) << 4;
      c1 |= ((qh[2 * (bg & 1) + 1] >> s) & 0x01010101u) << 4;
      a[f] = q6_frag(c0, c1, ds[hn], dm[hn]);
    }
  }
  static __device__ __forceinline__ int xoff(int f, int jA) { return Unit<FMT_Q4K>::xoff(f, jA); }
};

// Bits 0-3 of ``h`` moved to bit 0 of bytes 0-3 (h * (1 + 2^7 + 2^14 + 2^21)
// places bit i at 8i; the shifted copies do not overlap, so nothing carries).
__device__ __forceinline__ uint32_t spread4(uint32_t h) { return ((h & 15u) * 0x00204081u) & 0x01010101u; }

// Q5_1 unit: lane (row j = l%16, jA = l/16) owns K positions 64g + 16jA + [0, 16)
// (fragments 2g, 2g+1): positions 16(jA%2) + [0, 16) of its block 2g + jA/2,
// i.e. the low (jA even) or high (jA odd) nibbles of the block's 16 bytes, with
// bit 16(jA%2) + i of the high word as bit 4. w = fma(q, d, m), one rounding of
// d*q + m (kaggle/qwen38_tpu/quant.py:34-53), then RNE to BF16.
template <>
struct Unit<FMT_Q51> {
  u32x4 q[4];
  u32x4 aux0, aux1;  // blocks 2g + jA/2 for g = 0, 1 and 2, 3: (high word, d | m << 16)
  __device__ __forceinline__ void load(const Proj& p, int64_t e, int rgroup, int kb, int lane) {
    const uint8_t* u = unit_ptr<FMT_Q51>(p, e, rgroup, kb);
    const int j = lane & 15, hb = lane >> 5;
#pragma unroll
    for (int g = 0; g < 4; ++g) q[g] = ld16_stream(u + 512 * g + 256 * hb + 16 * j);
    aux0 = ld16_stream(u + 2048 + 64 * j + 32 * hb);
    aux1 = ld16_stream(u + 2048 + 64 * j + 32 * hb + 16);
  }
  __device__ __forceinline__ void decode(u32x4 a[8], int lane) const {
    const int odd = (lane >> 4) & 1;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4& ax = g < 2 ? aux0 : aux1;
      const uint32_t qh = ax[2 * (g & 1)], dm = ax[2 * (g & 1) + 1];
      const float d = half_bits_to_float(dm & 0xffff), m = half_bits_to_float(dm >> 16);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        uint32_t c0 = q[g][2 * e], c1 = q[g][2 * e + 1];
        c0 = (odd ? c0 >> 4 : c0) & 0x0f0f0f0fu;
        c1 = (odd ? c1 >> 4 : c1) & 0x0f0f0f0fu;
        const uint32_t hb8 = qh >> (16 * odd + 8 * e);
        c0 |= spread4(hb8) << 4;
        c1 |= spread4(hb8 >> 4) << 4;
        a[2 * g + e] = q6_frag(c0, c1, d, m);
      }
    }
  }
  static __device__ __forceinline__ int xoff(int f, int jA) { return q6_xfrag_offset(f, jA); }
};

// Stores a lane's 8 decoded A fragments of unit (rg, kb) -- row rg*16 + lane%16,
// K positions kb*256 + xoff(f) + [0, 8) -- into out [p.rows, p.k] (BF16 bits),
// skipping positions past the matrix. Used by the unit-decode probes.
template <typename XOff>
__device__ __forceinline__ void store_unit_frags(const u32x4 (&a)[8], uint16_t* out, const Proj& p, int rg,
                                                 int kb, int lane, XOff xoff) {
  const int row = rg * 16 + (lane & 15);
  if (row >= p.rows) return;
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const int c0 = kb * kQK + xoff(f, lane >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c0 + i < p.k) out[(int64_t)row * p.k + c0 + i] = (uint16_t)(a[f][i >> 1] >> (16 * (i & 1)));
  }
}

}  // namespace q6moe
