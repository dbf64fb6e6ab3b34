// Prefill-shaped routed experts: tiled grouped GEMM on BF16 MFMA over
// unit-major expert tables (gate/up Q6_K, Q8_0 or Q4_K; down Q6_K, Q8_0, Q5_1
// or Q4_K).
//
// The routing kernel (moe.hip) groups the routes by expert (ascending id,
// tokens ascending) and splits each expert's routes into tiles of 128. One
// workgroup (4 waves, one per SIMD; two workgroups per CU) computes a tile
// against a block of output rows; an expert's last, partial tile runs only the
// 16-route column groups it needs, rounded up to 32 routes:
//
//   moe_pf_gate_up_kernel  64 intermediate rows (gate and up) per workgroup;
//        g = RNE(x Wg^T), u = RNE(x Wu^T), a = RNE(RNE(g*sigmoid(g))*u)
//        (kaggle/qwen38_tpu/experts.py:103-107, grouped_experts.py:96-101).
//   moe_pf_down_kernel     128 hidden rows per workgroup; y = RNE(a Wd^T)
//        (experts.py:108). The combine kernel in moe.hip sums f32(y)*f32(r).
//
// Each wave owns 2 units (16 weight rows x one 256-wide K block) per K block,
// loads a unit's bytes into one of two register sets during the previous
// block's first K half, and decodes each half straight into MFMA A operands;
// decoded weights never leave registers. K runs in halves of 128 (so K needs
// only be a multiple of 128: a last, half K block multiplies its first half,
// and the unit's zero padding beyond K is never decoded). The 128 token
// rows of the current K half sit in LDS (double-buffered, XOR-swizzled so the
// 16 token columns of an MFMA read hit distinct banks), filled by direct
// buffer->LDS DMA, and every wave multiplies them against its own rows. The
// two workgroups of a CU run out of step, so one's decode (VALU) overlaps the
// other's MFMAs.
#include <hip/hip_ext.h>

#include <type_traits>

#include "moe_common.h"
#include "q6moe_api.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(uint32_t)(uintptr_t)(p))

namespace q6moe {

namespace pf {

constexpr int kWaves = 4;
constexpr int kM = 128;            // routes per tile (MFMA column groups of 16)
constexpr int kUnits = 2;          // units per wave per K block
constexpr int kHalfBytes = kM * 128 * 2;  // one K half of the token tile (32 KB)
constexpr int kXStages = 2;        // token-tile stages in LDS: the K half being multiplied and the next
// A tile of NCG (2, 4, 6 or 8) 16-route column groups: the token rows of a K
// half take NCG KB per wave, i.e. NCG DMA instructions of 1 KB per wave.
constexpr int kLds = kXStages * kHalfBytes;

static_assert(kLds <= 160 * 1024, "LDS budget");

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Wave index as a wave-uniform (SGPR) value, so that row groups and the
// weight addresses derived from it stay in scalar registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
// Direct buffer->LDS DMA of 16 bytes per lane: byte offset voff (per lane)
// plus soff (wave-uniform) into the buffer r, no address arithmetic in VGPRs;
// an offset past the buffer's end reads zeros.
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(lds), 16, voff, soff, 0, 0);
}
// Workgroup barrier without the memory fence of __syncthreads (whose release
// would wait for every outstanding DMA, including the ones prefetching the
// next stage). LDS visibility comes from each wave's own vmcnt wait before it.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The weights of one unit (a whole K block) in the registers of the lane that
// decodes them (row j = lane % 16, k-group jA = lane / 16); both K halves
// decode from one load. ``load`` issues kLoads vector-memory instructions
// (``half``: only the first K half is used, and a 32-value format re-reads
// its first half's code words for the second instead of the zero padding);
// ``half(h)`` gives the 4 A fragments of K half h; ``gran(f, jA)`` is the
// 8-column granule, within the half, of fragment f for k-group jA (the token
// operand it pairs with); ``pin`` makes the registers opaque to the compiler.
template <int FMT>
struct Block;

// Q6_K (bit-planar unit): the lane's four code words of each of the three code
// chunks, its sub-scale word and the row's FP16 scale. Fragment 2g + e of the
// unit covers positions 64g + 16jA + 8e + [0, 8) (q6_xfrag_offset).
template <>
struct Block<FMT_Q6> {
  static constexpr int kLoads = 5;
  u32x4 c0, c1, c2;
  uint32_t sc, d;
  __device__ __forceinline__ void load(const uint8_t* v, int lane, bool = false) {
    c0 = *reinterpret_cast<const u32x4*>(v + 16 * lane);
    c1 = *reinterpret_cast<const u32x4*>(v + 1024 + 16 * lane);
    c2 = *reinterpret_cast<const u32x4*>(v + 2048 + 16 * lane);
    sc = *reinterpret_cast<const uint32_t*>(v + 3072 + 4 * lane);
    d = *reinterpret_cast<const uint16_t*>(v + 3328 + 2 * (lane & 15));
  }
  __device__ __forceinline__ void pin() { asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(sc), "+v"(d)); }
  __device__ __forceinline__ void half(int h, int, u32x4 a[4]) const {
    const float dd = half_bits_to_float(d);
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
      q6p_group(c0[2 * h + gg], c1[2 * h + gg], c2[2 * h + gg], q6p_ds(dd, sc, 2 * h + gg), a[2 * gg],
                a[2 * gg + 1]);
  }
  static __device__ __forceinline__ int gran(int f, int jA) { return 8 * (f >> 1) + 2 * jA + (f & 1); }
};

// Q8_0: the lane's four code chunks (chunk g: fragments 2g, 2g+1 at the Q6_K
// positions) and the FP16 scales of its blocks 2g + jA/2; w = d * q exact,
// RNE to BF16 (gguf_quant.py:111-114).
template <>
struct Block<FMT_Q8> {
  static constexpr int kLoads = 5;
  u32x4 c[4];
  u32x2 dw;
  __device__ __forceinline__ void load(const uint8_t* v, int lane, bool half = false) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      c[g] = *reinterpret_cast<const u32x4*>(v + 1024 * (half ? g & 1 : g) + 16 * lane);
    dw = *reinterpret_cast<const u32x2*>(v + 4096 + 8 * (2 * (lane & 15) + (lane >> 5)));
  }
  __device__ __forceinline__ void pin() { asm volatile("" : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(dw)); }
  __device__ __forceinline__ void half(int h, int, u32x4 a[4]) const {
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int g = 2 * h + gg;
      const float d = half_bits_to_float((dw[g >> 1] >> (16 * (g & 1))) & 0xffffu);
      a[2 * gg] = q8_frag<true>(c[g][0], c[g][1], d);
      a[2 * gg + 1] = q8_frag<true>(c[g][2], c[g][3], d);
    }
  }
  static __device__ __forceinline__ int gran(int f, int jA) { return Block<FMT_Q6>::gran(f, jA); }
};

// Q5_1: the lane's four nibble chunks (chunk g: fragments 2g, 2g+1 at the
// Q6_K positions, the low or high nibbles of block 2g + jA/2) and the blocks'
// high-bit words and FP16 d, m; w = fma(q, d, m), one rounding, RNE to BF16
// (kaggle/qwen38_tpu/quant.py:34-53).
template <>
struct Block<FMT_Q51> {
  static constexpr int kLoads = 6;
  u32x4 q[4];
  u32x4 aux[2];  // blocks 2g + jA/2 of g = 0, 1 and of g = 2, 3: (high word, d | m << 16)
  __device__ __forceinline__ void load(const uint8_t* v, int lane, bool half = false) {
    const int j = lane & 15, hb = lane >> 5;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      q[g] = *reinterpret_cast<const u32x4*>(v + 512 * (half ? g & 1 : g) + 256 * hb + 16 * j);
    aux[0] = *reinterpret_cast<const u32x4*>(v + 2048 + 64 * j + 32 * hb);
    aux[1] = *reinterpret_cast<const u32x4*>(v + 2048 + 64 * j + 32 * hb + 16);
  }
  __device__ __forceinline__ void pin() {
    asm volatile("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(aux[0]), "+v"(aux[1]));
  }
  __device__ __forceinline__ void half(int h, int lane, u32x4 a[4]) const {
    const int odd = (lane >> 4) & 1;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int g = 2 * h + gg;
      const uint32_t qh = aux[h][2 * gg], dm = aux[h][2 * gg + 1];
      const float d = half_bits_to_float(dm & 0xffff), m = half_bits_to_float(dm >> 16);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        uint32_t c0 = q[g][2 * e], c1 = q[g][2 * e + 1];
        c0 = (odd ? c0 >> 4 : c0) & 0x0f0f0f0fu;
        c1 = (odd ? c1 >> 4 : c1) & 0x0f0f0f0fu;
        const uint32_t hb8 = qh >> (16 * odd + 8 * e);
        c0 |= spread4(hb8) << 4;
        c1 |= spread4(hb8 >> 4) << 4;
        a[2 * gg + e] = q6_frag(c0, c1, d, m);
      }
    }
  }
  static __device__ __forceinline__ int gran(int f, int jA) { return Block<FMT_Q6>::gran(f, jA); }
};

// Q4_K, with a lane map of its own (the unit's bytes are those of the other
// kernels): in K half h the lane decodes sub-block 4h + jA, positions
// 128h + 32jA + [0, 32), i.e. the low (jA even) or high (jA odd) nibbles of
// its row's qs bytes 32(2h + jA/2) + [0, 32) (chunks 1 + 2c and 2 + 2c of the
// unit, c = 2h + jA/2); fragment f holds positions 8f + [0, 8) of it. The
// codes enter v_fma_mix_f32 as FP16 subnormals (sub_frag): w = fma(q, d*sc,
// -dmin*m), one rounding, RNE to BF16 (gguf_quant.py:115-157).
template <>
struct Block<FMT_Q4K> {
  static constexpr int kLoads = 5;
  u32x4 hdr;
  u32x4 qs[2][2];  // [half][chunk]
  __device__ __forceinline__ void load(const uint8_t* v, int lane, bool = false) {
    const int j = lane & 15, jA = lane >> 4;
    hdr = *reinterpret_cast<const u32x4*>(v + 16 * j);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 2 * h + (jA >> 1);
      qs[h][0] = *reinterpret_cast<const u32x4*>(v + 16 * (16 * (1 + 2 * c) + j));
      qs[h][1] = *reinterpret_cast<const u32x4*>(v + 16 * (16 * (2 + 2 * c) + j));
    }
  }
  __device__ __forceinline__ void pin() {
    asm volatile("" : "+v"(hdr), "+v"(qs[0][0]), "+v"(qs[0][1]), "+v"(qs[1][0]), "+v"(qs[1][1]));
  }
  __device__ __forceinline__ void half(int h, int lane, u32x4 a[4]) const {
    const int jA = lane >> 4, odd = jA & 1;
    const float d = half_bits_to_float(hdr[0] & 0xffff);
    const float dmin = half_bits_to_float(hdr[0] >> 16);
    // sub-block 4h + jA: its 6-bit scale and min (gguf_quant.py:118-135)
    uint32_t scb, mnb;
    if (h == 0) {
      scb = (hdr[1] >> (8 * jA)) & 63;
      mnb = (hdr[2] >> (8 * jA)) & 63;
    } else {
      const uint32_t xb = hdr[3] >> (8 * jA);
      scb = (xb & 15) | ((hdr[1] >> (8 * jA + 2)) & 48);
      mnb = ((xb >> 4) & 15) | ((hdr[2] >> (8 * jA + 2)) & 48);
    }
    const float ds = d * (float)scb, dm = -(dmin * (float)mnb);
    const uint32_t m = odd ? 0x00F000F0u : 0x000F000Fu;
    const float s = ds * (odd ? 1048576.f : 16777216.f);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const uint32_t w0 = qs[h][f >> 1][2 * (f & 1)], w1 = qs[h][f >> 1][2 * (f & 1) + 1];
      a[f] = sub_frag(w0 & m, (w0 >> 8) & m, w1 & m, (w1 >> 8) & m, s, dm);
    }
  }
  static __device__ __forceinline__ int gran(int f, int jA) { return 4 * jA + f; }
};

// K position, inside a 256-wide block, of fragment f (0..7: K half f / 4) of k-group jA.
template <int FMT>
__device__ __forceinline__ int block_xoff(int f, int jA) {
  return 128 * (f >> 2) + 8 * Block<FMT>::gran(f & 3, jA);
}

// LDS byte offset of token-tile granule (token t, 8-column granule c) of a K half.
__device__ __forceinline__ int xgran(int t, int c) { return (t * 16 + (c ^ (t & 15))) * 16; }

struct Tile {
  int64_t expert;
  int r0, nv;  // first route position, valid routes (<= kM)
};

// Work item of workgroup blockIdx.x: (tile, column block), column block
// fastest. Workgroup i runs on XCD i % 8 (round-robin dispatch), so the items
// are split into eight contiguous runs, one per XCD, each walked in dispatch
// order: the workgroups that share a token tile (its column blocks) or an
// expert's weights (its tiles) run on one XCD at the same time and share its
// L2. Returns false past the last item.
__device__ __forceinline__ bool pf_item(const MoeWs& ws, int ncol, int& tile, int& col) {
  const int ntiles = ws.hdr[2];
  const int items = ntiles * ncol;
  const int run = (items + 7) >> 3;
  const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int item = xcd * run + k;
  if (k >= run || item >= items) return false;
  tile = item / ncol;
  col = item - tile * ncol;
  return true;
}

__device__ __forceinline__ void tile_info(const MoeWs& ws, int tile, Tile& T) {
  const PfTile d = ws.tile[tile];  // one scalar load
  T.expert = d.expert;
  T.r0 = d.r0;
  T.nv = d.nv;
}

// Token rows of this wave's token-tile DMA: instruction i fills granules
// (wave*NCG + i)*64 + lane, i.e. token t = that/16. All rows are read before
// any is used, so a row table's loads are in flight together.
template <int NCG, typename RowOf>
__device__ __forceinline__ void tile_rows(int (&rows)[NCG], RowOf row_of) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < NCG; ++i) rows[i] = row_of(((wave * NCG + i) * 64 + lane) >> 4);
}

// Per-lane byte offsets of those DMA instructions: row rows[i], swizzled
// granule (p % 16) ^ (t % 16) of p = (wave*NCG + i)*64 + lane, t = p/16.
template <int NCG>
__device__ __forceinline__ void x_offsets(uint32_t (&xoff)[NCG], const int (&rows)[NCG], int K) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < NCG; ++i) {
    const int p = (wave * NCG + i) * 64 + lane;
    const int t = p >> 4, c = (p & 15) ^ (t & 15);
    xoff[i] = opaque((uint32_t)((rows[i] * K + c * 8) * 2));
  }
}

// The streaming core shared by both kernels. ``rg_of(u)`` gives unit u's row
// group and ``row_of(t)`` the x row of the tile's token t; the token rows come
// in by DMA at per-lane offsets computed in the prologue.
// K half s (block s/2, half s%2) is step s. Each wave DMAs its share of the
// token tile into LDS stage s % kXStages one step before it is multiplied,
// and loads its own weights into registers a step and a half ahead; one
// workgroup barrier per step makes every wave's share visible and frees the
// stage read in the step before. The next step's loads go out in four parts,
// one after each fragment's MFMAs (the two halves of the token DMA, then, in a
// first-half step, the next block's weights for unit 0 and unit 1), so that
// the four waves of a workgroup do not all queue their vector-memory
// instructions at once right after the barrier.
// kEven: K is a multiple of 256 (whole K blocks); the loop then runs its
// steps in pairs with no branch between a block's two halves.
template <int FMT, int NCG, bool kEven, typename RowFn, typename RowOf>
__device__ __forceinline__ void pf_stream(uint8_t* smem, const Proj* projs, const int* unit_proj, RowFn rg_of,
                                          const uint16_t* x, int x_rows, RowOf row_of, int K, int64_t expert,
                                          f32x4 (&acc)[kUnits][NCG]) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int j = lane & 15, jA = lane >> 4;
  const int S = K / 128;           // K halves (K is a multiple of 128)
  const int kbs = (S + 1) >> 1;    // K blocks of the table, the last one possibly half used
  const bool odd = !kEven && (S & 1);
  constexpr int kWLoads = Block<FMT>::kLoads;
  constexpr int kUB = UnitBytes<FMT>::value;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)((uint32_t)x_rows * (uint32_t)K * 2u), 0x00020000);
  const uint8_t* units[kUnits];
  int rgs[kUnits];
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const Proj& p = projs[unit_proj[u]];
    units[u] = p.data + expert * p.dstride;
    rgs[u] = rg_of(u);
  }
  // Two register sets per unit, one per K block parity: block b+1's weights
  // are loaded during the first half of block b (after that step's token
  // DMA), so they have a step and a half to arrive; the second-half step that
  // follows waits only for its token DMA.
  static_assert(kXStages == 2, "two K halves per block");
  Block<FMT> wr[2][kUnits];
  uint32_t xoff[NCG];  // per-lane byte offsets of the token rows, set in the prologue
  // Issued step s (the step after the current one): token DMA in parts 0 and
  // 1; for a second-half s (block b = s/2), block b+1's weights in parts 2
  // and 3 (unit part-2) into register set ``wset``.
  auto issue_part = [&](int s, auto slot_c, auto part_c, auto wset_c) {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int part = decltype(part_c)::value;
    constexpr int wset = decltype(wset_c)::value;
    const int kb = s >> 1, h = s & 1;
    if constexpr (part < 2) {
      static_assert(NCG % 2 == 0, "the token DMA splits evenly over two parts");
      constexpr int per = NCG / 2, i0 = part * per;
      uint8_t* xs = smem + slot * kHalfBytes + wave * NCG * 1024;
#pragma unroll
      for (int i = i0; i < i0 + per; ++i) bdma16(xr, xoff[i], (uint32_t)(kb * kQK + h * 128) * 2u, xs + i * 1024);
    } else if constexpr (slot == 1 && part - 2 < kUnits) {
      if (kb + 1 < kbs)
        wr[wset][part - 2].load(units[part - 2] + ((int64_t)rgs[part - 2] * kbs + kb + 1) * kUB, lane,
                                kb + 2 == kbs && odd);
    }
  };
  auto step = [&](int s, auto slot_c, auto set_c) {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int set = decltype(set_c)::value;
    // this step's token DMA has landed once at most the next block's weight
    // loads (issued after it, in a first-half step) remain
    if (slot == 1 && (s >> 1) + 1 < kbs)
      wait_vm<kUnits * kWLoads>();
    else
      wait_vm<0>();
    wg_barrier();  // every wave's share of this step's tile is in LDS; the oldest stage is free
    // The wait above covered this block's weight registers. Re-define them
    // here so that the compiler does not also wait, after the next step's
    // loads are issued, for everything in flight before decoding them.
#pragma unroll
    for (int u = 0; u < kUnits; ++u) wr[set][u].pin();
    const bool more = s + 1 < S;
    const uint8_t* xs = smem + slot * kHalfBytes;
    u32x4 a[kUnits][4];
#pragma unroll
    for (int u = 0; u < kUnits; ++u) wr[set][u].half(slot, lane, a[u]);  // slot == s % 2 == h
    static_for<0, 4>([&](auto fc) {
      constexpr int f = decltype(fc)::value;
      const int c = Block<FMT>::gran(f, jA);
#pragma unroll
      for (int tg = 0; tg < NCG; ++tg) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + xgran(tg * 16 + j, c));
#pragma unroll
        for (int u = 0; u < kUnits; ++u) acc[u][tg] = mfma16(a[u][f], xv, acc[u][tg]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (more)
        issue_part(s + 1, std::integral_constant<int, 1 - slot>{}, fc, std::integral_constant<int, 1 - set>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // prologue: the tile's token rows (a table read, for gate/up), block 0's
  // weights, then step 0's token DMA once the rows have arrived; the weights
  // are in flight meanwhile
  {
    int rows[NCG];
    tile_rows(rows, row_of);
#pragma unroll
    for (int u = 0; u < kUnits; ++u) wr[0][u].load(units[u] + (int64_t)rgs[u] * kbs * kUB, lane, odd && S == 1);
    asm volatile("" ::: "memory");  // every load above issues before the offsets wait on the rows
    x_offsets(xoff, rows, K);
  }
  static_for<0, 2>([&](auto pc) {
    issue_part(0, std::integral_constant<int, 0>{}, pc, std::integral_constant<int, 1>{});
  });
  for (int s0 = 0; s0 < S; s0 += 4) {
    step(s0, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    if constexpr (kEven) {
      step(s0 + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
      if (s0 + 2 < S) {
        step(s0 + 2, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
        step(s0 + 3, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
      }
    } else {
      if (s0 + 1 < S) step(s0 + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
      if (s0 + 2 < S) step(s0 + 2, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
      if (s0 + 3 < S) step(s0 + 3, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    }
  }
}

// Calls f(std::integral_constant<int, NCG>) for the tile's column groups: its
// valid routes rounded up to 32 (2, 4, 6 or 8 groups of 16), so a partial tile
// issues only the MFMAs and token DMA of the routes it holds.
template <typename F>
__device__ __forceinline__ void with_column_groups(int nv, F&& f) {
  switch ((nv + 31) >> 5) {
    case 1: f(std::integral_constant<int, 2>{}); break;
    case 2: f(std::integral_constant<int, 4>{}); break;
    case 3: f(std::integral_constant<int, 6>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
  }
}

}  // namespace pf

template <int FMT>
__global__ void __launch_bounds__(64 * pf::kWaves, 2)
    moe_pf_gate_up_kernel(Proj gate, Proj up, MoeWs ws, const uint16_t* __restrict__ x, int tokens, int hidden,
                          uint16_t* __restrict__ act, int inter) {
  using namespace pf;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  Tile T;
  int tile, col;
  if (!pf_item(ws, inter / (16 * kWaves), tile, col)) return;
  tile_info(ws, tile, T);
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rgb = col * kWaves + wave;  // this wave's row group (gate and up)
  with_column_groups(T.nv, [&](auto ncg_c) {
    constexpr int NCG = decltype(ncg_c)::value;
    const Proj projs[2] = {gate, up};
    const int unit_proj[kUnits] = {0, 1};
    f32x4 acc[kUnits][NCG];
#pragma unroll
    for (int u = 0; u < kUnits; ++u)
#pragma unroll
      for (int t = 0; t < NCG; ++t) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto row_of = [&](int t) { return ws.route_tok[T.r0 + (t < T.nv ? t : T.nv - 1)]; };
    if (hidden % 256 == 0)
      pf_stream<FMT, NCG, true>(smem, projs, unit_proj, [&](int) { return rgb; }, x, tokens, row_of, hidden,
                                T.expert, acc);
    else
      pf_stream<FMT, NCG, false>(smem, projs, unit_proj, [&](int) { return rgb; }, x, tokens, row_of, hidden,
                                 T.expert, acc);
    const int row = rgb * 16 + 4 * jA;
#pragma unroll
    for (int tg = 0; tg < NCG; ++tg) {
      const int q = tg * 16 + j;
      if (q < T.nv) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = bf16_round(acc[0][tg][i]);
          const float u = bf16_round(acc[1][tg][i]);
          v[i] = bf16_round(g * sigmoid_acc(g)) * u;
        }
        u32x2 o;
        o[0] = pack_bf16x2(v[0], v[1]);
        o[1] = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<u32x2*>(act + (int64_t)(T.r0 + q) * inter + row) = o;
      }
    }
  });
}

template <int FMT>
__global__ void __launch_bounds__(64 * pf::kWaves, 2)
    moe_pf_down_kernel(Proj down, MoeWs ws, const uint16_t* __restrict__ act, int routes, int inter,
                       uint16_t* __restrict__ y, int hidden) {
  using namespace pf;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  Tile T;
  int tile, col;
  if (!pf_item(ws, hidden / (32 * kWaves), tile, col)) return;
  tile_info(ws, tile, T);
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rgb = col * 2 * kWaves + 2 * wave;  // this wave's two row groups
  with_column_groups(T.nv, [&](auto ncg_c) {
    constexpr int NCG = decltype(ncg_c)::value;
    const Proj projs[1] = {down};
    const int unit_proj[kUnits] = {0, 0};
    f32x4 acc[kUnits][NCG];
#pragma unroll
    for (int u = 0; u < kUnits; ++u)
#pragma unroll
      for (int t = 0; t < NCG; ++t) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto row_of = [&](int t) { return T.r0 + (t < T.nv ? t : T.nv - 1); };
    if (inter % 256 == 0)
      pf_stream<FMT, NCG, true>(smem, projs, unit_proj, [&](int u) { return rgb + u; }, act, routes, row_of, inter,
                                T.expert, acc);
    else
      pf_stream<FMT, NCG, false>(smem, projs, unit_proj, [&](int u) { return rgb + u; }, act, routes, row_of, inter,
                                 T.expert, acc);
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      const int row = (rgb + u) * 16 + 4 * jA;
#pragma unroll
      for (int tg = 0; tg < NCG; ++tg) {
        const int q = tg * 16 + j;
        if (q < T.nv) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[u][tg][0], acc[u][tg][1]);
          o[1] = pack_bf16x2(acc[u][tg][2], acc[u][tg][3]);
          *reinterpret_cast<u32x2*>(y + (int64_t)(T.r0 + q) * hidden + row) = o;
        }
      }
    }
  });
}

// The tiled kernels take K in halves of 128 and whole workgroup row blocks:
// gate/up 64 intermediate rows, down 128 hidden rows.
bool pf_gate_up_supported(int fmt, int64_t H, int64_t I) {
  return (fmt == FMT_Q6 || fmt == FMT_Q8 || fmt == FMT_Q4K) && H % 128 == 0 && I % (16 * pf::kWaves) == 0;
}
bool pf_down_supported(int fmt, int64_t H, int64_t I) {
  return (fmt == FMT_Q6 || fmt == FMT_Q8 || fmt == FMT_Q51 || fmt == FMT_Q4K) && I % 128 == 0 &&
         H % (32 * pf::kWaves) == 0;
}

int64_t pf_tile_routes() { return pf::kM; }

template <typename F>
static void dispatch_pf_format(int fmt, F&& f) {
  switch (fmt) {
    case FMT_Q8: f(std::integral_constant<int, FMT_Q8>{}); break;
    case FMT_Q51: f(std::integral_constant<int, FMT_Q51>{}); break;
    case FMT_Q4K: f(std::integral_constant<int, FMT_Q4K>{}); break;
    default: f(std::integral_constant<int, FMT_Q6>{}); break;
  }
}

static dim3 pf_grid(int ncol, int max_tiles) { return dim3((unsigned)(((int64_t)ncol * max_tiles + 7) / 8 * 8)); }

int launch_moe_prefill_gate_up(int fmt, const Proj& g, const Proj& u, const MoeWs& ws, int max_tiles,
                               const uint16_t* x, int B, int H, int I, hipStream_t s, void* gate_up_start,
                               void* after_gate_up) {
  dispatch_pf_format(fmt, [&](auto fc) {
    constexpr int FMT = decltype(fc)::value;
    static std::atomic<uint64_t> attr_done{0};
    once_per_device(attr_done, [] {
      (void)hipFuncSetAttribute((const void*)moe_pf_gate_up_kernel<FMT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                pf::kLds);
    });
    const dim3 grid = pf_grid(I / (16 * pf::kWaves), max_tiles);
    if (gate_up_start && after_gate_up) {
      // the events take the kernel's own start and end timestamps
      hipExtLaunchKernelGGL(moe_pf_gate_up_kernel<FMT>, grid, dim3(64 * pf::kWaves), pf::kLds, s,
                            (hipEvent_t)gate_up_start, (hipEvent_t)after_gate_up, 0, g, u, ws, x, B, H, ws.act, I);
    } else {
      hipLaunchKernelGGL(moe_pf_gate_up_kernel<FMT>, grid, dim3(64 * pf::kWaves), pf::kLds, s, g, u, ws, x, B, H,
                         ws.act, I);
      if (after_gate_up) (void)hipEventRecord((hipEvent_t)after_gate_up, s);
    }
  });
  return Q6MOE_OK;
}

int launch_moe_prefill_down(int fmt, const Proj& d, const MoeWs& ws, int max_tiles, int routes, int H, int I,
                            hipStream_t s) {
  dispatch_pf_format(fmt, [&](auto fc) {
    constexpr int FMT = decltype(fc)::value;
    static std::atomic<uint64_t> attr_done{0};
    once_per_device(attr_done, [] {
      (void)hipFuncSetAttribute((const void*)moe_pf_down_kernel<FMT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                pf::kLds);
    });
    hipLaunchKernelGGL(moe_pf_down_kernel<FMT>, pf_grid(H / (32 * pf::kWaves), max_tiles), dim3(64 * pf::kWaves),
                       pf::kLds, s, d, ws, ws.act, routes, I, ws.y, H);
  });
  return Q6MOE_OK;
}

// Unit-decode probe of this path: Block::load and Block::half of both K
// halves, the prefill kernels' register path. grid (units per expert, experts).
template <int FMT>
__global__ void __launch_bounds__(64) moe_pf_unpack_kernel(Proj p, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x;
  const int e = blockIdx.y, rg = blockIdx.x / p.kb, kb = blockIdx.x - rg * p.kb;
  pf::Block<FMT> w;
  w.load(p.data + (int64_t)e * p.dstride + ((int64_t)rg * p.kb + kb) * UnitBytes<FMT>::value, lane);
  u32x4 a[8];
  w.half(0, lane, a);
  w.half(1, lane, a + 4);
  store_unit_frags(a, out + (int64_t)e * p.rows * p.k, p, rg, kb, lane,
                   [](int f, int jA) { return pf::block_xoff<FMT>(f, jA); });
}

bool pf_unpack_supported(int fmt) { return fmt == FMT_Q6 || fmt == FMT_Q8 || fmt == FMT_Q51 || fmt == FMT_Q4K; }

int launch_pf_unpack(int fmt, const Proj& p, int experts, uint16_t* out, hipStream_t s) {
  const dim3 grid((unsigned)(cdiv(p.rows, 16) * p.kb), (unsigned)experts);
  dispatch_pf_format(fmt, [&](auto fc) {
    hipLaunchKernelGGL(moe_pf_unpack_kernel<decltype(fc)::value>, grid, dim3(64), 0, s, p, out);
  });
  return Q6MOE_OK;
}

}  // namespace q6moe
