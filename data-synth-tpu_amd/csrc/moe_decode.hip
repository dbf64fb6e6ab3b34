// Decode-shaped routed experts: three launches per step, one wave per workgroup.
//
//   moe_dec_gate_up_kernel  grid (16-row group, expert slot). The wave derives
//        the (small) routing itself -- merged BF16 route weight per (token,
//        expert) (kaggle/qwen38_tpu/experts.py:66-73), active experts in
//        ascending id (:74-76), the slot's tokens ascending -- then streams its
//        16 rows of gate and up over the full K and applies SwiGLU in
//        registers: a = RNE(RNE(g * sigmoid(g)) * u) (experts.py:103-107).
//        Row group 0 of every slot publishes that slot's routing tables.
//   moe_dec_down_kernel     grid (block of kDownRows row groups, expert slot).
//        The wave streams its rows of down, y = RNE(a Wd^T) (experts.py:108),
//        and stores the exact FP32 product f32(y) * f32(r) token-major at the
//        route's rank among its token's experts (ascending expert id).
//   moe_dec_combine_kernel  out = RNE(sum over ranks of the contributions),
//        i.e. the FP32 sum over experts in ascending id (experts.py:129-131),
//        plus RNE(routed + shared) with a shared expert (engine.py:199-203).
//
// Memory pipeline: each wave owns a ring of kStages weight units (16 rows x
// one 256-wide K block) in LDS, filled by direct global->LDS DMA
// (global_load_lds) kStages-1 units ahead of the unit being decoded, so bytes
// in flight cost no registers. The token operands of a K block (at most 16
// tokens: one per MFMA column) are loaded into one of two register sets
// together with the first unit of the previous K block. Every wait count is a
// compile-time constant of the unit's position in its K block. One-wave
// workgroups spread the waves evenly over the SIMDs. Weights are read once
// per 16 routes of an expert.
#include <hip/hip_ext.h>

#include <type_traits>

#include "moe_common.h"
#include "q6moe_api.h"

// LDS address of a generic pointer into shared memory (its low 32 bits).
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(uint32_t)(uintptr_t)(p))

namespace q6moe {

constexpr int kDecMaxEntries = 1024;  // tokens * top_k handled by the decode path
constexpr int kDecMaxTokens = 256;    // tokens handled by the decode path
constexpr int kMaskWords = kMaxExperts / 32;  // expert bit mask of the small-batch routing
constexpr int kStages = 3;
constexpr int kDownRows = 4;  // 16-row groups of down per wave
constexpr int kPassTokens = 16;  // routes per weight pass (MFMA columns)

// One ring stage holds a unit as its DMA writes it (Q4_K 2304 B, Q5_K
// 2816 B, Q5_1 3072 B, Q8_0 4352 B; Q6_K 3360 B with its FP16 scales repeated
// up to 3584 B).
template <int FMT>
constexpr int stage_bytes() {
  return FMT == FMT_Q8 ? 4352 : FMT == FMT_Q4K ? 2304 : FMT == FMT_Q5K ? 2816 : FMT == FMT_Q51 ? 3072 : 3584;
}
template <int FMT>
constexpr int ring_bytes() { return kStages * stage_bytes<FMT>(); }
constexpr int kXLoads = 8;   // token-operand loads per K block (one per MFMA)

// Per-wave LDS of the gate/up kernel: the weight ring, which the routing
// scratch overlays before the ring fills (for up to 64 entries the expert bit
// mask; for more: ids, merged weights and per-expert counts, 8 bytes per
// entry plus 4 per expert rounded up to 256 experts), then the slot's token
// list. Sized per launch, so that a layer with small units and few routes
// keeps more waves per CU.
__host__ __device__ constexpr int route_scratch_bytes(int n, int experts) {
  return n > 64 ? 8 * ((n + 3) & ~3) + 4 * ((experts + 255) & ~255) : 4 * kMaskWords;
}
template <int FMT>
__host__ __device__ constexpr int gu_wave_lds(int n, int experts) {
  const int r = ring_bytes<FMT>(), sc = route_scratch_bytes(n, experts);
  return (((r > sc ? r : sc) + 255) & ~255) + 4 * kDecMaxTokens;
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Stream addresses are a wave-uniform base (SGPRs) plus a 32-bit per-lane
// offset that stays in one VGPR for the whole stream.
// (readfirstlane pins the base to SGPRs so the load uses the SGPR-base form.)
__device__ __forceinline__ const uint8_t* sgpr_ptr(const uint8_t* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(((uint64_t)hi << 32) | lo);
}
// Hides how a per-lane offset was formed, so that no constant part of it is
// re-associated into a 64-bit per-lane address.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t voff, void* lds_base) {
  __builtin_amdgcn_global_load_lds(sgpr_ptr(base) + voff, LDS_PTR(lds_base), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const uint8_t* base, uint32_t voff, void* lds_base) {
  __builtin_amdgcn_global_load_lds(sgpr_ptr(base) + voff, LDS_PTR(lds_base), 4, 0, 0);
}

// Token operands are read through a buffer resource (base in SGPRs).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(n) with lgkmcnt/expcnt left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Device-scope (all XCDs) relaxed accesses: stores written through to the
// coherence point (sc1) and loads that read from it. The fused decode kernel
// passes the gate/up items' activations and routing tables to its down items
// on other XCDs this way: a producer's stores complete (s_waitcnt vmcnt(0))
// before its flag store, and a consumer issues its loads after it has read
// every flag it needs.
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The flag value of one call: a function of the workspace's call counter
// that is odd (never 0) and differs between consecutive calls.
__device__ __forceinline__ uint64_t sync_tag(uint32_t epoch) {
  return ((uint64_t)epoch + 1ull) * 0x9E3779B97F4A7C15ull | 1ull;
}
constexpr int kHdrEpoch = 8;   // hdr word: calls of the fused kernel on this workspace (any start value)
constexpr int kHdrStall = 9;   // hdr word: set when a down item gave up waiting (outputs marked NaN)
constexpr int kSpinLimit = 1 << 22;  // polls of a waiting down item (64-cycle sleeps, about 0.1 s)

// Vector-memory instructions issued for unit p of P per K block: the unit's
// D DMA instructions, plus the next K block's token operands with unit 0.
template <int P, int D>
constexpr int unit_ops(int p) {
  return D + (p % P == 0 ? kXLoads : 0);
}
template <int P, int D>
constexpr int younger_ops(int p, int ahead) {
  int s = 0;
  for (int i = 1; i <= ahead; ++i) s += unit_ops<P, D>(p + i);
  return s;
}

// One expert's projection streamed as units of 16 rows x one K block into a
// ring stage; decode() turns a stage into the 8 MFMA A operands of the lane.
template <int FMT>
struct WStream;

template <>
struct WStream<FMT_Q6> {
  static constexpr int kDma = 5;  // DMA instructions per unit
  const uint8_t* data;            // the expert's units
  int kbs;
  uint32_t v16, v4, v_d;  // per-lane byte offsets
  __device__ __forceinline__ WStream(const Proj& p, int64_t e, int lane) {
    data = p.data + e * p.dstride;
    kbs = p.kb;
    v16 = opaque(16 * lane);
    v4 = opaque(4 * lane);
    v_d = opaque(4 * (lane & 7));
  }
  // unit (row group rg, K block kb): one contiguous 3360-byte block copied as
  // it lies (the FP16 scales repeat eight times over the stage's last 256 B)
  __device__ __forceinline__ void issue(int rg, int kb, uint8_t* st) const {
    const uint8_t* u = data + ((int64_t)rg * kbs + kb) * kQ6Unit;
    dma16(u, v16, st);
    dma16(u + 1024, v16, st + 1024);
    dma16(u + 2048, v16, st + 2048);
    dma4(u + 3072, v4, st + 3072);
    dma4(u + 3328, v_d, st + 3328);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const u32x4 c0 = *reinterpret_cast<const u32x4*>(st + 16 * lane);
    const u32x4 c1 = *reinterpret_cast<const u32x4*>(st + 1024 + 16 * lane);
    const u32x4 c2 = *reinterpret_cast<const u32x4*>(st + 2048 + 16 * lane);
    const uint32_t sc = *reinterpret_cast<const uint32_t*>(st + 3072 + 4 * lane);
    const uint32_t d = *reinterpret_cast<const uint16_t*>(st + 3328 + 2 * (lane & 15));
    q6p_decode(c0, c1, c2, sc, d, a);
  }
};

template <>
struct WStream<FMT_Q4K> {
  static constexpr int kDma = 3;
  const uint8_t* data;
  int kbs;
  uint32_t v16, v4;
  __device__ __forceinline__ WStream(const Proj& p, int64_t e, int lane) {
    data = p.data + e * p.dstride;
    kbs = p.kb;
    v16 = opaque(16 * lane);
    v4 = opaque(4 * lane);
  }
  // unit: chunks 0-7 (2 KB) and chunk 8 (256 B), copied as they lie
  __device__ __forceinline__ void issue(int rg, int kb, uint8_t* st) const {
    const uint8_t* u = data + ((int64_t)rg * kbs + kb) * kQ4Unit;
    dma16(u, v16, st);
    dma16(u + 1024, v16, st + 1024);
    dma4(u + 2048, v4, st + 2048);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const int jj = lane & 15, jA = lane >> 4;
    auto chunk = [&](int c) -> u32x4 { return *reinterpret_cast<const u32x4*>(st + 16 * (c * 16 + jj)); };
    Unit<FMT_Q4K> u;
    u.hdr = chunk(0);
    u.qa = chunk(1 + 2 * jA);
    u.qb = chunk(2 + 2 * jA);
    u.decode(a, lane);
  }
};

template <>
struct WStream<FMT_Q8> {
  static constexpr int kDma = 5;
  const uint8_t* data;
  int kbs, hk;
  uint32_t v16, v4;
  __device__ __forceinline__ WStream(const Proj& p, int64_t e, int lane) {
    data = p.data + e * p.dstride;
    kbs = p.kb;
    hk = half_block(p);
    v16 = opaque(16 * lane);
    v4 = opaque(4 * lane);
  }
  // unit: four 1 KB code chunks and the 256 B of scales, copied as they lie;
  // in a K block whose second half lies past the matrix (K block hk), code
  // chunks 2 and 3 hold only zero padding, so their DMA re-reads chunks 0 and
  // 1 (cache hits) instead: those positions meet zeroed token operands and
  // zero scales.
  __device__ __forceinline__ void issue(int rg, int kb, uint8_t* st) const {
    const uint8_t* u = data + ((int64_t)rg * kbs + kb) * kQ8Unit;
    const int o2 = kb == hk ? 0 : 2048;
    dma16(u, v16, st);
    dma16(u + 1024, v16, st + 1024);
    dma16(u + o2, v16, st + 2048);
    dma16(u + o2 + 1024, v16, st + 3072);
    dma4(u + 4096, v4, st + 4096);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    u32x4 c[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) c[g] = *reinterpret_cast<const u32x4*>(st + 1024 * g + 16 * lane);
    const u32x2 d = *reinterpret_cast<const u32x2*>(st + 4096 + 8 * (2 * (lane & 15) + (lane >> 5)));
    q8_decode(c, d, a);
  }
};

template <>
struct WStream<FMT_Q5K> {
  static constexpr int kDma = 5;
  const uint8_t* data;
  int kbs;
  uint32_t v16, v4;
  __device__ __forceinline__ WStream(const Proj& p, int64_t e, int lane) {
    data = p.data + e * p.dstride;
    kbs = p.kb;
    v16 = opaque(16 * lane);
    v4 = opaque(4 * lane);
  }
  // unit: chunks 0-7 (2 KB) and chunks 8-10 (768 B), copied as they lie
  __device__ __forceinline__ void issue(int rg, int kb, uint8_t* st) const {
    const uint8_t* u = data + ((int64_t)rg * kbs + kb) * kQ5KUnit;
    dma16(u, v16, st);
    dma16(u + 1024, v16, st + 1024);
    dma4(u + 2048, v4, st + 2048);
    dma4(u + 2304, v4, st + 2304);
    dma4(u + 2560, v4, st + 2560);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const int jj = lane & 15, jA = lane >> 4;
    auto chunk = [&](int c) -> u32x4 { return *reinterpret_cast<const u32x4*>(st + 16 * (c * 16 + jj)); };
    Unit<FMT_Q5K> u;
    u.hdr = chunk(0);
    u.qh0 = chunk(1);
    u.qh1 = chunk(2);
    u.qa = chunk(3 + 2 * jA);
    u.qb = chunk(4 + 2 * jA);
    u.decode(a, lane);
  }
};

template <>
struct WStream<FMT_Q51> {
  static constexpr int kDma = 3;
  const uint8_t* data;
  int kbs, hk;
  uint32_t v16;
  __device__ __forceinline__ WStream(const Proj& p, int64_t e, int lane) {
    data = p.data + e * p.dstride;
    kbs = p.kb;
    hk = half_block(p);
    v16 = opaque(16 * lane);
  }
  // unit: three 1 KB runs, copied as they lie; in K block hk (second half past
  // the matrix) the nibble run of blocks 4-7 holds only padding and re-reads
  // the first run instead (zero scales there)
  __device__ __forceinline__ void issue(int rg, int kb, uint8_t* st) const {
    const uint8_t* u = data + ((int64_t)rg * kbs + kb) * kQ51Unit;
    dma16(u, v16, st);
    dma16(u + (kb == hk ? 0 : 1024), v16, st + 1024);
    dma16(u + 2048, v16, st + 2048);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const int j = lane & 15, hb = lane >> 5;
    Unit<FMT_Q51> u;
#pragma unroll
    for (int g = 0; g < 4; ++g) u.q[g] = *reinterpret_cast<const u32x4*>(st + 512 * g + 256 * hb + 16 * j);
    u.aux0 = *reinterpret_cast<const u32x4*>(st + 2048 + 64 * j + 32 * hb);
    u.aux1 = *reinterpret_cast<const u32x4*>(st + 2048 + 64 * j + 32 * hb + 16);
    u.decode(a, lane);
  }
};

// Token operands: lane (token column j, K group jA) reads row ``row`` of the
// BF16 matrix [rows, k] at columns kb*256 + xoff(f, jA); xoff splits into a
// lane part xoff(0, jA) and a fragment part xoff(f, 0) in both formats.
// kCoh: the loads read from the device coherence point (sc1), for rows that
// another XCD wrote in the same kernel.
template <int FMT, bool kFullK, bool kCoh = false>
struct XStream {
  static constexpr int kAux = kCoh ? 16 : 0;  // cache policy: sc1
  rsrc_t r;
  int v_row, k, lane_col;
  __device__ __forceinline__ XStream(const uint16_t* x, int nrows, int k_, int row, int lane) {
    k = k_;
    r = make_rsrc(x, (uint32_t)nrows * (uint32_t)k * 2u);
    lane_col = Unit<FMT>::xoff(0, lane >> 4);
    v_row = (int)opaque(2 * (row * k + lane_col));
  }
  __device__ __forceinline__ void load(u32x4 (&xb)[8], int kb) const {
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int fo = Unit<FMT>::xoff(f, 0);
      if (kFullK) {
        xb[f] = __builtin_bit_cast(u32x4,
                                   __builtin_amdgcn_raw_buffer_load_b128(r, v_row, kb * 2 * kQK + 2 * fo, kAux));
      } else {
        int vo = v_row + 2 * fo;
        if (kb * kQK + lane_col + fo + 8 > k) vo = v_row - 2 * lane_col;  // in bounds; zeroed at use
        xb[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, kb * 2 * kQK, kAux));
      }
    }
  }
  __device__ __forceinline__ void mask(u32x4 (&xb)[8], int kb) const {
    if (!kFullK) {
#pragma unroll
      for (int f = 0; f < 8; ++f)
        if (kb * kQK + lane_col + Unit<FMT>::xoff(f, 0) + 8 > k) xb[f] = u32x4{0u, 0u, 0u, 0u};
    }
  }
};

// Streams P units per K block over the kbs K blocks kb0.. through the wave's
// ring: unit (kb, p) is DMA'd by issue_w(p, kb, stage) and multiplied into acc[p].
// The token operands of K block kb are loaded with unit (kb, 0), one K block
// ahead of their use, into the register set of kb's parity. The steady-state
// loop issues unconditionally so that the compiler's own wait counts for the
// token operands stay exact across the back edge.
template <int FMT, bool kFullK, int P, bool kCoh, typename IssueW>
__device__ __forceinline__ void stream_units(uint8_t* ring, int kb0, int kbs, const XStream<FMT, kFullK, kCoh>& xs,
                                             IssueW&& issue_w, f32x4 (&acc)[P]) {
  static_assert(kStages == 3 && P >= kStages - 1, "one K block of token operands in flight");
  const int lane = threadIdx.x & 63;
  u32x4 xA[8], xB[8];
  auto stage = [&](int u) { return ring + (u % kStages) * stage_bytes<FMT>(); };
  auto compute = [&](auto pc, int u, u32x4(&xc)[8]) {
    constexpr int p = decltype(pc)::value;
    if constexpr (p == 0) xs.mask(xc, kb0 + u / P);
    u32x4 a[8];
    WStream<FMT>::decode(stage(u), lane, a);
#pragma unroll
    for (int f = 0; f < 8; ++f) acc[p] = mfma16(a[f], xc[f], acc[p]);
  };
  // K block kb when K block kb+1 exists: every unit issues the one 2 ahead.
  auto steady = [&](int kb, u32x4(&xc)[8], u32x4(&xo)[8]) {
    static_for<0, P>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr int pv = (p + 2) % P, dkb = (p + 2) / P;
      const int u = kb * P + p;
      issue_w(pv, kb0 + kb + dkb, stage(u + 2));
      if constexpr (pv == 0) xs.load(xo, kb0 + kb + 1);
      wait_vm<younger_ops<P, WStream<FMT>::kDma>(p, 2)>();
      compute(pc, u, xc);
    });
  };
  // The last K block: only units inside it remain to be issued.
  auto last = [&](int kb, u32x4(&xc)[8]) {
    static_for<0, P>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr int ahead = P - 1 - p < 2 ? P - 1 - p : 2;
      const int u = kb * P + p;
      if constexpr (p + 2 < P) issue_w(p + 2, kb0 + kb, stage(u + 2));
      wait_vm<younger_ops<P, WStream<FMT>::kDma>(p, ahead)>();
      compute(pc, u, xc);
    });
  };
  issue_w(0, kb0, stage(0));
  xs.load(xA, kb0);
  issue_w(1, kb0, stage(1));  // P >= 2: unit (0, 1)
  int kb = 0;
  for (; kb + 2 < kbs; kb += 2) {
    steady(kb, xA, xB);
    steady(kb + 1, xB, xA);
  }
  if (kb + 1 < kbs) {
    steady(kb, xA, xB);
    last(kb + 1, xB);
  } else {
    last(kb, xA);
  }
}

// Wave-level routing. Fills ``tok`` with the slot's tokens (ascending) and
// returns the slot's expert, first route position and route count; returns
// false for an inactive slot. ``publish`` also writes the slot's route tables,
// and slot 0 the per-slot and per-token tables.
struct SlotRoute {
  int expert, t0, cnt;
};

// Routing for at most 64 entries (tokens * top_k <= 64), one entry per lane,
// with cross-lane reads instead of LDS loops: only the expert bit mask (LDS
// atomics) and the token list touch LDS, and no workgroup barrier is needed,
// since every wave works in its own scratch.
__device__ __forceinline__ uint64_t token_lanes(int b, int K) {
  const uint64_t m = K >= 64 ? ~0ull : (1ull << K) - 1ull;
  return m << (b * K);
}

__device__ bool dec_route_small(const DecRoute& R, int slot, bool publish, const DecTables& T, uint8_t* scratch,
                                int* tok, SlotRoute& out) {
  const int lane = threadIdx.x & 63;
  const int n = R.B * R.K;
  uint32_t* s_mask = reinterpret_cast<uint32_t*>(scratch);  // one bit per expert
  // Up to 256 experts the mask is 8 words, read as two 16-byte words; a wider
  // layer's further words are read in one more batch.
  const bool wide = R.E > 256;
  if (lane < (wide ? kMaskWords : 8)) s_mask[lane] = 0u;
  int id = -1;
  float rw = 0.f;
  if (lane < n) {
    id = R.ids[lane];
    rw = bf16_to_float(R.wts[lane]);
  }
  const int b = lane / R.K, kk = lane - b * R.K;
  // Merged weight (experts.py:66-73): the first occurrence of an id in its
  // token carries the sum, in position order, of the token's weights for it.
  bool first = lane < n && id >= 0 && id < R.E;
  float s = 0.f;
  for (int k0 = 0; k0 < R.K; k0 += 8) {
    int id2[8];
    float r2[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int src = b * R.K + (k0 + q < R.K ? k0 + q : 0);
      id2[q] = __shfl(id, src);
      r2[q] = __shfl(rw, src);
    }
    // branch-free: terms that do not match add +0, which leaves the sum as is
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int k2 = k0 + q;
      const bool same = id2[q] == id;
      first = first && !(k2 < kk && same);
      s += (k2 >= kk && k2 < R.K && same) ? r2[q] : 0.f;
    }
  }
  float r = first ? bf16_round(s) : 0.f;
  r = r != 0.f ? r : 0.f;
  const bool live = r != 0.f;
  if (live) atomicOr(&s_mask[id >> 5], 1u << (id & 31));
  const u32x4 mA = *reinterpret_cast<const u32x4*>(s_mask), mB = *reinterpret_cast<const u32x4*>(s_mask + 4);
  uint32_t m[kMaskWords];
  int total = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    m[q] = __builtin_amdgcn_readfirstlane(mA[q]);
    m[q + 4] = __builtin_amdgcn_readfirstlane(mB[q]);
  }
#pragma unroll
  for (int q = 8; q < kMaskWords; ++q) m[q] = 0u;
  if (wide) {
    u32x4 mw[kMaskWords / 4 - 2];
#pragma unroll
    for (int c = 0; c < kMaskWords / 4 - 2; ++c) mw[c] = *reinterpret_cast<const u32x4*>(s_mask + 8 + 4 * c);
#pragma unroll
    for (int c = 0; c < kMaskWords / 4 - 2; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) m[8 + 4 * c + q] = __builtin_amdgcn_readfirstlane(mw[c][q]);
#pragma unroll
    for (int q = 8; q < kMaskWords; ++q) total += __builtin_popcount(m[q]);
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) total += __builtin_popcount(m[q]);
  const uint64_t lm = __ballot(live);
  if (publish && slot == 0) {
    if (lane == 0) {
      st_agent(&T.hdr[0], total);
      st_agent(&T.hdr[1], (int)__popcll(lm));
    }
    if (lane < R.B) st_agent(&T.tok_n[lane], (int)__popcll(lm & token_lanes(lane, R.K)));
  }
  const bool alive = slot < total;
  if (alive) {
    // the slot's expert: the slot-th set bit of the mask (ascending id)
    int e = 0, rem = slot;
    const auto find = [&](auto q) {
      const int c = __builtin_popcount(m[q]);
      if (rem >= 0 && rem < c) {
        uint32_t w = m[q];
        for (int i = 0; i < rem; ++i) w &= w - 1u;
        e = 32 * q + __builtin_ctz(w);
      }
      rem -= c;
    };
    static_for<0, 8>(find);
    if (wide && rem >= 0) static_for<8, kMaskWords>(find);
    const uint64_t below = __ballot(live && id < e);
    const uint64_t mine = __ballot(live && id == e);
    const int t0 = __popcll(below), cnt = __popcll(mine);
    if (live && id == e) {
      const int rank = __popcll(mine & ((1ull << lane) - 1ull));
      tok[rank] = b;
      if (publish) {
        st_agent(&T.route_w[t0 + rank], r);
        st_agent(&T.route_dst[t0 + rank], b * R.K + (int)__popcll(below & token_lanes(b, R.K)));
      }
    }
    if (publish && lane == 0) {
      st_agent(&T.slot_e[slot], e);
      st_agent(&T.slot_t0[slot], t0);
      st_agent(&T.slot_cnt[slot], cnt);
    }
    out = SlotRoute{e, t0, cnt};
  }
  // Stores must not count against the ring's wait counts, and the mask (in the
  // ring's first stage) and token list must be read and written before the ring fills.
  wait_vm<0>();
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  return alive;
}

__device__ bool dec_route(const DecRoute& R, int slot, bool publish, const DecTables& T, uint8_t* scratch,
                          int* tok, SlotRoute& out) {
  const int lane = threadIdx.x & 63;
  const int n = R.B * R.K;
  if (n <= 64) return dec_route_small(R, slot, publish, T, scratch, tok, out);
  int* s_ids = reinterpret_cast<int*>(scratch);
  const int n4 = (n + 3) & ~3;  // route_scratch_bytes(n) bytes: ids, weights, counts
  float* s_r = reinterpret_cast<float*>(scratch + 4 * n4);
  int* s_cnt = reinterpret_cast<int*>(scratch + 8 * n4);
  const int e256 = (R.E + 255) & ~255;  // counts zeroed in whole chunks of 256 experts
  for (int i = lane; i < e256; i += 64) s_cnt[i] = 0;
  for (int i = lane; i < n; i += 64) {
    s_ids[i] = R.ids[i];
    s_r[i] = bf16_to_float(R.wts[i]);
  }
  __syncthreads();
  // merged weight at the first occurrence of each id in a token; 0 elsewhere.
  // A chunk's sums read entries at or after their own position only, which
  // still hold raw weights when the chunk's results are written.
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    float r = 0.f;
    int id = -1;
    if (i < n && R.K <= 16) {
      // top_k <= 16: the token's entries read in one batch (clamped to entry
      // 0 past top_k, and masked below), then the same comparisons and
      // summation order as the loops of the general case
      const int b = i / R.K, kk = i - b * R.K;
      int id2[16];
      float r2[16];
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        const int o = b * R.K + (k2 < R.K ? k2 : 0);
        id2[k2] = s_ids[o];
        r2[k2] = s_r[o];
      }
      id = s_ids[i];
      bool first = id >= 0 && id < R.E;
      float s = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        const bool same = k2 < R.K && id2[k2] == id;
        first = first && !(same && k2 < kk);
        s += (same && k2 >= kk) ? r2[k2] : 0.f;
      }
      if (first) {
        r = bf16_round(s);
        r = r != 0.f ? r : 0.f;
      }
    } else if (i < n) {
      const int b = i / R.K, kk = i - b * R.K;
      id = s_ids[i];
      bool first = id >= 0 && id < R.E;
      for (int k2 = 0; k2 < kk && first; ++k2) first = s_ids[b * R.K + k2] != id;
      if (first) {
        float s = 0.f;
        for (int k2 = kk; k2 < R.K; ++k2)
          if (s_ids[b * R.K + k2] == id) s += s_r[b * R.K + k2];
        r = bf16_round(s);
        r = r != 0.f ? r : 0.f;
      }
    }
    __syncthreads();
    if (i < n) {
      s_r[i] = r;
      if (r != 0.f) atomicAdd(&s_cnt[id], 1);
    }
    __syncthreads();
  }
  // exclusive scans over experts of active flags and counts, in chunks of
  // 256 experts (4 per lane), each chunk starting from the earlier chunks' totals
  const bool tables = publish && slot == 0;
  int total = 0, routes = 0;
  int my_e = -1, my_t0 = 0, my_c = 0;
  for (int c0 = 0; c0 < R.E; c0 += 256) {
    int act[4], cnt[4], la = 0, lc = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      cnt[q] = s_cnt[c0 + lane * 4 + q];
      act[q] = cnt[q] > 0;
      la += act[q];
      lc += cnt[q];
    }
    int ia = la, ic = lc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int ta = __shfl_up(ia, off), tc = __shfl_up(ic, off);
      if (lane >= off) {
        ia += ta;
        ic += tc;
      }
    }
    int ea = total + ia - la, ec = routes + ic - lc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (act[q]) {
        const int e = c0 + lane * 4 + q;
        if (ea == slot) {
          my_e = e;
          my_t0 = ec;
          my_c = cnt[q];
        }
        if (tables) {
          st_agent(&T.slot_e[ea], e);
          st_agent(&T.slot_t0[ea], ec);
          st_agent(&T.slot_cnt[ea], cnt[q]);
        }
      }
      ea += act[q];
      ec += cnt[q];
    }
    total += __builtin_amdgcn_readfirstlane(__shfl(ia, 63));
    routes += __builtin_amdgcn_readfirstlane(__shfl(ic, 63));
  }
  if (tables) {
    if (lane == 0) {
      st_agent(&T.hdr[0], total);
      st_agent(&T.hdr[1], routes);
    }
    for (int b = lane; b < R.B; b += 64) {
      int m = 0;
      for (int kk = 0; kk < R.K; ++kk) m += s_r[b * R.K + kk] != 0.f;
      st_agent(&T.tok_n[b], m);
    }
  }
  bool live = slot < total;
  if (live) {
    const unsigned long long own = __ballot(my_e >= 0);
    const int src = __ffsll((long long)own) - 1;
    const int e = __shfl(my_e, src), t0 = __shfl(my_t0, src), c = __shfl(my_c, src);
    int run = 0;
    for (int c0 = 0; c0 < n; c0 += 64) {
      const int i = c0 + lane;
      const bool hit = i < n && s_ids[i] == e && s_r[i] != 0.f;
      const unsigned long long m = __ballot(hit);
      if (hit) {
        const int rank = run + __popcll(m & ((1ull << lane) - 1ull));
        const int b = i / R.K;
        tok[rank] = b;
        if (publish) {
          int er = 0;  // routed experts of this token with a smaller id
          if (R.K <= 16) {
            int id2[16];
            float r2[16];
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
              const int o = b * R.K + (kk < R.K ? kk : 0);
              id2[kk] = s_ids[o];
              r2[kk] = s_r[o];
            }
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) er += kk < R.K && r2[kk] != 0.f && id2[kk] < e;
          } else {
            for (int kk = 0; kk < R.K; ++kk) {
              const int o = b * R.K + kk;
              er += (s_r[o] != 0.f) && s_ids[o] < e;
            }
          }
          st_agent(&T.route_w[t0 + rank], s_r[i]);
          st_agent(&T.route_dst[t0 + rank], b * R.K + er);
        }
      }
      run += __popcll(m);
    }
    out = SlotRoute{__builtin_amdgcn_readfirstlane(e), __builtin_amdgcn_readfirstlane(t0),
                    __builtin_amdgcn_readfirstlane(c)};
  }
  // Stores must not count against the ring's wait counts; the ring overlays
  // this scratch, so its reads finish first as well.
  wait_vm<0>();
  __syncthreads();
  return live;
}

// K split: a workgroup of NS waves (blockDim.x / 64) computes one item; wave
// w streams K blocks [w*kbs/NS, (w+1)*kbs/NS) through its own ring and the
// partial sums meet in LDS, added in wave order by wave 0. NS > 1 when the
// items alone would leave SIMDs idle (few tokens or experts).

__device__ __forceinline__ int split_waves() { return __builtin_amdgcn_readfirstlane(blockDim.x >> 6); }
__device__ __forceinline__ int split_wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Sums the P accumulators of all waves into wave 0's (wave order); every wave
// passes its barriers. The other waves' rings (``wave_lds`` bytes apart) are
// free when this is called.
template <int P>
__device__ __forceinline__ void split_reduce(uint8_t* smem, int ns, int wave, f32x4 (&acc)[P], int wave_lds) {
  if (ns == 1) return;
  const int lane = threadIdx.x & 63;
  __syncthreads();
  if (wave > 0) {
    float* red = reinterpret_cast<float*>(smem + wave * wave_lds);
#pragma unroll
    for (int p = 0; p < P; ++p) *reinterpret_cast<f32x4*>(red + (p * 64 + lane) * 4) = acc[p];
  }
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < ns; ++w) {
      const float* red = reinterpret_cast<const float*>(smem + w * wave_lds);
#pragma unroll
      for (int p = 0; p < P; ++p) acc[p] += *reinterpret_cast<const f32x4*>(red + (p * 64 + lane) * 4);
    }
  }
  __syncthreads();
}

// One gate/up item: row group rg of an expert's gate and up, over its tokens
// tok[0..cnt) in passes of 16; a = RNE(RNE(g*sig(g)) * u) into act rows
// t0 + q (row stride ``inter``). kCoh: each lane's four rows are one
// device-scope 8-byte store (inter a multiple of 16).
template <int FMT, bool kFullK, bool kCoh = false>
__device__ __forceinline__ void dec_gate_up_item(uint8_t* smem, uint8_t* ring, int wave_lds, const Proj& gate,
                                                 const Proj& up, int64_t expert, int rg, int t0, int cnt,
                                                 const int* tok, const uint16_t* __restrict__ x, int nx, int hidden,
                                                 uint16_t* __restrict__ act, int inter) {
  const int ns = split_waves(), wave = split_wave();
  const int lane = threadIdx.x & 63, jA = lane >> 4, j = lane & 15;
  const WStream<FMT> wg(gate, expert, lane), wu(up, expert, lane);
  const int kb0 = wave * gate.kb / ns, kb1 = (wave + 1) * gate.kb / ns;
  for (int tc = 0; tc < cnt; tc += kPassTokens) {
    const int nt = cnt - tc < kPassTokens ? cnt - tc : kPassTokens;
    if (tc) wait_vm<0>();  // the previous pass's stores
    const XStream<FMT, kFullK> xs(x, nx, hidden, tok[tc + (j < nt ? j : nt - 1)], lane);
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    if (kb1 > kb0)
      stream_units<FMT, kFullK, 2>(
          ring, kb0, kb1 - kb0, xs, [&](int p, int kb, uint8_t* st) { (p ? wu : wg).issue(rg, kb, st); }, acc);
    split_reduce<2>(smem, ns, wave, acc, wave_lds);
    // lane holds rows 4*(lane/16)+q, token column lane%16 of both accumulators
    if (wave == 0 && j < nt) {
      if constexpr (kCoh) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g = bf16_round(acc[0][q]);
          const float uu = bf16_round(acc[1][q]);
          v[q] = bf16_round(g * sigmoid_acc(g)) * uu;
        }
        const uint64_t w = (uint64_t)pack_bf16x2(v[0], v[1]) | ((uint64_t)pack_bf16x2(v[2], v[3]) << 32);
        st_agent(reinterpret_cast<uint64_t*>(act + (int64_t)(t0 + tc + j) * inter + rg * 16 + 4 * jA), w);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = rg * 16 + 4 * jA + q;
          if (row < inter) {
            const float g = bf16_round(acc[0][q]);
            const float uu = bf16_round(acc[1][q]);
            const float sg = bf16_round(g * sigmoid_acc(g));
            act[(int64_t)(t0 + tc + j) * inter + row] = bf16_bits(sg * uu);
          }
        }
      }
    }
  }
}

// Items: the shared expert's (row group, pass of 16 tokens) first (sh.is > 0),
// then (row group, expert slot) with the row group fastest.
template <int FMT, bool kFullK>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
    moe_dec_gate_up_kernel(Proj gate, Proj up, DecRoute R, DecTables T, const uint16_t* __restrict__ x,
                           int hidden, uint16_t* __restrict__ act, int inter, DecShared sh) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int wave = split_wave();
  const int wl = gu_wave_lds<FMT>(R.B * R.K, R.E);
  uint8_t* ring = smem + wave * wl;
  int* tok = reinterpret_cast<int*>(ring + wl - 4 * kDecMaxTokens);
  const int sh_groups = (sh.is + 15) / 16, passes = (R.B + kPassTokens - 1) / kPassTokens;
  const int sh_items = sh.is ? sh_groups * passes : 0;
  const int item = blockIdx.x;
  if (item < sh_items) {
    // every token, weight 1; item (row group, pass of 16 tokens)
    const int lane = threadIdx.x & 63;
    const int rg = item % sh_groups, t0 = (item / sh_groups) * kPassTokens;
    const int cnt = R.B - t0 < kPassTokens ? R.B - t0 : kPassTokens;
    if (lane < cnt) tok[lane] = t0 + lane;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the list is in LDS before the ring fills
    dec_gate_up_item<FMT, kFullK>(smem, ring, wl, sh.gate, sh.up, 0, rg, t0, cnt, tok, x, R.B, hidden, sh.act,
                                  sh.is);
    return;
  }
  const int groups_i = (inter + 15) / 16;
  const int rg = (item - sh_items) % groups_i, slot = (item - sh_items) / groups_i;
  SlotRoute sr;
  if (!dec_route(R, slot, rg == 0 && wave == 0, T, ring, tok, sr)) return;
  dec_gate_up_item<FMT, kFullK>(smem, ring, wl, gate, up, sr.expert, rg, sr.t0, sr.cnt, tok, x, R.B, hidden, act,
                                inter);
}

// One routed down item: row groups kDownRows*blk.. of slot ``slot``'s expert,
// over the slot's routes in passes of 16; stores the exact FP32 product
// f32(RNE(y)) * f32(r) token-major at the route's rank among its token's
// experts. The slot tables and header come from ``t0s``/``cnts``/``exps``/
// ``hdr`` (kCoh: read at the device coherence point, with the activations).
template <int FMT, bool kFullK, bool kCoh>
__device__ __forceinline__ void dec_down_item(uint8_t* smem, uint8_t* ring, const Proj& down, const DecTables& T,
                                              const uint16_t* __restrict__ act, int inter,
                                              float* __restrict__ contrib, int hidden, int blk, int slot,
                                              const int* t0s, const int* cnts, const int* exps, const int* hdr) {
  const int ns = split_waves(), wave = split_wave();
  const int lane = threadIdx.x & 63, jA = lane >> 4, j = lane & 15;
  const int groups = (hidden + 15) / 16;
  auto ld = [](const auto* p) { return kCoh ? ld_agent(p) : *p; };
  // The slot's tables are read together with the active-slot count (every
  // slot below max_slots <= E is in bounds; an inactive one's values are
  // never used), so the weight stream's expert is known one load latency
  // after the start rather than two.
  const int t0 = ld(t0s + slot), cnt = ld(cnts + slot), expert = ld(exps + slot);
  const int nact = ld(hdr), routes = ld(hdr + 1);
  asm volatile("" ::: "memory");  // keeps the loads above issued here, not sunk below the branches
  if (slot >= nact) return;
  const WStream<FMT> wd(down, expert, lane);
  const int rg0 = blk * kDownRows;
  const int kb0 = wave * down.kb / ns, kb1 = (wave + 1) * down.kb / ns;
  for (int tc = 0; tc < cnt; tc += kPassTokens) {
    const int nt = cnt - tc < kPassTokens ? cnt - tc : kPassTokens;
    if (tc) wait_vm<0>();
    const int pos = t0 + tc + (j < nt ? j : nt - 1);
    const int dst = ld(T.route_dst + pos);
    const float w = ld(T.route_w + pos);
    f32x4 acc[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    const XStream<FMT, kFullK, kCoh> xs(act, routes, inter, pos, lane);
    if (kb1 > kb0)
      stream_units<FMT, kFullK, kDownRows>(
          ring, kb0, kb1 - kb0, xs,
          [&](int p, int kb, uint8_t* st) {
            const int rg = rg0 + p < groups ? rg0 + p : groups - 1;  // clamped rows are discarded
            wd.issue(rg, kb, st);
          },
          acc);
    split_reduce<kDownRows>(smem, ns, wave, acc, ring_bytes<FMT>());
    if (wave == 0 && j < nt) {
#pragma unroll
      for (int r = 0; r < kDownRows; ++r) {
        const int row = (rg0 + r) * 16 + 4 * jA;
        f32x4 c;
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = bf16_round(acc[r][q]) * w;  // exact product
        if (row + 4 <= hidden) {
          *reinterpret_cast<f32x4*>(contrib + (int64_t)dst * hidden + row) = c;
        } else {
          for (int q = 0; q < 4; ++q)
            if (row + q < hidden) contrib[(int64_t)dst * hidden + row + q] = c[q];
        }
      }
    }
  }
}

// Items: the shared expert's down (kShRows row groups and 16 tokens each,
// output BF16 y = RNE(acc) into sh.y [B, H]) first, then (block of kDownRows row groups,
// expert slot), which store the exact FP32 product f32(RNE(y)) * f32(r)
// token-major at the route's rank among its token's experts.
constexpr int kShRows = 2;

template <int FMT, bool kFullK>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
    moe_dec_down_kernel(Proj down, DecTables T, const uint16_t* __restrict__ act, int inter,
                        float* __restrict__ contrib, int hidden, DecShared sh, int tokens) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int ns = split_waves(), wave = split_wave();
  uint8_t* ring = smem + wave * ring_bytes<FMT>();
  const int lane = threadIdx.x & 63, jA = lane >> 4, j = lane & 15;
  const int groups = (hidden + 15) / 16;
  const int sh_blocks = (groups + kShRows - 1) / kShRows, passes = (tokens + kPassTokens - 1) / kPassTokens;
  const int sh_items = sh.is ? sh_blocks * passes : 0;
  const int item = blockIdx.x;
  if (item < sh_items) {
    // item (block of kShRows row groups, pass of 16 tokens)
    const int rg0 = (item % sh_blocks) * kShRows, t0 = (item / sh_blocks) * kPassTokens;
    const int kb0 = wave * sh.down.kb / ns, kb1 = (wave + 1) * sh.down.kb / ns;
    const WStream<FMT> wd(sh.down, 0, lane);
    const int nt = tokens - t0 < kPassTokens ? tokens - t0 : kPassTokens;
    const XStream<FMT, kFullK> xs(sh.act, tokens, sh.is, t0 + (j < nt ? j : nt - 1), lane);
    f32x4 acc[kShRows];
#pragma unroll
    for (int r = 0; r < kShRows; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (kb1 > kb0)
      stream_units<FMT, kFullK, kShRows>(
          ring, kb0, kb1 - kb0, xs,
          [&](int p, int kb, uint8_t* st) { wd.issue(rg0 + p < groups ? rg0 + p : groups - 1, kb, st); }, acc);
    split_reduce<kShRows>(smem, ns, wave, acc, ring_bytes<FMT>());
    if (wave == 0 && j < nt) {
#pragma unroll
      for (int r = 0; r < kShRows; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = (rg0 + r) * 16 + 4 * jA + q;
          if (row < hidden) sh.y[(int64_t)(t0 + j) * hidden + row] = bf16_bits(acc[r][q]);
        }
    }
    return;
  }
  const int dn_x = (groups + kDownRows - 1) / kDownRows;
  dec_down_item<FMT, kFullK, false>(smem, ring, down, T, act, inter, contrib, hidden, (item - sh_items) % dn_x,
                                    (item - sh_items) / dn_x, T.slot_t0, T.slot_cnt, T.slot_e, T.hdr);
}

// The decode step's gate/up and down in one launch (one wave per item, no
// shared expert): items 0 .. groups_i*max_slots-1 are the gate/up items (row
// group fastest, then slot), the rest the down items (block of kDownRows row
// groups fastest, then slot). A gate/up item stores its activations and, for
// row group 0, its slot's tables with device-scope stores, waits for them to
// complete and then writes the call's tag into its (slot, row group) flag; a
// down item waits until every row group of its slot and row group 0 of slot 0
// (which wrote the header) carry the tag, then streams its rows of down.
// Workgroups of a launch start in index order, so every gate/up item has
// started before any down item waits, and the waits end; a wait that exceeds
// kSpinLimit polls gives up and marks the call (the combine then writes NaN).
// The tag is a function of the workspace's call counter (hdr[kHdrEpoch]),
// which the combine kernel advances, so flags of an earlier call never match.
//
// The kernel holds both item bodies; at three waves per SIMD, the register
// budget of the separate kernels, it spills (about 30 VGPRs), so it runs at
// two.
template <int FG, int FD, bool kFullK>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
    moe_dec_fused_kernel(Proj gate, Proj up, Proj down, DecRoute R, DecTables T, const uint16_t* __restrict__ x,
                         int hidden, uint16_t* __restrict__ act, int inter, float* __restrict__ contrib,
                         uint64_t* __restrict__ flags, int max_slots) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int groups_i = (inter + 15) / 16, groups_h = (hidden + 15) / 16;
  const int dn_x = (groups_h + kDownRows - 1) / kDownRows;
  const int items_gu = groups_i * max_slots;
  const int item = blockIdx.x;
  if (item < items_gu) {
    const int rg = item % groups_i, slot = item / groups_i;
    const int wl = gu_wave_lds<FG>(R.B * R.K, R.E);
    int* tok = reinterpret_cast<int*>(smem + wl - 4 * kDecMaxTokens);
    if (item == 0 && lane == 0) st_agent(&T.hdr[kHdrStall], 0);
    SlotRoute sr;
    if (dec_route(R, slot, rg == 0, T, smem, tok, sr))
      dec_gate_up_item<FG, kFullK, true>(smem, smem, wl, gate, up, sr.expert, rg, sr.t0, sr.cnt, tok, x, R.B,
                                         hidden, act, inter);
    const uint64_t tag = sync_tag((uint32_t)T.hdr[kHdrEpoch]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every store of this item is at the coherence point
    if (lane == 0) st_agent(flags + (int64_t)slot * groups_i + rg, tag);
    return;
  }
  const int d = item - items_gu;
  const int blk = d % dn_x, slot = d / dn_x;
  const uint64_t* fs = flags + (int64_t)slot * groups_i;
  const uint64_t tag = sync_tag((uint32_t)T.hdr[kHdrEpoch]);
  for (int it = 0;; ++it) {
    const uint64_t f = lane < groups_i ? ld_agent(fs + lane) : tag;
    const uint64_t f0 = ld_agent(flags);
    if (__ballot(f != tag || f0 != tag) == 0) break;
    if (it == kSpinLimit) {
      if (lane == 0) st_agent(&T.hdr[kHdrStall], 1);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");  // the down item's loads stay behind the flags
  dec_down_item<FD, kFullK, true>(smem, smem, down, T, act, inter, contrib, hidden, blk, slot, T.slot_t0, T.slot_cnt,
                                  T.slot_e, T.hdr);
}

// out[b, h] = RNE(sum_r contrib[b, r, h]) over the token's routes in rank
// (= ascending expert id) order; with a shared expert RNE(f32(routed) + shared).
// One lane per 4 hidden columns; the rank rows are loaded 8 at a time before
// they are summed in order.
__global__ void __launch_bounds__(64)
    moe_dec_combine_kernel(DecTables T, const float* __restrict__ contrib, int hidden, int K,
                           const uint16_t* __restrict__ sh_y, const uint16_t* __restrict__ sh_scale,
                           uint16_t* __restrict__ out, int fused) {
  const int b = blockIdx.x;
  const int h = (blockIdx.y * 64 + threadIdx.x) * 4;
  // after the fused kernel: advance the workspace's call counter (no other
  // workgroup reads it) and note whether a down item gave up waiting
  const bool stalled = fused && T.hdr[kHdrStall] != 0;
  if (fused && b == 0 && blockIdx.y == 0 && threadIdx.x == 0) T.hdr[kHdrEpoch] = T.hdr[kHdrEpoch] + 1;
  if (h >= hidden) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const float* base = contrib + (int64_t)b * K * hidden + h;
  // The first 8 rank rows are loaded together with the token's route count,
  // without waiting for it (rows past K repeat row K-1, so every load is in
  // bounds), then only its m routes are summed; later rows, for top-k above
  // 8, after it.
  f32x4 v0[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    v0[i] = *reinterpret_cast<const f32x4*>(base + (int64_t)(i < K ? i : K - 1) * hidden);
  asm volatile("" ::: "memory");  // keeps the loads above issued here, not sunk into the sum's branches
  const int m = T.tok_n[b];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < m) acc += v0[i];
  for (int r0 = 8; r0 < m; r0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (r0 + i < m) v[i] = *reinterpret_cast<const f32x4*>(base + (int64_t)(r0 + i) * hidden);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (r0 + i < m) acc += v[i];
  }
  u32x2 o;
  if (sh_y) {
    const u32x2 sv = *reinterpret_cast<const u32x2*>(sh_y + (int64_t)b * hidden + h);
    const float gs = sh_scale ? bf16_to_float(sh_scale[b]) : 1.f;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float sy = bf16_to_float((uint16_t)(sv[c >> 1] >> (16 * (c & 1))));
      if (sh_scale) sy = bf16_round(sy * gs);
      v[c] = bf16_round(acc[c]) + sy;
    }
    o[0] = pack_bf16x2(v[0], v[1]);
    o[1] = pack_bf16x2(v[2], v[3]);
  } else {
    o[0] = pack_bf16x2(acc[0], acc[1]);
    o[1] = pack_bf16x2(acc[2], acc[3]);
  }
  if (stalled) o = u32x2{0x7fc07fc0u, 0x7fc07fc0u};  // BF16 NaN: the call's result is not valid
  *reinterpret_cast<u32x2*>(out + (int64_t)b * hidden + h) = o;
}

// Waves per workgroup (K split) for a launch of ``items`` workgroups at most.
// A launch with few items gets up to 4 waves per item, until it has about 2.5
// waves per SIMD (streams of a few units per wave then keep enough bytes in
// flight). ``split_long`` asks for 2 waves per item when the launch is not
// short of items but each item is long: the down items' K blocks (kDownRows
// units each) split evenly in two. Measured on the decode steps of the
// 128-expert Q6_K layer (1 wave best for both kernels) and the 64-expert Q4_K
// layer (1 token: 4 and 4; 8 tokens: down 2; 16 tokens and more: 1).
static int split_for(int64_t items, bool split_long) {
  // SIMDs of the current device (4 per CU), looked up once per device id
  static std::atomic<int> simds_of[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::atomic<int>& slot = simds_of[dev & 63];
  int simds = slot.load(std::memory_order_relaxed);
  if (!simds) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    simds = 4 * cus;
    slot.store(simds, std::memory_order_relaxed);
  }
  int ns = 1;
  while (ns < 4 && items * ns * 2 * 4 <= 10 * (int64_t)simds) ns *= 2;
  if (ns == 1 && split_long) ns = 2;
  return ns;
}

// FG: gate/up table format, FD: down table format.
template <int FG, int FD, bool kFullK>
static int launch(const DecArgs& A, hipStream_t s) {
  const int groups_i = (int)cdiv(A.I, 16), groups_h = (int)cdiv(A.H, 16);
  // per-wave LDS: the gate/up ring sized for this launch's routing entries
  const int lds_gu = gu_wave_lds<FG>((int)(A.R.B * A.R.K), A.R.E);
  constexpr int lds_dn = ring_bytes<FD>();
  static std::atomic<uint64_t> attr_done{0};
  once_per_device(attr_done, [] {  // the most any launch asks for
    (void)hipFuncSetAttribute((const void*)moe_dec_gate_up_kernel<FG, kFullK>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              4 * gu_wave_lds<FG>(kDecMaxEntries, kMaxExperts));
    (void)hipFuncSetAttribute((const void*)moe_dec_down_kernel<FD, kFullK>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 4 * ring_bytes<FD>());
  });
  const int dn_x = (int)cdiv(groups_h, kDownRows);
  const int passes = (int)cdiv(A.R.B, kPassTokens);
  const int sh_gu = A.S.is ? (int)cdiv(A.S.is, 16) * passes : 0;
  const int sh_dn = A.S.is ? (int)cdiv(groups_h, kShRows) * passes : 0;
  const int64_t items_gu = (int64_t)groups_i * A.max_slots + sh_gu, items_dn = (int64_t)dn_x * A.max_slots + sh_dn;
  // long down items: an even number of K blocks, at least 4 (so 2 waves each
  // stream 2 or more K blocks of kDownRows units), and the routing of at most
  // 64 entries that every wave repeats cheaply
  const int kb_i = (int)cdiv(A.I, kQK);
  const bool long_dn = kb_i % 2 == 0 && kb_i >= 4 && A.R.B * A.R.K <= 64;
  const int ns_gu = split_for(items_gu, false), ns_dn = split_for(items_dn, long_dn);
  // One launch for gate/up and down where the routes are spread thin (fewer
  // than 0.4 routes per expert on average: most active experts see one route,
  // each item is short, and the separate launches' ramps and tails dominate);
  // it needs one wave per item, no shared expert, and whole 16-row groups of at
  // most 64 per slot (one flag per lane). Measured against the separate
  // launches: the 512-expert top-10 layer at 8 and 16 tokens 11 % and 8 %
  // faster, at 32 and 64 tokens 3 % and 9 % slower; the 128-expert top-8
  // layer at 8 tokens (0.5 routes per expert) 3 % slower.
  const bool thin = 5 * A.R.B * A.R.K < 2 * A.R.E;
  const bool fused = thin && A.flags && ns_gu == 1 && ns_dn == 1 && !A.S.is && A.I % 16 == 0 && groups_i <= 64;
  if (fused) {
    const int lds = lds_gu > lds_dn ? lds_gu : lds_dn;
    static std::atomic<uint64_t> fused_attr{0};
    once_per_device(fused_attr, [] {
      constexpr int a = gu_wave_lds<FG>(kDecMaxEntries, kMaxExperts), b = ring_bytes<FD>();
      (void)hipFuncSetAttribute((const void*)moe_dec_fused_kernel<FG, FD, kFullK>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, a > b ? a : b);
    });
    const dim3 grid((unsigned)(items_gu + items_dn));
    if (A.gate_up_start && A.after_gate_up) {
      hipExtLaunchKernelGGL((moe_dec_fused_kernel<FG, FD, kFullK>), grid, dim3(64), lds, s,
                            (hipEvent_t)A.gate_up_start, (hipEvent_t)A.after_gate_up, 0, A.gate, A.up, A.down, A.R,
                            A.T, A.x, A.H, A.act, A.I, A.contrib, A.flags, A.max_slots);
    } else {
      hipLaunchKernelGGL((moe_dec_fused_kernel<FG, FD, kFullK>), grid, dim3(64), lds, s, A.gate, A.up, A.down, A.R,
                         A.T, A.x, A.H, A.act, A.I, A.contrib, A.flags, A.max_slots);
      if (A.after_gate_up) (void)hipEventRecord((hipEvent_t)A.after_gate_up, s);
    }
    if (A.after_down) (void)hipEventRecord((hipEvent_t)A.after_down, s);
  } else {
    if (A.gate_up_start && A.after_gate_up) {
      // the events take the kernel's own start and end timestamps
      hipExtLaunchKernelGGL((moe_dec_gate_up_kernel<FG, kFullK>), dim3((unsigned)items_gu), dim3(64 * ns_gu),
                            ns_gu * lds_gu, s, (hipEvent_t)A.gate_up_start, (hipEvent_t)A.after_gate_up, 0, A.gate,
                            A.up, A.R, A.T, A.x, A.H, A.act, A.I, A.S);
    } else {
      hipLaunchKernelGGL((moe_dec_gate_up_kernel<FG, kFullK>), dim3((unsigned)items_gu), dim3(64 * ns_gu),
                         ns_gu * lds_gu, s, A.gate, A.up, A.R, A.T, A.x, A.H, A.act, A.I, A.S);
      if (A.after_gate_up) (void)hipEventRecord((hipEvent_t)A.after_gate_up, s);
    }
    hipLaunchKernelGGL((moe_dec_down_kernel<FD, kFullK>), dim3((unsigned)items_dn), dim3(64 * ns_dn),
                       ns_dn * lds_dn, s, A.down, A.T, A.act, A.I, A.contrib, A.H, A.S, A.R.B);
    if (A.after_down) (void)hipEventRecord((hipEvent_t)A.after_down, s);
  }
  hipLaunchKernelGGL(moe_dec_combine_kernel, dim3(A.R.B, (unsigned)cdiv(A.H, 256)), dim3(64), 0, s, A.T,
                     A.contrib, A.H, A.R.K, A.sh_y, A.sh_scale, A.out, fused ? 1 : 0);
  return Q6MOE_OK;
}

bool dec_supported(int64_t B, int64_t K, int64_t E, int64_t width) {
  // the token streams address rows with 32-bit byte offsets (routes x width BF16)
  return B <= kDecMaxTokens && B * K <= kDecMaxEntries && E <= kMaxExperts && B * K * width * 2 < (1ll << 31);
}

template <int FG, int FD>
static int launch_k(const DecArgs& A, hipStream_t s) {
  const bool full = A.H % kQK == 0 && A.I % kQK == 0 && (A.S.is == 0 || A.S.is % kQK == 0);
  return full ? launch<FG, FD, true>(A, s) : launch<FG, FD, false>(A, s);
}

int launch_moe_decode(int fmt_gu, int fmt_dn, const DecArgs& A, hipStream_t s) {
  int rc = Q6MOE_OK;
  dispatch_formats(fmt_gu, fmt_dn,
                   [&](auto fg, auto fd) { rc = launch_k<decltype(fg)::value, decltype(fd)::value>(A, s); });
  return rc;
}

// Unit-decode probe of this path: one wave per unit copies the unit into an
// LDS ring stage with the kernels' own DMA (WStream::issue) and decodes it with
// WStream::decode, exactly as the streaming loop does, then stores the BF16
// weights. grid (units per expert, experts).
template <int FMT>
__global__ void __launch_bounds__(64) moe_dec_unpack_kernel(Proj p, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t st[stage_bytes<FMT>()];
  const int lane = threadIdx.x;
  const int e = blockIdx.y, rg = blockIdx.x / p.kb, kb = blockIdx.x - rg * p.kb;
  const WStream<FMT> ws(p, e, lane);
  ws.issue(rg, kb, st);
  wait_vm<0>();
  __builtin_amdgcn_s_waitcnt(0xc07f);
  u32x4 a[8];
  WStream<FMT>::decode(st, lane, a);
  store_unit_frags(a, out + (int64_t)e * p.rows * p.k, p, rg, kb, lane,
                   [](int f, int jA) { return Unit<FMT>::xoff(f, jA); });
}

int launch_dec_unpack(int fmt, const Proj& p, int experts, uint16_t* out, hipStream_t s) {
  const dim3 grid((unsigned)(cdiv(p.rows, 16) * p.kb), (unsigned)experts);
  if (fmt == FMT_Q6)
    hipLaunchKernelGGL(moe_dec_unpack_kernel<FMT_Q6>, grid, dim3(64), 0, s, p, out);
  else if (fmt == FMT_Q4K)
    hipLaunchKernelGGL(moe_dec_unpack_kernel<FMT_Q4K>, grid, dim3(64), 0, s, p, out);
  else if (fmt == FMT_Q5K)
    hipLaunchKernelGGL(moe_dec_unpack_kernel<FMT_Q5K>, grid, dim3(64), 0, s, p, out);
  else if (fmt == FMT_Q51)
    hipLaunchKernelGGL(moe_dec_unpack_kernel<FMT_Q51>, grid, dim3(64), 0, s, p, out);
  else
    hipLaunchKernelGGL(moe_dec_unpack_kernel<FMT_Q8>, grid, dim3(64), 0, s, p, out);
  return Q6MOE_OK;
}

}  // namespace q6moe
