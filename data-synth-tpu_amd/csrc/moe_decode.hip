// Decode-shaped routed experts: three launches per step.
//
//   moe_dec_gate_up_kernel  every workgroup derives the (small) routing itself
//        -- merged BF16 route weights (kaggle/qwen38_tpu/experts.py:66-73),
//        active experts in ascending id (:74-76), the expert's tokens in
//        ascending order -- then each wave streams one 16-row group of gate
//        and up over the full K for that expert and applies SwiGLU in
//        registers: a = RNE(RNE(g * sigmoid(g)) * u) (experts.py:103-107).
//        Workgroups of row block 0 publish the routing tables.
//   moe_dec_down_kernel     each wave streams one 16-row group of down,
//        y = RNE(a Wd^T) (experts.py:108), and stores the exact FP32 product
//        f32(y) * f32(r) token-major at the route's rank among its token's
//        experts (ascending expert id).
//   moe_dec_combine_kernel  out = RNE(sum over ranks of the contributions),
//        i.e. the FP32 sum over experts in ascending id (experts.py:129-131),
//        plus RNE(routed + shared) with a shared expert (engine.py:199-203).
//
// Memory pipeline: each wave owns a ring of kStages weight units (16 rows x
// one 256-wide K block) in LDS, filled by direct global->LDS DMA
// (global_load_lds) kStages-1 units ahead of the unit being decoded, so the
// bytes in flight do not cost registers. The token activations a workgroup
// multiplies are staged in LDS once, so inside the main loop the only vector
// memory traffic is the ring DMA and every wait count is a compile-time
// constant. Weights are read exactly once per step.
#include "moe_common.h"
#include "q6moe_api.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

namespace q6moe {

constexpr int kDecMaxEntries = 1024;  // tokens * top_k handled by the decode path
constexpr int kDecMaxTokens = 256;    // tokens handled by the decode path
constexpr int kDecMaxExperts = 256;
constexpr int kDecWaves = 4;
constexpr int kStages = 2;
constexpr int kLdsBudget = 40 * 1024;  // per workgroup: four workgroups per CU

// One unit in LDS. Q6_K: ql 2048 B and qh 1024 B chunk-major (slot = chunk*16 +
// row), sub-scales 256 B and FP16 d 32 B (+ padding) row-major. Q4_K: 16 rows x
// 9 chunks of 16 B, chunk-major in three 1 KB groups.
constexpr int kStageBytes = 3584;
constexpr int kUnitDma = 5;  // DMA instructions per unit (both formats)

__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, LDS_PTR(lds_base), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, LDS_PTR(lds_base), 4, 0, 0);
}

// s_waitcnt vmcnt(n) with lgkmcnt/expcnt left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until at most ``ahead`` units issued after the current one are pending.
__device__ __forceinline__ void wait_units(int ahead) {
  if (kStages > 2 && ahead >= 2)
    wait_vm<2 * kUnitDma>();
  else if (ahead >= 1)
    wait_vm<kUnitDma>();
  else
    wait_vm<0>();
}

template <int FMT>
struct LdsUnit;

template <>
struct LdsUnit<FMT_Q6> {
  // Issue the DMA of rows 16*(rg%4).. of tile (rg/4), K block kb into ``st``.
  static __device__ __forceinline__ void issue(const Proj& p, int64_t e, int rg, int kb, int lane,
                                               uint8_t* st) {
    const int64_t t = (int64_t)(rg >> 2) * p.kb + kb;
    const uint8_t* tile = p.data + e * p.dstride + t * kTileBytes;
    const int r0 = (rg & 3) * 16, j = lane & 15, c = lane >> 4;
    const uint8_t* ql = tile + kQlOff + (r0 + j) * 128 + 16 * c;
    dma16(ql, st);
    dma16(ql + 64, st + 1024);
    dma16(tile + kQhOff + (r0 + j) * 64 + 16 * c, st + 2048);
    dma4(tile + kScOff + r0 * 16 + 4 * lane, st + 3072);
    dma4(p.scales + e * p.sstride + t * 128 + r0 * 2 + 4 * (lane & 7), st + 3328);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const int j = lane & 15, jA = lane >> 4;
    Q6Raw r;
    r.qlA = *reinterpret_cast<const u32x4*>(st + 16 * (jA * 16 + j));
    r.qlB = *reinterpret_cast<const u32x4*>(st + 1024 + 16 * (jA * 16 + j));
    r.qhA = *reinterpret_cast<const u32x4*>(st + 2048 + 16 * ((jA & 1) * 16 + j));
    r.qhB = *reinterpret_cast<const u32x4*>(st + 2048 + 16 * (((jA & 1) + 2) * 16 + j));
    r.sc = *reinterpret_cast<const u32x4*>(st + 3072 + 16 * j);
    r.d = *reinterpret_cast<const uint16_t*>(st + 3328 + 2 * j);
    q6_decode_unit(r, jA, a);
  }
};

template <>
struct LdsUnit<FMT_Q4K> {
  // 16 GGUF rows (144 B each) of K block kb: chunk c (16 B) of row j goes to
  // group c/4, slot (c%4)*16 + j. Chunk 0 is the header, chunks 1-8 the codes.
  static __device__ __forceinline__ void issue(const Proj& p, int64_t e, int rg, int kb, int lane,
                                               uint8_t* st) {
    const int j = lane & 15, c = lane >> 4;
    int row = rg * 16 + j;
    row = row < p.rows ? row : p.rows - 1;  // stay in bounds; result row discarded
    const uint8_t* blk = p.data + e * p.dstride + ((int64_t)row * p.kb + kb) * 144;
    dma16(blk + 16 * c, st);
    dma16(blk + 64 + 16 * c, st + 1024);
    dma16(blk + 128, st + 2048);  // chunk 8 (each lane group repeats it)
    dma4(blk, st + 3072);         // keeps kUnitDma uniform; not read
    dma4(blk, st + 3328);
  }
  static __device__ __forceinline__ void decode(const uint8_t* st, int lane, u32x4 a[8]) {
    const int j = lane & 15, jA = lane >> 4;
    auto chunk = [&](int c) -> u32x4 {
      return *reinterpret_cast<const u32x4*>(st + 1024 * (c >> 2) + 16 * ((c & 3) * 16 + j));
    };
    Unit<FMT_Q4K> u;
    u.hdr = chunk(0);
    u.qa = chunk(1 + 2 * jA);
    u.qb = chunk(2 + 2 * jA);
    u.decode(a, lane);
  }
};

// Per-workgroup routing. On return (uniform across the block): slot's expert,
// first position and count, the active-expert count, and the slot's token list
// in LDS. Returns false for an inactive slot.
__device__ bool dec_route(const DecRoute& R, int slot, int publish, const DecTables& T, int* s_ids,
                          float* s_r, int* s_cnt, int* s_tok, int* s_info) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int n = R.B * R.K;
  for (int e = tid; e < R.E; e += nthr) s_cnt[e] = 0;
  for (int i = tid; i < n; i += nthr) s_ids[i] = R.ids[i];
  __syncthreads();
  for (int i = tid; i < n; i += nthr) {
    const int b = i / R.K, kk = i - b * R.K;
    const int id = s_ids[i];
    bool first = id >= 0 && id < R.E;
    for (int k2 = 0; k2 < kk && first; ++k2) first = s_ids[b * R.K + k2] != id;
    float r = 0.f;
    if (first) {
      float s = 0.f;
      for (int k2 = kk; k2 < R.K; ++k2)
        if (s_ids[b * R.K + k2] == id) s += bf16_to_float(R.wts[b * R.K + k2]);
      r = bf16_round(s);
      if (r != 0.f) atomicAdd(&s_cnt[id], 1);
      else r = 0.f;
    }
    s_r[i] = r;
  }
  __syncthreads();
  if (tid < 64) {
    // wave 0: exclusive scans over experts (4 per lane) of active flags and counts
    const int lane = tid;
    int act[4], cnt[4];
    int la = 0, lc = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = lane * 4 + q;
      cnt[q] = e < R.E ? s_cnt[e] : 0;
      act[q] = cnt[q] > 0;
      la += act[q];
      lc += cnt[q];
    }
    int ia = la, ic = lc;  // inclusive scans across lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int ta = __shfl_up(ia, off), tc = __shfl_up(ic, off);
      if (lane >= off) {
        ia += ta;
        ic += tc;
      }
    }
    int ea = ia - la, ec = ic - lc;
    const int total_active = __shfl(ia, 63);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (act[q]) {
        if (ea == slot) {
          s_info[0] = lane * 4 + q;
          s_info[1] = ec;
          s_info[2] = cnt[q];
        }
        if (publish) {
          T.slot_e[ea] = lane * 4 + q;
          T.slot_t0[ea] = ec;
          T.slot_cnt[ea] = cnt[q];
        }
      }
      ea += act[q];
      ec += cnt[q];
    }
    if (lane == 0) s_info[3] = total_active;
    if (publish && lane == 0) T.hdr[0] = total_active;
  }
  if (publish && slot == 0) {
    // one workgroup publishes each token's route count
    for (int b = tid; b < R.B; b += nthr) {
      int m = 0;
      for (int kk = 0; kk < R.K; ++kk) m += s_r[b * R.K + kk] != 0.f;
      T.tok_n[b] = m;
    }
  }
  __syncthreads();
  const int total_active = s_info[3];
  if (slot >= total_active) return false;
  const int e = s_info[0], t0 = s_info[1];
  if (tid < 64) {
    // wave 0: this expert's routes in ascending entry (= token) order
    int run = 0;
    for (int c0 = 0; c0 < n; c0 += 64) {
      const int i = c0 + tid;
      const bool hit = i < n && s_ids[i] == e && s_r[i] != 0.f;
      const unsigned long long m = __ballot(hit);
      if (hit) {
        const int rank = run + __popcll(m & ((1ull << tid) - 1ull));
        const int b = i / R.K;
        s_tok[rank] = b;
        if (publish) {
          // rank of this route among its token's routes = routed experts with a smaller id
          int er = 0;
          for (int kk = 0; kk < R.K; ++kk) {
            const int o = b * R.K + kk;
            er += (s_r[o] != 0.f) && s_ids[o] < e;
          }
          T.route_w[t0 + rank] = s_r[i];
          T.route_dst[t0 + rank] = b * R.K + er;
        }
      }
      run += __popcll(m);
    }
  }
  __syncthreads();
  return true;
}

// Copy ``rows`` activation rows (row r -> src_row(r)) of width k into LDS.
template <typename RowFn>
__device__ __forceinline__ void stage_rows(uint16_t* xs, int rows, int k, RowFn src_row) {
  const int per_row = k / 8;
  for (int i = threadIdx.x; i < rows * per_row; i += blockDim.x) {
    const int r = i / per_row, c = (i - r * per_row) * 8;
    *reinterpret_cast<u32x4*>(xs + r * k + c) = *reinterpret_cast<const u32x4*>(src_row(r) + c);
  }
}

// 8 x operands of K block kb for token row ``xr`` (LDS), zero past k.
template <int FMT, bool kFullK>
__device__ __forceinline__ void lds_x(u32x4 xf[8], const uint16_t* xr, int kb, int jA, int k) {
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const int col = kb * kQK + Unit<FMT>::xoff(f, jA);
    xf[f] = (kFullK || col + 8 <= k) ? *reinterpret_cast<const u32x4*>(xr + col) : u32x4{0u, 0u, 0u, 0u};
  }
}

// The shared memory of one decode workgroup: [token list | x stage | rings].
// The routing scratch overlays the rings (it is dead before the first DMA).
struct DecLds {
  int* tok;
  uint16_t* xs;
  uint8_t* ring;
  int* s_ids;
  float* s_r;
  int* s_cnt;
  int* info;
};

__device__ __forceinline__ DecLds carve(uint8_t* base, int xt, int k) {
  DecLds L;
  L.info = reinterpret_cast<int*>(base);
  L.tok = reinterpret_cast<int*>(base + 64);
  L.xs = reinterpret_cast<uint16_t*>(base + 64 + 4 * kDecMaxTokens);
  L.ring = base + 64 + 4 * kDecMaxTokens + 2 * xt * k;
  L.s_ids = reinterpret_cast<int*>(L.ring);
  L.s_r = reinterpret_cast<float*>(L.ring + 4 * kDecMaxEntries);
  L.s_cnt = reinterpret_cast<int*>(L.ring + 8 * kDecMaxEntries);
  return L;
}

size_t dec_lds_bytes(int xt, int k) {
  return 64 + 4 * kDecMaxTokens + 2 * (size_t)xt * k + (size_t)kDecWaves * kStages * kStageBytes;
}

// Token rows staged per pass so that one workgroup stays within both the
// budget (four workgroups per CU) and the device's per-workgroup LDS limit.
int dec_x_tokens(int k, int max_lds) {
  const int64_t fixed = 64 + 4 * kDecMaxTokens + (int64_t)kDecWaves * kStages * kStageBytes;
  const int64_t budget = max_lds < kLdsBudget ? max_lds : kLdsBudget;
  int64_t xt = (budget - fixed) / (2 * (int64_t)k);
  return (int)(xt > 16 ? 16 : xt);
}

static int device_max_lds() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 65536;
  return v;
}

template <int FMT, bool kFullK>
__global__ void __launch_bounds__(64 * kDecWaves) __attribute__((amdgpu_waves_per_eu(4)))
    moe_dec_gate_up_kernel(Proj gate, Proj up, DecRoute R, DecTables T, const uint16_t* __restrict__ x,
                           int hidden, uint16_t* __restrict__ act, int inter, int xt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const DecLds L = carve(smem, xt, hidden);
  const int slot = blockIdx.x;
  const int publish = blockIdx.y == 0;
  if (!dec_route(R, slot, publish, T, L.s_ids, L.s_r, L.s_cnt, L.tok, L.info)) return;
  const int64_t e = L.info[0];
  const int t0 = L.info[1], cnt = L.info[2];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rg = blockIdx.y * kDecWaves + wave;
  const bool live = rg * 16 < inter;
  uint8_t* ring = L.ring + wave * kStages * kStageBytes;
  const int kbs = gate.kb;
  const int nu = 2 * kbs;  // units: gate kb, up kb, gate kb+1, ...
  for (int tc = 0; tc < cnt; tc += xt) {
    const int nt = cnt - tc < xt ? cnt - tc : xt;
    __syncthreads();  // previous chunk's readers are done with the x stage
    stage_rows(L.xs, nt, hidden, [&](int r) { return x + (int64_t)L.tok[tc + r] * hidden; });
    __syncthreads();
    if (live) {
      const uint16_t* xr = L.xs + (j < nt ? j : 0) * hidden;
      f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
      auto issue = [&](int u) {
        LdsUnit<FMT>::issue((u & 1) ? up : gate, e, rg, u >> 1, lane, ring + (u % kStages) * kStageBytes);
      };
      for (int u = 0; u < kStages - 1 && u < nu; ++u) issue(u);
      u32x4 xf[8];
      for (int u = 0; u < nu; ++u) {
        if (u + kStages - 1 < nu) issue(u + kStages - 1);
        const int ahead = nu - 1 - u;
        wait_units(ahead < kStages - 1 ? ahead : kStages - 1);
        if (!(u & 1)) lds_x<FMT, kFullK>(xf, xr, u >> 1, jA, hidden);
        u32x4 a[8];
        LdsUnit<FMT>::decode(ring + (u % kStages) * kStageBytes, lane, a);
        if (u & 1) {
#pragma unroll
          for (int f = 0; f < 8; ++f) au = mfma16(a[f], xf[f], au);
        } else {
#pragma unroll
          for (int f = 0; f < 8; ++f) ag = mfma16(a[f], xf[f], ag);
        }
      }
      // lane holds rows 4*(lane/16)+i, token column lane%16 of both accumulators
      if (j < nt) {
        const int q = tc + j;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = rg * 16 + 4 * jA + i;
          if (row < inter) {
            const float g = bf16_round(ag[i]);
            const float uu = bf16_round(au[i]);
            const float sg = bf16_round(g * sigmoid_acc(g));
            act[(int64_t)(t0 + q) * inter + row] = bf16_bits(sg * uu);
          }
        }
      }
    }
  }
}

template <int FMT, bool kFullK>
__global__ void __launch_bounds__(64 * kDecWaves) __attribute__((amdgpu_waves_per_eu(4)))
    moe_dec_down_kernel(Proj down, DecTables T, const uint16_t* __restrict__ act, int inter,
                        float* __restrict__ contrib, int hidden, int xt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const DecLds L = carve(smem, xt, inter);
  const int slot = blockIdx.x;
  const int n_active = T.hdr[0];
  if (slot >= n_active) return;
  const int64_t e = T.slot_e[slot];
  const int t0 = T.slot_t0[slot], cnt = T.slot_cnt[slot];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rg = blockIdx.y * kDecWaves + wave;
  const bool live = rg * 16 < hidden;
  uint8_t* ring = L.ring + wave * kStages * kStageBytes;
  const int kbs = down.kb;
  for (int tc = 0; tc < cnt; tc += xt) {
    const int nt = cnt - tc < xt ? cnt - tc : xt;
    __syncthreads();
    stage_rows(L.xs, nt, inter, [&](int r) { return act + (int64_t)(t0 + tc + r) * inter; });
    __syncthreads();
    if (live) {
      const uint16_t* xr = L.xs + (j < nt ? j : 0) * inter;
      const int pos = t0 + tc + (j < nt ? j : 0);
      const int dst = T.route_dst[pos];
      const float w = T.route_w[pos];
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      auto issue = [&](int u) {
        LdsUnit<FMT>::issue(down, e, rg, u, lane, ring + (u % kStages) * kStageBytes);
      };
      for (int u = 0; u < kStages - 1 && u < kbs; ++u) issue(u);
      for (int u = 0; u < kbs; ++u) {
        if (u + kStages - 1 < kbs) issue(u + kStages - 1);
        const int ahead = kbs - 1 - u;
        wait_units(ahead < kStages - 1 ? ahead : kStages - 1);
        u32x4 xf[8];
        lds_x<FMT, kFullK>(xf, xr, u, jA, inter);
        u32x4 a[8];
        LdsUnit<FMT>::decode(ring + (u % kStages) * kStageBytes, lane, a);
#pragma unroll
        for (int f = 0; f < 8; ++f) acc = mfma16(a[f], xf[f], acc);
      }
      if (j < nt) {
        f32x4 c;
#pragma unroll
        for (int i = 0; i < 4; ++i) c[i] = bf16_round(acc[i]) * w;  // exact product
        const int row = rg * 16 + 4 * jA;
        if (row + 4 <= hidden) {
          *reinterpret_cast<f32x4*>(contrib + (int64_t)dst * hidden + row) = c;
        } else {
          for (int i = 0; i < 4; ++i)
            if (row + i < hidden) contrib[(int64_t)dst * hidden + row + i] = c[i];
        }
      }
    }
  }
}

// out[b, h] = RNE(sum_r contrib[b, r, h]) over the token's routes in rank
// (= ascending expert id) order; with a shared expert RNE(f32(routed) + shared).
__global__ void __launch_bounds__(256)
    moe_dec_combine_kernel(DecTables T, const float* __restrict__ contrib, int hidden, int K,
                           const uint16_t* __restrict__ sh_y, const uint16_t* __restrict__ sh_scale,
                           uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int h = (blockIdx.y * blockDim.x + threadIdx.x) * 8;
  if (h >= hidden) return;
  const int m = T.tok_n[b];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const float* base = contrib + (int64_t)b * K * hidden + h;
  for (int r = 0; r < m; ++r) {
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(base + (int64_t)r * hidden);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(base + (int64_t)r * hidden + 4);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      acc[c] += v0[c];
      acc[4 + c] += v1[c];
    }
  }
  u32x4 o;
  if (sh_y) {
    const u32x4 sv = *reinterpret_cast<const u32x4*>(sh_y + (int64_t)b * hidden + h);
    const float gs = sh_scale ? bf16_to_float(sh_scale[b]) : 1.f;
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float sy = bf16_to_float((uint16_t)(sv[c >> 1] >> (16 * (c & 1))));
      if (sh_scale) sy = bf16_round(sy * gs);
      v[c] = bf16_round(acc[c]) + sy;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = pack_bf16x2(v[2 * c], v[2 * c + 1]);
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = pack_bf16x2(acc[2 * c], acc[2 * c + 1]);
  }
  *reinterpret_cast<u32x4*>(out + (int64_t)b * hidden + h) = o;
}

template <int FMT, bool kFullK>
static int launch(const DecArgs& A, hipStream_t s) {
  const int max_lds = device_max_lds();
  const int xt1 = dec_x_tokens(A.H, max_lds), xt2 = dec_x_tokens(A.I, max_lds);
  if (xt1 < 1 || xt2 < 1) {
    set_error("moe_forward: hidden/intermediate too wide for the decode kernels' LDS stage");
    return Q6MOE_ERR_UNSUPPORTED;
  }
  const size_t lds1 = dec_lds_bytes(xt1, A.H), lds2 = dec_lds_bytes(xt2, A.I);
  hipFuncSetAttribute((const void*)moe_dec_gate_up_kernel<FMT, kFullK>,
                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
  hipFuncSetAttribute((const void*)moe_dec_down_kernel<FMT, kFullK>,
                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
  hipLaunchKernelGGL((moe_dec_gate_up_kernel<FMT, kFullK>),
                     dim3(A.max_slots, (unsigned)cdiv(A.I, 16 * kDecWaves)), dim3(64 * kDecWaves), lds1, s, A.gate, A.up, A.R, A.T, A.x, A.H, A.act, A.I, xt1);
  if (A.after_gate_up) hipEventRecord((hipEvent_t)A.after_gate_up, s);
  hipLaunchKernelGGL((moe_dec_down_kernel<FMT, kFullK>),
                     dim3(A.max_slots, (unsigned)cdiv(A.H, 16 * kDecWaves)), dim3(64 * kDecWaves), lds2, s, A.down, A.T, A.act, A.I, A.contrib, A.H, xt2);
  if (A.after_down) hipEventRecord((hipEvent_t)A.after_down, s);
  hipLaunchKernelGGL(moe_dec_combine_kernel, dim3(A.R.B, (unsigned)cdiv(A.H, 256 * 8)), dim3(256), 0, s, A.T,
                     A.contrib, A.H, A.R.K, A.sh_y, A.sh_scale, A.out);
  return Q6MOE_OK;
}

bool dec_supported(int64_t B, int64_t K, int64_t E) {
  return B <= kDecMaxTokens && B * K <= kDecMaxEntries && E <= kDecMaxExperts;
}

int launch_moe_decode(int fmt, const DecArgs& A, hipStream_t s) {
  const bool full = A.H % kQK == 0 && A.I % kQK == 0;
  if (fmt == FMT_Q6) return full ? launch<FMT_Q6, true>(A, s) : launch<FMT_Q6, false>(A, s);
  return full ? launch<FMT_Q4K, true>(A, s) : launch<FMT_Q4K, false>(A, s);
}

}  // namespace q6moe
