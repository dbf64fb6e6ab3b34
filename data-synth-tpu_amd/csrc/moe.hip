// Routed SwiGLU expert FFN over packed Q6_K / Q4_K experts.
//
// Replaces expert_parallel / grouped_expert_parallel's per-shard body
// (kaggle/qwen38_tpu/experts.py:61-131, grouped_experts.py:185-292) on one GPU:
//
//   moe_route_kernel     route weights per (token, expert) with duplicate ids
//                        summed in BF16 (experts.py:66-73), active experts in
//                        ascending id (:74-76), routes grouped by expert with
//                        tokens ascending, per-token route lists for the combine.
//   moe_gate_up_kernel   g = RNE(x Wg^T), u = RNE(x Wu^T), a = RNE(RNE(g*sig(g))*u)
//                        (experts.py:103-107, math.py:10-20) fused in one pass.
//   moe_down_kernel      y = RNE(a Wd^T) (experts.py:108).
//   moe_combine_kernel   out[b] = RNE(sum over experts, ascending id, of
//                        f32(y) * f32(r)) (experts.py:108-110,129-131), plus the
//                        optional always-on shared expert RNE(routed + shared).
//
// No atomics touch floating-point data, so results are bitwise reproducible.
#include <algorithm>
#include <mutex>

#include "moe_common.h"
#include "q6moe_api.h"

namespace q6moe {

constexpr int kChunk = 256;  // tokens per routing workgroup
constexpr int kChunkWords = kChunk / 32;
constexpr int kExpertsPerLane = kMaxExperts / kChunk;  // experts per lane of a routing workgroup

__device__ __forceinline__ bool is_route(float r) { return r != 0.f || r != r; }

// Copies n (>= 1) consecutive values of two arrays into LDS, converted by
// cva and cvb. Every lane's loads of both (eight of each per pass) are issued
// before its first store, so a chunk's rows arrive in one memory round trip
// per 8 * kChunk values. Indexes past n are clamped to n - 1 for the load and
// the store alike (a repeat store of element n-1's own value), so no load or
// store sits behind a branch.
template <typename DA, typename SA, typename CvA, typename DB, typename SB, typename CvB>
__device__ __forceinline__ void stage_chunk2(DA* da, const SA* __restrict__ sa, CvA cva, DB* db,
                                             const SB* __restrict__ sb, CvB cvb, int n) {
  for (int i0 = threadIdx.x; i0 < n; i0 += 8 * kChunk) {
    SA va[8];
    SB vb[8];
    int ix[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      ix[u] = i0 + u * kChunk < n ? i0 + u * kChunk : n - 1;
      va[u] = sa[ix[u]];
      vb[u] = sb[ix[u]];
    }
    asm volatile("" ::: "memory");  // the loads above stay ahead of the stores below
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      da[ix[u]] = cva(va[u]);
      db[ix[u]] = cvb(vb[u]);
    }
  }
}

// Routing with G lanes per token (top_k <= KM, the token's row in registers;
// lane g of a group takes slots g, g + G, ...), used by the one-launch
// routing of few tokens.
template <int KM>
__device__ __forceinline__ void load_row(const int* s_ids, const float* s_v, int b, int K, int (&rid)[KM],
                                         float (&rv)[KM]) {
#pragma unroll
  for (int k2 = 0; k2 < KM; ++k2) {
    rid[k2] = k2 < K ? s_ids[b * K + k2] : -1;
    rv[k2] = k2 < K ? s_v[b * K + k2] : 0.f;
  }
}

// Merged BF16 weight of slot kk of token b (experts.py:66-73: the sum of the
// weights of slots kk.. with its id, in slot order, on the first occurrence of
// an id in range; 0 otherwise, as route_merge) into s_m, the expert's route
// count in cnt and the token's bit in the expert's token bitmap.
template <int KM>
__device__ __forceinline__ void merge_grp(const int* s_ids, const float* s_w, float* s_m, int* cnt, uint32_t* bits,
                                          int b, int g, int G, int K, int E) {
  int rid[KM];
  float rw[KM];
  load_row<KM>(s_ids, s_w, b, K, rid, rw);
  for (int kk = g; kk < K; kk += G) {
    const int e = s_ids[b * K + kk];  // from LDS: a run-time index into rid would go to scratch
    bool first = e >= 0 && e < E;
    float sum = 0.f;
#pragma unroll
    for (int k2 = 0; k2 < KM; ++k2) {
      first = first && !(k2 < kk && rid[k2] == e);
      if (k2 >= kk && rid[k2] == e) sum += rw[k2];
    }
    const float m = first ? bf16_round(sum) : 0.f;
    const bool route = first && is_route(m);
    s_m[b * K + kk] = route ? m : 0.f;
    if (route) {
      atomicAdd(&cnt[e], 1);
      atomicOr(&bits[e * kChunkWords + (b >> 5)], 1u << (b & 31));
    }
  }
}

// Places the routes of token b (of the chunk; bglob in the batch): a route's
// position is its expert's first position s_pos[e] plus the number of earlier
// tokens of the chunk routed to e (token bitmaps); route_tok and route_w at
// that position, and the position into the token's row tp at the number of
// the token's routes to smaller expert ids (positions are expert-major, so the
// row is ascending); the row's slots from the token's route count on hold -1.
template <int KM>
__device__ __forceinline__ void place_grp(const int* s_ids, const float* s_m, const uint32_t* bits, const int* s_pos,
                                          int b, int g, int G, int K, int bglob, int* tp, MoeWs ws) {
  int rid[KM];
  float rm[KM];
  load_row<KM>(s_ids, s_m, b, K, rid, rm);
  int nr = 0;
#pragma unroll
  for (int k2 = 0; k2 < KM; ++k2) nr += is_route(rm[k2]);
  for (int kk = g; kk < K; kk += G) {
    const int e = s_ids[b * K + kk];
    const float r = s_m[b * K + kk];
    if (is_route(r)) {
      int q = 0;
#pragma unroll
      for (int k2 = 0; k2 < KM; ++k2) q += is_route(rm[k2]) && rid[k2] < e;
      int rank = __popc(bits[e * kChunkWords + (b >> 5)] & ((1u << (b & 31)) - 1u));
#pragma unroll
      for (int w = 0; w < kChunkWords - 1; ++w)
        if (w < (b >> 5)) rank += __popc(bits[e * kChunkWords + w]);
      const int p = s_pos[e] + rank;
      ws.route_tok[p] = bglob;
      ws.route_w[p] = r;
      tp[q] = p;
    }
    if (kk >= nr) tp[kk] = -1;
  }
}

// Merged BF16 weight of each first occurrence of an id in a token
// (experts.py:66-73; 0 for repeats and out-of-range ids), in place of the
// staged weights s_w, and the per-expert route counts cnt, for the nb staged
// tokens of a chunk (lane tid = token tid).
// top_k <= KM: the token's entries in registers, every loop unrolled (the
// same comparisons and the same summation order as merge_grp)
template <int KM>
__device__ __forceinline__ void route_merge_regs(const int* s_ids, float* s_w, int* cnt, int K, int E) {
  const int tid = threadIdx.x;
  int id[KM];
  float w[KM], mg[KM];
#pragma unroll
  for (int kk = 0; kk < KM; ++kk) {
    id[kk] = kk < K ? s_ids[tid * K + kk] : -1;
    w[kk] = kk < K ? s_w[tid * K + kk] : 0.f;
  }
#pragma unroll
  for (int kk = 0; kk < KM; ++kk) {
    const int e = id[kk];
    bool first = kk < K && e >= 0 && e < E;
#pragma unroll
    for (int k2 = 0; k2 < kk; ++k2) first = first && id[k2] != e;
    float sum = 0.f;
#pragma unroll
    for (int k2 = kk; k2 < KM; ++k2)
      if (k2 < K && id[k2] == e) sum += w[k2];
    const float m = first ? bf16_round(sum) : 0.f;
    if (first && is_route(m)) atomicAdd(&cnt[e], 1);
    mg[kk] = is_route(m) ? m : 0.f;
  }
#pragma unroll
  for (int kk = 0; kk < KM; ++kk)
    if (kk < K) s_w[tid * K + kk] = mg[kk];
}

__device__ __forceinline__ void route_merge(const int* s_ids, float* s_w, int* cnt, int nb, int K, int E) {
  const int tid = threadIdx.x;
  if (tid < nb && K <= 8) {
    route_merge_regs<8>(s_ids, s_w, cnt, K, E);
  } else if (tid < nb && K <= 16) {
    route_merge_regs<16>(s_ids, s_w, cnt, K, E);
  } else if (tid < nb) {
    route_merge_regs<32>(s_ids, s_w, cnt, K, E);
  }
}

// Routing, pass 1 (one workgroup per chunk of kChunk tokens, one lane per
// token): merged BF16 weight of each first occurrence of an id in a token
// (experts.py:66-73; 0 for repeats and out-of-range ids) and the chunk's
// route count per expert.
__global__ void __launch_bounds__(kChunk)
    moe_route_count_kernel(const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int B, int K,
                           int E, MoeWs ws, int* __restrict__ chunk_cnt) {
  extern __shared__ int sm[];
  int* s_ids = sm;                                            // [kChunk * K]
  float* s_w = reinterpret_cast<float*>(sm + kChunk * K);     // [kChunk * K] weights, then merged weights
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x, b0 = blockIdx.x * kChunk;
  const int nb = B - b0 < kChunk ? B - b0 : kChunk;
  const int64_t e0 = (int64_t)b0 * K;
  for (int e = tid; e < E; e += kChunk) cnt[e] = 0;
  stage_chunk2(s_ids, ids + e0, [](int v) { return v; }, s_w, wts + e0, [](uint16_t v) { return bf16_to_float(v); },
               nb * K);
  __syncthreads();
  route_merge(s_ids, s_w, cnt, nb, K, E);
  __syncthreads();
  for (int i = tid; i < nb * K; i += kChunk) ws.ent_r[e0 + i] = s_w[i];
  for (int e = tid; e < E; e += kChunk) chunk_cnt[(int64_t)blockIdx.x * E + e] = cnt[e];
}

// Scans over experts (lane e = expert e, whole waves of the workgroup; lanes
// from E on carry nothing): each expert's first route position (returned)
// and, with ``publish``, the active experts in ascending id
// (experts.py:74-76) into ws.active, their first positions into ws.act_off,
// the prefill tiles of mtile routes, and the totals in ws.hdr (written by the
// workgroup's last lane).
__device__ __forceinline__ int route_scan(int e, int E, int total, int mtile, MoeWs ws,
                                          int (*s_wt)[kMaxExperts / 64], bool publish = true) {
  const int lane = e & 63, wv = e >> 6;
  const int act = total > 0, nt = (total + mtile - 1) / mtile;
  // inclusive scans of (active, routes, tiles) in expert order: within each
  // wave by shuffles, then plus the totals of the earlier waves
  int ia = act, ic = total, it = nt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int ta = __shfl_up(ia, off), tc = __shfl_up(ic, off), tt = __shfl_up(it, off);
    if (lane >= off) {
      ia += ta;
      ic += tc;
      it += tt;
    }
  }
  if (lane == 63) {
    s_wt[0][wv] = ia;
    s_wt[1][wv] = ic;
    s_wt[2][wv] = it;
  }
  __syncthreads();
  for (int w = 0; w < wv; ++w) {
    ia += s_wt[0][w];
    ic += s_wt[1][w];
    it += s_wt[2][w];
  }
  const int slot = ia - act, base = ic - total, t0 = it - nt;
  if (!publish) return base;
  if (e < E) {
    if (act) {
      ws.active[slot] = e;
      ws.act_off[slot] = base;
      for (int j = 0; j < nt; ++j) {
        const int r0 = base + j * mtile;
        ws.tile[t0 + j] = PfTile{e, r0, total - j * mtile < mtile ? total - j * mtile : mtile, slot};
      }
    }
  }
  if (e == (int)blockDim.x - 1) {  // lanes past E add nothing: the last one holds the totals
    ws.act_off[ia] = ic;
    ws.hdr[0] = ia;
    ws.hdr[1] = ic;
    ws.hdr[2] = it;
  }
  return base;
}

// Routing, pass 2 (one workgroup of E lanes rounded up to whole waves, one
// lane per expert): active experts in ascending id (experts.py:74-76), each
// expert's first route position, the 128-route prefill tiles, each chunk's
// first position per expert relative to the expert's first (chunk_cnt is
// rewritten in place) and, in row nchunks of chunk_cnt, each expert's first
// position.
__global__ void __launch_bounds__(kMaxExperts)
    moe_route_scan_kernel(int E, int nchunks, int mtile, MoeWs ws, int* __restrict__ chunk_cnt) {
  __shared__ int s_wt[3][kMaxExperts / 64];  // per-wave totals of the three scans
  const int e = threadIdx.x;
  int total = 0;
  if (e < E) {
    for (int c0 = 0; c0 < nchunks; c0 += 8) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u < nchunks ? c0 + u : nchunks - 1;
        v[u] = chunk_cnt[(int64_t)c * E + e];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + u < nchunks) {
          chunk_cnt[(int64_t)(c0 + u) * E + e] = total;
          total += v[u];
        }
    }
  }
  const int base = route_scan(e, E, total, mtile, ws, s_wt);
  if (e < E) chunk_cnt[(int64_t)nchunks * E + e] = base;
}

// Places a chunk's routes (lane tid = token b0 + tid of the nb staged ones):
// per-expert token bitmaps give each route its rank among the chunk's tokens
// of its expert, so its position is s_pos[e] (the expert's first position
// plus the chunk's offset within it) plus that rank; route_tok and route_w at
// the position; per token, its positions in ascending expert id into s_tp.
// top_k <= KM: the token's entries and its position list in registers; the
// list is sorted by an odd-even transposition network (non-routes last)
template <int KM>
__device__ __forceinline__ void route_place_regs(const int* s_ids, const float* s_r, int* s_tp,
                                                 const uint32_t* bits, const int* s_pos, int K, int b0, MoeWs ws) {
  const int tid = threadIdx.x;
  int pos[KM];
#pragma unroll
  for (int kk = 0; kk < KM; ++kk) {
    pos[kk] = 0x7fffffff;
    const float r = kk < K ? s_r[tid * K + kk] : 0.f;
    if (kk < K && is_route(r)) {
      const int e = s_ids[tid * K + kk];
      int rank = __popc(bits[e * kChunkWords + (tid >> 5)] & ((1u << (tid & 31)) - 1u));
#pragma unroll
      for (int w = 0; w < kChunkWords - 1; ++w)
        if (w < (tid >> 5)) rank += __popc(bits[e * kChunkWords + w]);
      const int p = s_pos[e] + rank;
      ws.route_tok[p] = b0 + tid;
      ws.route_w[p] = r;
      pos[kk] = p;
    }
  }
#pragma unroll
  for (int pass = 0; pass < KM; ++pass)
#pragma unroll
    for (int i = pass & 1; i + 1 < KM; i += 2)
      if (pos[i] > pos[i + 1]) {
        const int t = pos[i];
        pos[i] = pos[i + 1];
        pos[i + 1] = t;
      }
  int* tp = s_tp + tid * K;
#pragma unroll
  for (int q = 0; q < KM; ++q)
    if (q < K) tp[q] = pos[q] == 0x7fffffff ? -1 : pos[q];
}

__device__ __forceinline__ void route_place(const int* s_ids, const float* s_r, int* s_tp, uint32_t* bits,
                                            const int* s_pos, int nb, int K, int b0, MoeWs ws) {
  const int tid = threadIdx.x;
  if (tid < nb)
    for (int kk = 0; kk < K; ++kk)
      if (is_route(s_r[tid * K + kk]))
        atomicOr(&bits[s_ids[tid * K + kk] * kChunkWords + (tid >> 5)], 1u << (tid & 31));
  __syncthreads();
  if (tid < nb && K <= 8) {
    route_place_regs<8>(s_ids, s_r, s_tp, bits, s_pos, K, b0, ws);
  } else if (tid < nb && K <= 16) {
    route_place_regs<16>(s_ids, s_r, s_tp, bits, s_pos, K, b0, ws);
  } else if (tid < nb) {
    route_place_regs<32>(s_ids, s_r, s_tp, bits, s_pos, K, b0, ws);
  }
  __syncthreads();
}

// Routing, pass 3 (one workgroup per chunk): a route's position is its
// expert's first position, plus its chunk's first position within the
// expert, plus the number of earlier tokens of the chunk routed to that expert
// (per-expert token bitmaps), so routes are grouped by expert with tokens
// ascending. Per token, its positions in ascending expert id feed the combine.
__global__ void __launch_bounds__(kChunk)
    moe_route_scatter_kernel(const int32_t* __restrict__ ids, int B, int K, int E, int nchunks, MoeWs ws,
                             const int* __restrict__ chunk_pos) {
  extern __shared__ int sm[];
  int* s_ids = sm;                                          // [kChunk * K]
  float* s_r = reinterpret_cast<float*>(sm + kChunk * K);   // [kChunk * K]
  int* s_tp = sm + 2 * kChunk * K;                          // [kChunk * K]
  uint32_t* bits = reinterpret_cast<uint32_t*>(sm + 3 * kChunk * K);  // [E][kChunkWords] token bitmaps
  int* s_pos = sm + 3 * kChunk * K + E * kChunkWords;       // [E]
  const int tid = threadIdx.x, b0 = blockIdx.x * kChunk;
  const int nb = B - b0 < kChunk ? B - b0 : kChunk;
  const int64_t e0 = (int64_t)b0 * K;
  for (int i = tid; i < E * kChunkWords; i += kChunk) bits[i] = 0u;
  // experts tid + kChunk * q: their first positions and this chunk's offsets
  // within them, loaded together with the chunk's entries (indexes past E
  // repeat expert E - 1; the loads past the first kChunk experts are skipped
  // for smaller layers)
  int pe[kExpertsPerLane];
#pragma unroll
  for (int q = 0; q < kExpertsPerLane; ++q) {
    pe[q] = 0;
    if (q == 0 || q * kChunk < E) {
      const int ec = tid + q * kChunk < E ? tid + q * kChunk : E - 1;
      pe[q] = chunk_pos[(int64_t)nchunks * E + ec] + chunk_pos[(int64_t)blockIdx.x * E + ec];
    }
  }
  stage_chunk2(s_ids, ids + e0, [](int v) { return v; }, s_r, ws.ent_r + e0, [](float v) { return v; }, nb * K);
#pragma unroll
  for (int q = 0; q < kExpertsPerLane; ++q)
    if (tid + q * kChunk < E) s_pos[tid + q * kChunk] = pe[q];
  __syncthreads();
  route_place(s_ids, s_r, s_tp, bits, s_pos, nb, K, b0, ws);
  for (int i = tid; i < nb * K; i += kChunk) ws.tok_pos[e0 + i] = s_tp[i];
}

// Routing, passes 2 and 3 in one launch for at most kFoldChunks chunks (one
// workgroup per chunk of max(kChunk, E rounded up to whole waves) lanes):
// every workgroup scans the chunks' counts itself (lane e = expert e: its
// expert's total and the routes of the earlier chunks, integer sums), chunk
// 0's workgroup writes the tables, and each places its chunk's routes as pass
// 3 does. The counts come from the count launch before it.
constexpr int kFoldChunks = 32;

__global__ void __launch_bounds__(kMaxExperts)
    moe_route_scan_scatter_kernel(const int32_t* __restrict__ ids, int B, int K, int E, int nchunks, int mtile,
                                  MoeWs ws, const int* __restrict__ chunk_cnt) {
  extern __shared__ int sm[];
  int* s_ids = sm;                                                     // [kChunk * K]
  float* s_r = reinterpret_cast<float*>(sm + kChunk * K);              // [kChunk * K]
  int* s_tp = sm + 2 * kChunk * K;                                     // [kChunk * K]
  uint32_t* bits = reinterpret_cast<uint32_t*>(sm + 3 * kChunk * K);   // [E][kChunkWords]
  int* s_pos = sm + 3 * kChunk * K + E * kChunkWords;                  // [E]
  __shared__ int s_wt[3][kMaxExperts / 64];
  const int tid = threadIdx.x, n = (int)blockDim.x, c = blockIdx.x, b0 = c * kChunk;
  const int nb = B - b0 < kChunk ? B - b0 : kChunk;
  const int64_t e0 = (int64_t)b0 * K;
  for (int i = tid; i < E * kChunkWords; i += n) bits[i] = 0u;
  // the expert's count in every chunk, loaded in one batch with the chunk's
  // entries (lanes past E read expert E - 1's and use none of it)
  int v[kFoldChunks];
  const int ec = tid < E ? tid : E - 1;
#pragma unroll
  for (int q = 0; q < kFoldChunks; ++q) v[q] = q < nchunks ? chunk_cnt[(int64_t)q * E + ec] : 0;
  if (tid < kChunk)
    stage_chunk2(s_ids, ids + e0, [](int x) { return x; }, s_r, ws.ent_r + e0, [](float x) { return x; }, nb * K);
  int total = 0, off = 0;
#pragma unroll
  for (int q = 0; q < kFoldChunks; ++q) {
    total += v[q];
    off += q < c ? v[q] : 0;
  }
  if (tid >= E) total = off = 0;
  const int base = route_scan(tid, E, total, mtile, ws, s_wt, c == 0);
  if (tid < E) s_pos[tid] = base + off;
  __syncthreads();
  route_place(s_ids, s_r, s_tp, bits, s_pos, nb, K, b0, ws);
  for (int i = tid; i < nb * K; i += n) ws.tok_pos[e0 + i] = s_tp[i];
}

// Routing of at most kChunk tokens in one launch: the three passes above in
// one workgroup of max(kChunk, E rounded up to whole waves) lanes, merge and
// placement with G lanes per token (so few tokens still spread over every
// wave), the chunk's counts and positions kept in LDS (its offsets within
// each expert are 0). Same outputs as the three launches.
__global__ void __launch_bounds__(kMaxExperts)
    moe_route_small_kernel(const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int B, int K, int E,
                           int mtile, MoeWs ws) {
  extern __shared__ int sm[];
  int* s_ids = sm;                                                     // [kChunk * K]
  float* s_w = reinterpret_cast<float*>(sm + kChunk * K);              // [kChunk * K] staged weights
  float* s_m = reinterpret_cast<float*>(sm + 2 * kChunk * K);          // [kChunk * K] merged weights
  uint32_t* bits = reinterpret_cast<uint32_t*>(sm + 3 * kChunk * K);   // [E][kChunkWords]
  int* s_pos = sm + 3 * kChunk * K + E * kChunkWords;                  // [E]
  int* cnt = s_pos + E;                                                // [E]
  __shared__ int s_wt[3][kMaxExperts / 64];
  const int tid = threadIdx.x, n = (int)blockDim.x, nent = B * K;
  for (int e = tid; e < E; e += n) cnt[e] = 0;
  for (int i = tid; i < E * kChunkWords; i += n) bits[i] = 0u;
  if (tid < kChunk)
    stage_chunk2(s_ids, ids, [](int v) { return v; }, s_w, wts, [](uint16_t v) { return bf16_to_float(v); }, nent);
  __syncthreads();
  // G lanes per token: doubled while below top_k and B * G stays within the
  // lanes; with one lane per token the token-parallel passes' functions
  int G = 1;
  while (G < K && B * G * 2 <= n) G <<= 1;
  if (G == 1) {
    route_merge(s_ids, s_w, cnt, B, K, E);
    __syncthreads();
    const int base = route_scan(tid, E, tid < E ? cnt[tid] : 0, mtile, ws, s_wt);
    if (tid < E) s_pos[tid] = base;
    __syncthreads();
    int* s_tp = reinterpret_cast<int*>(s_m);
    route_place(s_ids, s_w, s_tp, bits, s_pos, B, K, 0, ws);
    for (int i = tid; i < nent; i += n) ws.tok_pos[i] = s_tp[i];
    return;
  }
  const int b = tid / G, g = tid & (G - 1);
  if (b < B) {
    if (K <= 8)
      merge_grp<8>(s_ids, s_w, s_m, cnt, bits, b, g, G, K, E);
    else if (K <= 16)
      merge_grp<16>(s_ids, s_w, s_m, cnt, bits, b, g, G, K, E);
    else
      merge_grp<32>(s_ids, s_w, s_m, cnt, bits, b, g, G, K, E);
  }
  __syncthreads();
  const int base = route_scan(tid, E, tid < E ? cnt[tid] : 0, mtile, ws, s_wt);
  if (tid < E) s_pos[tid] = base;
  __syncthreads();
  if (b < B) {
    int* tp = ws.tok_pos + (int64_t)b * K;
    if (K <= 8)
      place_grp<8>(s_ids, s_m, bits, s_pos, b, g, G, K, b, tp, ws);
    else if (K <= 16)
      place_grp<16>(s_ids, s_m, bits, s_pos, b, g, G, K, b, tp, ws);
    else
      place_grp<32>(s_ids, s_m, bits, s_pos, b, g, G, K, b, tp, ws);
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped expert GEMMs: each workgroup owns one (expert slot, block of
// RPW 16-row groups); its KW waves split the K blocks, each wave decoding its
// units straight into MFMA operands; partial sums meet in LDS in wave order.
// Tokens of the expert are processed in chunks of 16*NT (one chunk at decode).
// ---------------------------------------------------------------------------

__device__ __forceinline__ u32x4 load_row8(const uint16_t* row, int col, int k) {
  if (col + 8 <= k) return *reinterpret_cast<const u32x4*>(row + col);
  u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t e = (col + i < k) ? (uint32_t)row[col + i] : 0u;
    v[i >> 1] |= e << (16 * (i & 1));
  }
  return v;
}

struct SlotInfo {
  int64_t expert;
  int t0, cnt;
};

__device__ __forceinline__ bool slot_info(const TokenSrc& src, int slot, SlotInfo& si) {
  if (src.dense) {
    if (slot != 0) return false;
    si.expert = 0;
    si.t0 = 0;
    si.cnt = src.tokens;
    return true;
  }
  if (slot >= src.hdr[0]) return false;
  si.expert = src.active[slot];
  si.t0 = src.act_off[slot];
  si.cnt = src.act_off[slot + 1] - si.t0;
  return true;
}

template <int FMT, int NT, int RPW>
__global__ void __launch_bounds__(512)
    moe_gate_up_kernel(Proj gate, Proj up, TokenSrc src, const uint16_t* __restrict__ x, int hidden,
                       uint16_t* __restrict__ act, int inter, int kw) {
  __shared__ float red[8][2][RPW][NT][256];
  SlotInfo si;
  if (!slot_info(src, blockIdx.x, si)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rg0 = blockIdx.y * RPW;
  for (int tc = 0; tc < si.cnt; tc += 16 * NT) {
    f32x4 ag[RPW][NT], au[RPW][NT];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) ag[r][t] = au[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t* xr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int q = tc + t * 16 + j;
      const int tok = q < si.cnt ? (src.dense ? q : src.route_tok[si.t0 + q]) : -1;
      xr[t] = tok >= 0 ? x + (int64_t)tok * hidden : nullptr;
    }
    if constexpr (NT == 1) {
      // Two K blocks per pass: all four units' loads are in flight together
      // (the second block is clamped to the first when it does not exist).
      static_assert(RPW == 1, "one row group per workgroup");
      const int rg = rg0;
      for (int kb0 = wave; kb0 < gate.kb && rg * 16 < inter; kb0 += 2 * kw) {
        const bool two = kb0 + kw < gate.kb;
        const int kbs[2] = {kb0, two ? kb0 + kw : kb0};
        Unit<FMT> ug[2], uu[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          ug[b].load(gate, si.expert, rg, kbs[b], lane);
          uu[b].load(up, si.expert, rg, kbs[b], lane);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          if (b == 1 && !two) break;
          u32x4 xf[8];
#pragma unroll
          for (int f = 0; f < 8; ++f)
            xf[f] = xr[0] ? load_row8(xr[0], kbs[b] * kQK + Unit<FMT>::xoff(f, jA), hidden) : u32x4{0u, 0u, 0u, 0u};
          u32x4 a[8];
          ug[b].decode(a, lane);
#pragma unroll
          for (int f = 0; f < 8; ++f) ag[0][0] = mfma16(a[f], xf[f], ag[0][0]);
          uu[b].decode(a, lane);
#pragma unroll
          for (int f = 0; f < 8; ++f) au[0][0] = mfma16(a[f], xf[f], au[0][0]);
        }
      }
    } else {
      for (int kb = wave; kb < gate.kb; kb += kw) {
        u32x4 xf[NT][8];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int f = 0; f < 8; ++f)
            xf[t][f] = xr[t] ? load_row8(xr[t], kb * kQK + Unit<FMT>::xoff(f, jA), hidden)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const int rg = rg0 + r;
          if (rg * 16 >= inter) break;
          Unit<FMT> ug, uu;
          ug.load(gate, si.expert, rg, kb, lane);
          uu.load(up, si.expert, rg, kb, lane);
          u32x4 a[8];
          ug.decode(a, lane);
#pragma unroll
          for (int f = 0; f < 8; ++f)
#pragma unroll
            for (int t = 0; t < NT; ++t) ag[r][t] = mfma16(a[f], xf[t][f], ag[r][t]);
          uu.decode(a, lane);
#pragma unroll
          for (int f = 0; f < 8; ++f)
#pragma unroll
            for (int t = 0; t < NT; ++t) au[r][t] = mfma16(a[f], xf[t][f], au[r][t]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          red[wave][0][r][t][lane * 4 + i] = ag[r][t][i];
          red[wave][1][r][t][lane * 4 + i] = au[r][t][i];
        }
    __syncthreads();
    for (int idx = threadIdx.x; idx < RPW * NT * 256; idx += blockDim.x) {
      const int r = idx / (NT * 256), t = (idx / 256) % NT, e = idx & 255;
      float g = 0.f, u = 0.f;
      for (int w = 0; w < kw; ++w) {
        g += red[w][0][r][t][e];
        u += red[w][1][r][t][e];
      }
      const int ln = e >> 2;
      const int row = (rg0 + r) * 16 + 4 * (ln >> 4) + (e & 3);
      const int q = tc + t * 16 + (ln & 15);
      if (row < inter && q < si.cnt) {
        g = bf16_round(g);
        u = bf16_round(u);
        const float sg = bf16_round(g * sigmoid_acc(g));
        act[(int64_t)(si.t0 + q) * inter + row] = bf16_bits(sg * u);
      }
    }
    __syncthreads();
  }
}

template <int FMT, int NT, int RPW>
__global__ void __launch_bounds__(512)
    moe_down_kernel(Proj down, TokenSrc src, const uint16_t* __restrict__ act, int inter,
                    uint16_t* __restrict__ y, int hidden, int kw) {
  __shared__ float red[8][RPW][NT][256];
  SlotInfo si;
  if (!slot_info(src, blockIdx.x, si)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int jA = lane >> 4, j = lane & 15;
  const int rg0 = blockIdx.y * RPW;
  for (int tc = 0; tc < si.cnt; tc += 16 * NT) {
    f32x4 acc[RPW][NT];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t* ar[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int q = tc + t * 16 + j;
      ar[t] = q < si.cnt ? act + (int64_t)(si.t0 + q) * inter : nullptr;
    }
    // All RPW units of a K block are loaded before the first is decoded (row
    // groups past the matrix are clamped to its last one and not used); with
    // four token groups, Q8_0, Q5_1 and Q5_K units are loaded one at a time (registers).
    // With one token group, two K blocks per pass, all their units in flight
    // together (the second block clamped to the first when it does not exist).
    constexpr int kPre = (FMT == FMT_Q8 || FMT == FMT_Q51 || FMT == FMT_Q5K) && NT > 1 ? 1 : RPW;
    constexpr int kBat = NT == 1 ? 2 : 1;
    for (int kb0 = wave; kb0 < down.kb; kb0 += kBat * kw) {
      Unit<FMT> udb[kBat][kPre];
#pragma unroll
      for (int bt = 0; bt < kBat; ++bt) {
        const int kbb = kb0 + bt * kw < down.kb ? kb0 + bt * kw : kb0;
#pragma unroll
        for (int r = 0; r < kPre; ++r) {
          const int rg = rg0 + r < (hidden + 15) / 16 ? rg0 + r : (hidden + 15) / 16 - 1;
          udb[bt][r].load(down, si.expert, rg, kbb, lane);
        }
      }
#pragma unroll
      for (int bt = 0; bt < kBat; ++bt) {
      if (bt > 0 && kb0 + bt * kw >= down.kb) break;
      const int kb = kb0 + bt * kw;
      Unit<FMT>(&ud)[kPre] = udb[bt];
      u32x4 xf[NT][8];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int f = 0; f < 8; ++f)
          xf[t][f] = ar[t] ? load_row8(ar[t], kb * kQK + Unit<FMT>::xoff(f, jA), inter)
                           : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        if ((rg0 + r) * 16 >= hidden) break;
        u32x4 a[8];
        if constexpr (kPre == RPW) {
          ud[r].decode(a, lane);
        } else {
          if (r > 0) ud[0].load(down, si.expert, rg0 + r, kb, lane);
          ud[0].decode(a, lane);
        }
#pragma unroll
        for (int f = 0; f < 8; ++f)
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[r][t] = mfma16(a[f], xf[t][f], acc[r][t]);
      }
      }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][r][t][lane * 4 + i] = acc[r][t][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < RPW * NT * 256; idx += blockDim.x) {
      const int r = idx / (NT * 256), t = (idx / 256) % NT, e = idx & 255;
      float s = 0.f;
      for (int w = 0; w < kw; ++w) s += red[w][r][t][e];
      const int ln = e >> 2;
      const int row = (rg0 + r) * 16 + 4 * (ln >> 4) + (e & 3);
      const int q = tc + t * 16 + (ln & 15);
      if (row < hidden && q < si.cnt) y[(int64_t)(si.t0 + q) * hidden + row] = bf16_bits(s);
    }
    __syncthreads();
  }
}

// out[b, h] = RNE(sum_i f32(y[pos_i, h]) * r_i) over the token's routes in
// ascending expert id; with a shared expert RNE(f32(routed) + f32(shared)).
__global__ void __launch_bounds__(256)
    moe_combine_kernel(const int* __restrict__ tok_pos, const float* __restrict__ route_w,
                       const uint16_t* __restrict__ y, int K, int hidden,
                       const uint16_t* __restrict__ sh_y, const uint16_t* __restrict__ sh_scale,
                       uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int h = (blockIdx.y * blockDim.x + threadIdx.x) * 8;
  if (h >= hidden) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < K; ++i) {
    const int pos = tok_pos[(int64_t)b * K + i];
    if (pos < 0) break;
    const float w = route_w[pos];
    const u32x4 v = *reinterpret_cast<const u32x4*>(y + (int64_t)pos * hidden + h);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += bf16_to_float((uint16_t)(v[q >> 1] >> (16 * (q & 1)))) * w;
  }
  u32x4 o;
  if (sh_y) {
    const u32x4 sv = *reinterpret_cast<const u32x4*>(sh_y + (int64_t)b * hidden + h);
    const float gs = sh_scale ? bf16_to_float(sh_scale[b]) : 1.f;
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float sy = bf16_to_float((uint16_t)(sv[q >> 1] >> (16 * (q & 1))));
      if (sh_scale) sy = bf16_round(sy * gs);
      v[q] = bf16_round(acc[q]) + sy;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  }
  *reinterpret_cast<u32x4*>(out + (int64_t)b * hidden + h) = o;
}

// Shared-expert gate (kaggle/qwen38_tpu/math.py:283 with linear and sigmoid of
// math.py:10-24): gate[b] = RNE(sigmoid(RNE(x[b] . w))), x BF16 [B, H], w BF16
// [H], FP32 accumulation. One wave per token; lane l sums the products of
// columns 8(l + 64i) .. +7 in column order, then the 64 lane sums meet in a
// fixed butterfly, so the result does not depend on scheduling.
__global__ void __launch_bounds__(64)
    moe_shared_gate_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int hidden,
                           uint16_t* __restrict__ gate) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const uint16_t* xr = x + (int64_t)b * hidden;
  float acc = 0.f;
  for (int h = 8 * lane; h < hidden; h += 512) {
    const u32x4 xv = *reinterpret_cast<const u32x4*>(xr + h);
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + h);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      acc += bf16_to_float((uint16_t)(xv[q >> 1] >> (16 * (q & 1)))) *
             bf16_to_float((uint16_t)(wv[q >> 1] >> (16 * (q & 1))));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane == 0) {
    const float g = bf16_round(acc);
    gate[b] = bf16_bits(sigmoid_acc(g));
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct WsLayout {
  size_t hdr, active, act_off, tile, ent_r, route_tok, route_w, tok_pos, act,
      y, sh_act, sh_y, sh_gate, xq, xq_s, aq, aq_s, slot_e, slot_t0, slot_cnt, tok_n, route_dst, contrib, chunk_cnt,
      flags, total;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace regions of one call. The routing result, the activations and the
// shared expert's buffers are common; the decode kernels' per-slot tables and
// token-major FP32 contributions, and the grouped kernels' route lists, tiles
// and BF16 expert outputs, are each needed by one path only, so a call reserves
// the regions of the path it takes (``decode``).
static WsLayout ws_layout(int64_t B, int64_t K, int64_t E, int64_t H, int64_t I, int64_t Is, int64_t mtile,
                          bool decode) {
  WsLayout L{};
  const int64_t n = B * K;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.hdr = take(64);
  L.route_w = take(4 * n);
  L.act = take(2 * n * I);
  L.sh_act = take(Is > 0 ? 2 * B * Is : 0);
  L.sh_y = take(Is > 0 ? 2 * B * H : 0);
  L.sh_gate = take(Is > 0 ? 2 * B : 0);
  if (decode) {
    L.slot_e = take(4 * E);
    L.slot_t0 = take(4 * E);
    L.slot_cnt = take(4 * E);
    L.tok_n = take(4 * B);
    L.route_dst = take(4 * n);
    L.contrib = take(4 * n * H);
    L.flags = take(8 * std::min(E, n) * cdiv(I, 16));  // the fused kernel's per-(slot, row group) tags
  } else {
    L.active = take(4 * E);
    L.act_off = take(4 * (E + 1));
    L.tile = take(sizeof(PfTile) * (E + n / mtile + 1));
    L.ent_r = take(4 * n);
    L.route_tok = take(4 * n);
    L.tok_pos = take(4 * n);
    L.y = take(2 * n * H);
    L.chunk_cnt = take(4 * (cdiv(B, kChunk) + 1) * E);
    // the int8_q8 policy's quantised x and SwiGLU activations (codes, FP32 scales)
    L.xq = take(B * H);
    L.xq_s = take(4 * B * (H / 32));
    L.aq = take(n * I);
    L.aq_s = take(4 * n * (I / 32));
  }
  L.total = o;
  return L;
}

constexpr int64_t kPrefillTile = 128;  // routes per prefill tile (moe_prefill.hip kM)

static Proj make_proj(const q6moe_table& t, int rows, int k) {
  Proj p;
  p.data = t.data;
  p.dstride = t.data_stride;
  p.rows = rows;
  p.k = k;
  p.kb = (int)cdiv(k, kQK);
  return p;
}

// Bytes of one expert's unit-major table.
static int64_t unit_table_bytes(int qtype, int64_t rows, int64_t k) {
  int unit = 0;
  switch (qtype) {
    case Q6MOE_Q6_K: unit = kQ6Unit; break;
    case Q6MOE_Q5_K: unit = kQ5KUnit; break;
    case Q6MOE_Q4_K: unit = kQ4Unit; break;
    case Q6MOE_Q8_0: unit = kQ8Unit; break;
    case Q6MOE_Q5_1: unit = kQ51Unit; break;
  }
  return cdiv(rows, 16) * cdiv(k, kQK) * unit;
}

static bool expert_qtype(int q) {
  return q == Q6MOE_Q6_K || q == Q6MOE_Q5_K || q == Q6MOE_Q4_K || q == Q6MOE_Q8_0 || q == Q6MOE_Q5_1;
}
static bool gate_up_qtype(int q) { return q == Q6MOE_Q6_K || q == Q6MOE_Q5_K || q == Q6MOE_Q4_K || q == Q6MOE_Q8_0; }
static bool block32_qtype(int q) { return q == Q6MOE_Q8_0 || q == Q6MOE_Q5_1; }  // 32-value blocks
static int fmt_of(int q) {
  switch (q) {
    case Q6MOE_Q6_K: return FMT_Q6;
    case Q6MOE_Q5_K: return FMT_Q5K;
    case Q6MOE_Q4_K: return FMT_Q4K;
    case Q6MOE_Q5_1: return FMT_Q51;
    default: return FMT_Q8;
  }
}

static int validate_table(const q6moe_table& t, const char* name, int64_t rows, int64_t k, int64_t experts) {
  std::string n(name);
  if (!t.data) {
    set_error(n + ": null data");
    return Q6MOE_ERR_INVALID;
  }
  if (!expert_qtype(t.qtype)) {
    set_error(n + ": qtype must be Q6_K, Q5_K, Q4_K, Q8_0 or Q5_1");
    return Q6MOE_ERR_UNSUPPORTED;
  }
  const int64_t need = unit_table_bytes(t.qtype, rows, k);
  if (!aligned(t.data, 16) || (experts > 1 && (t.data_stride % 16 || t.data_stride < need))) {
    set_error(n + ": expert tables must be 16-byte aligned unit-major tables (q6moe_moe_pack) "
                  "with a stride covering one expert");
    return Q6MOE_ERR_INVALID;
  }
  return Q6MOE_OK;
}

// FG: gate/up table format, FD: down table format.
template <int FG>
static void launch_gate_up(const Proj& g, const Proj& u, const TokenSrc& src, int grid_x, int max_tokens,
                           const uint16_t* x, int H, int I, uint16_t* act, hipStream_t s) {
  const int kw1 = g.kb < 8 ? g.kb : 8;
  const unsigned rb1 = (unsigned)cdiv(I, 16);
  if (max_tokens <= 16)
    hipLaunchKernelGGL((moe_gate_up_kernel<FG, 1, 1>), dim3(grid_x, rb1), dim3(64 * kw1), 0, s, g, u, src, x,
                       H, act, I, kw1);
  else
    hipLaunchKernelGGL((moe_gate_up_kernel<FG, 4, 1>), dim3(grid_x, rb1), dim3(64 * kw1), 0, s, g, u, src, x,
                       H, act, I, kw1);
}

template <int FD>
static void launch_down(const Proj& d, const TokenSrc& src, int grid_x, int max_tokens, const uint16_t* act,
                        int H, int I, uint16_t* y, hipStream_t s) {
  const int kw2 = d.kb < 8 ? d.kb : 8;
  if (max_tokens <= 16)  // one token group: one row group per workgroup (twice the workgroups)
    hipLaunchKernelGGL((moe_down_kernel<FD, 1, 1>), dim3(grid_x, (unsigned)cdiv(H, 16)), dim3(64 * kw2), 0, s, d,
                       src, act, I, y, H, kw2);
  else
    hipLaunchKernelGGL((moe_down_kernel<FD, 4, 2>), dim3(grid_x, (unsigned)cdiv(H, 16 * 2)), dim3(64 * kw2), 0, s,
                       d, src, act, I, y, H, kw2);
}

template <int FG, int FD, typename Mark>
static void launch_phases(const Proj& g, const Proj& u, const Proj& d, const TokenSrc& src, int grid_x,
                          int max_tokens, const uint16_t* x, int H, int I, uint16_t* act, uint16_t* y,
                          hipStream_t s, Mark mark) {
  launch_gate_up<FG>(g, u, src, grid_x, max_tokens, x, H, I, act, s);
  mark(2);
  launch_down<FD>(d, src, grid_x, max_tokens, act, H, I, y, s);
}

// ---------------------------------------------------------------------------
// W8A8 policy for Q8_0 tables: kaggle/qwen38_tpu/compute.py:20-34 (q8_matmul).
// The activations are quantised per row and 32-value group -- scale
// s = max|x| / 127 in FP32, codes clip(rint(x / (s ? s : 1)), -127, 127) --
// and each group's INT8 x INT8 dot products (INT32, exact) are scaled as
// (f32(partial) * s) * d_weight and summed over the groups in FP32; the sum is
// rounded to BF16.
// ---------------------------------------------------------------------------

// One thread per (row, group): 32 BF16 values -> 32 codes and the FP32 scale.
// ``row_count`` (device, may be NULL) bounds the rows that hold data.
__global__ void __launch_bounds__(256)
    moe_act_q8_kernel(const uint16_t* __restrict__ src, int64_t groups_total, int groups_per_row,
                      const int* __restrict__ row_count, int8_t* __restrict__ codes, float* __restrict__ scales) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= groups_total || (row_count && gid / groups_per_row >= *row_count)) return;
  const u32x4* p = reinterpret_cast<const u32x4*>(src + gid * 32);  // rows are whole groups
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = p[i];
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(bf16_to_float((uint16_t)(v[i >> 3][(i >> 1) & 3] >> (16 * (i & 1))))));
  const float sc = m / 127.f;
  const float div = sc == 0.f ? 1.f : sc;
  uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float x = bf16_to_float((uint16_t)(v[i >> 3][(i >> 1) & 3] >> (16 * (i & 1))));
    const float q = fminf(fmaxf(__builtin_rintf(x / div), -127.f), 127.f);
    w[i >> 2] |= ((uint32_t)(int32_t)q & 0xffu) << (8 * (i & 3));
  }
  u32x4* o = reinterpret_cast<u32x4*>(codes + gid * 32);
  o[0] = u32x4{w[0], w[1], w[2], w[3]};
  o[1] = u32x4{w[4], w[5], w[6], w[7]};
  scales[gid] = sc;
}

// Quantised activations: codes [rows, k] and scales [rows, k / 32].
struct W8Src {
  const int8_t* codes;
  const float* scales;
  int k;
};

__device__ __forceinline__ i32x4 mfma_i8(uint64_t a, uint64_t b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, c, 0, 0, 0);
}

// W8A8 projection(s) of a slot's tokens over Q8_0 unit-major tables, on the
// INT8 matrix cores (v_mfma_i32_16x16x32_i8: one MFMA per 32-value group).
// PAIR: gate p0 and up p1 with the SwiGLU epilogue a = RNE(RNE(g*sig(g)) * u)
// into out [routes, rows]; otherwise one projection y = RNE(acc) into
// out [routes or tokens, rows]. Activation row of token q of the slot: q
// (dense), the route's token (routed gate/up) or the route position (routed
// down, ``route_rows``). The waves of a workgroup split the K blocks; their
// partial sums meet in LDS and are added in wave order.
// Lane (column j = lane % 16, k-group kq = lane / 16) feeds codes 8kq..8kq+7 of
// each group: in a Q8_0 unit those of row j, block 2g + h sit at
// 1024g + 16(16(2h + kq/2) + j) + 8(kq % 2) (moe_common.h).
template <bool PAIR>
__global__ void __launch_bounds__(512)
    moe_w8_kernel(Proj p0, Proj p1, TokenSrc src, int route_rows, W8Src a, uint16_t* __restrict__ out, int kw) {
  __shared__ float red[8][2][256];
  SlotInfo si;
  if (!slot_info(src, blockIdx.x, si)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kq = lane >> 4, j = lane & 15;
  const int rg = blockIdx.y;
  const int rows = p0.rows, groups = a.k / 32;
  constexpr int NU = PAIR ? 2 : 1;
  for (int tc = 0; tc < si.cnt; tc += 16) {
    const int q = tc + j;
    int64_t arow = -1;
    if (q < si.cnt) arow = src.dense ? q : (route_rows ? si.t0 + q : src.route_tok[si.t0 + q]);
    f32x4 acc[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb = wave; kb < p0.kb; kb += kw) {
      const int ng = groups - 8 * kb < 8 ? groups - 8 * kb : 8;  // groups of this K block
      uint64_t b[8];
      float sa[8];
#pragma unroll
      for (int G = 0; G < 8; ++G) {
        const bool ok = arow >= 0 && G < ng;
        b[G] = ok ? *reinterpret_cast<const uint64_t*>(a.codes + arow * a.k + kb * kQK + 32 * G + 8 * kq) : 0ull;
        sa[G] = ok ? a.scales[arow * groups + 8 * kb + G] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const Proj& p = u ? p1 : p0;
        const uint8_t* un = unit_ptr<FMT_Q8>(p, si.expert, rg, kb);
        u32x4 sw[4];  // block scales of rows 4kq + i: half 4h + g of the row's 16-byte line
#pragma unroll
        for (int i = 0; i < 4; ++i) sw[i] = *reinterpret_cast<const u32x4*>(un + 4096 + 16 * (4 * kq + i));
#pragma unroll
        for (int G = 0; G < 8; ++G) {
          if (G >= ng) break;
          const int g = G >> 1, h = G & 1;
          const uint64_t w = *reinterpret_cast<const uint64_t*>(
              un + 1024 * g + 16 * (16 * (2 * h + (kq >> 1)) + j) + 8 * (kq & 1));
          const i32x4 pr = mfma_i8(w, b[G], i32x4{0, 0, 0, 0});
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t word = sw[i][h * 2 + (g >> 1)];
            const float dw = half_bits_to_float((word >> (16 * (g & 1))) & 0xffffu);
            acc[u][i] += ((float)pr[i] * sa[G]) * dw;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][u][lane * 4 + i] = acc[u][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
      float v[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        v[u] = 0.f;
        for (int w = 0; w < kw; ++w) v[u] += red[w][u][idx];
      }
      const int ln = idx >> 2;
      const int row = rg * 16 + 4 * (ln >> 4) + (idx & 3);
      const int qq = tc + (ln & 15);
      if (row < rows && qq < si.cnt) {
        const int64_t orow = src.dense ? qq : si.t0 + qq;
        if (PAIR) {
          const float g = bf16_round(v[0]), uu = bf16_round(v[NU - 1]);
          out[orow * rows + row] = bf16_bits(bf16_round(g * sigmoid_acc(g)) * uu);
        } else {
          out[orow * rows + row] = bf16_bits(v[0]);
        }
      }
    }
    __syncthreads();
  }
}

static void launch_act_q8(const uint16_t* src, int64_t rows, int k, const int* row_count, int8_t* codes,
                          float* scales, hipStream_t s) {
  const int64_t groups = rows * (k / 32);
  hipLaunchKernelGGL(moe_act_q8_kernel, dim3((unsigned)cdiv(groups, 256)), dim3(256), 0, s, src, groups, k / 32,
                     row_count, codes, scales);
}

static void launch_w8(bool pair, const Proj& p0, const Proj& p1, const TokenSrc& src, int grid_x, int route_rows,
                      const W8Src& a, uint16_t* out, hipStream_t s) {
  const int kw = p0.kb < 8 ? p0.kb : 8;
  const dim3 grid((unsigned)grid_x, (unsigned)cdiv(p0.rows, 16));
  if (pair)
    hipLaunchKernelGGL(moe_w8_kernel<true>, grid, dim3(64 * kw), 0, s, p0, p1, src, route_rows, a, out, kw);
  else
    hipLaunchKernelGGL(moe_w8_kernel<false>, grid, dim3(64 * kw), 0, s, p0, p1, src, route_rows, a, out, kw);
}

// GGUF expert tables [experts][rows][K blocks][block bytes] -> unit-major
// tables (layout in moe_common.h), expert blockIdx.y per grid row.
// Six-bit code of position p (0..255) of a GGUF Q6_K block
// (kaggle/glm53_offload/gguf_quant.py:159-167): low nibble from ql, high two
// bits from qh.
__device__ __forceinline__ uint32_t q6_code_at(const uint8_t* blk, int p) {
  const int n = p >> 7, q = (p >> 5) & 3, l = p & 31;
  const uint32_t ql = blk[64 * n + l + 32 * (q & 1)];
  const uint32_t qh = blk[128 + 32 * n + l];
  return ((q >= 2 ? ql >> 4 : ql) & 15u) | (((qh >> (2 * q)) & 3u) << 4);
}

// One 4-byte word of a unit-major table per thread. Q6_K units are
// bit-planar (see q6p_decode): code word g of chunk c of lane l (row l % 16,
// sub-block 4g + l / 16) at 1024c + 16l + 4g, the lane's four sub-scales at
// 3072 + 4l, the rows' FP16 scales at 3328. Q4_K (Q5_K) units are the rows'
// 144-byte (176-byte) blocks in 16-byte chunks (chunk c of row j at
// 16 * (16c + j)). Q8_0 units hold lane l's 16 codes of chunk g at 1024g + 16l
// and the rows' 8 block scales at 4096. Q5_1 units hold the 16 nibble bytes of
// row j's block 2g + h at 512g + 256h + 16j, then its high word, d and m at
// 2048 + 64j + 32h + 8g. Rows (and Q8_0 / Q5_1 blocks) past the projection's
// are zero. rblocks: GGUF blocks per row in raw (K/256 for the K-quants, K/32
// for Q8_0 and Q5_1).
template <int FMT>
__global__ void __launch_bounds__(256) moe_pack_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride, int rows,
                                                       int kbs, int rblocks, uint8_t* __restrict__ dst,
                                                       int64_t dst_stride, int64_t words) {
  constexpr int U = UnitBytes<FMT>::value;
  constexpr int BS = FMT == FMT_Q6 ? 210 : FMT == FMT_Q4K ? 144 : FMT == FMT_Q5K ? 176 : FMT == FMT_Q51 ? 24 : 34;
  const int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (wi >= words) return;
  const int64_t e = blockIdx.y, o = wi * 4;
  const int64_t unit = o / U;
  const int ob = (int)(o - unit * U);
  const int rg = (int)(unit / kbs), kb = (int)(unit - (int64_t)rg * kbs);
  auto block = [&](int row) { return raw + e * raw_stride + ((int64_t)(rg * 16 + row) * rblocks + kb) * BS; };
  uint32_t v = 0;
  if (FMT == FMT_Q51) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int b = ob + t;
      int j, blk, src;  // row in the group, Q5_1 block in the row, byte in the block
      if (b < 2048) {
        j = (b >> 4) & 15;
        blk = 8 * kb + 2 * (b >> 9) + ((b >> 8) & 1);
        src = 8 + (b & 15);
      } else {
        const int a = b - 2048, k = a & 7;
        j = a >> 6;
        blk = 8 * kb + 2 * ((a >> 3) & 3) + ((a >> 5) & 1);
        src = k < 4 ? 4 + k : k - 4;  // high word, then d, then m
      }
      const int row = rg * 16 + j;
      const uint32_t byte =
          row < rows && blk < rblocks ? raw[e * raw_stride + ((int64_t)row * rblocks + blk) * BS + src] : 0u;
      v |= byte << (8 * t);
    }
  } else if (FMT == FMT_Q8) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int b = ob + t;
      int j, blk, src;  // row in the group, Q8_0 block in the row, byte in the block
      if (b < 4096) {
        const int g = b >> 10, l = (b >> 4) & 63;
        j = l & 15;
        blk = 8 * kb + 2 * g + (l >> 5);
        src = 2 + 16 * ((l >> 4) & 1) + (b & 15);
      } else {
        const int idx = (b - 4096) >> 1;
        j = idx >> 3;
        blk = 8 * kb + 2 * (idx & 3) + ((idx >> 2) & 1);
        src = b & 1;
      }
      const int row = rg * 16 + j;
      const uint32_t byte =
          row < rows && blk < rblocks ? raw[e * raw_stride + ((int64_t)row * rblocks + blk) * BS + src] : 0u;
      v |= byte << (8 * t);
    }
  } else if (FMT == FMT_Q6 && ob < 3072) {
    const int c = ob >> 10, l = (ob >> 4) & 63, g = (ob >> 2) & 3;
    const int j = l & 15, jA = l >> 4;
    if (rg * 16 + j < rows) {
      const uint8_t* blk = block(j);
      const int p0 = 64 * g + 16 * jA;  // the sub-block; pair k holds positions p0 + 2k, p0 + 2k + 1
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = 0; t < 2; ++t) v |= q6_code_at(blk, p0 + 2 * (2 * c + t) + h) << (4 + 6 * t + 16 * h);
        if (c < 2) {
          v |= (q6_code_at(blk, p0 + 2 * (6 + c) + h) & 15u) << (16 * h);
        } else {
#pragma unroll
          for (int t = 0; t < 2; ++t) v |= (q6_code_at(blk, p0 + 2 * (6 + t) + h) >> 4) << (2 * t + 16 * h);
        }
      }
    }
  } else if (FMT == FMT_Q6 && ob < 3328) {
    const int l = (ob - 3072) >> 2, j = l & 15, jA = l >> 4;
    if (rg * 16 + j < rows) {
      const uint8_t* blk = block(j);
#pragma unroll
      for (int g = 0; g < 4; ++g) v |= (uint32_t)blk[192 + 4 * g + jA] << (8 * g);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int b = ob + t;
      int row, src;  // row within the group, byte within that row's block
      if (FMT == FMT_Q6) {
        row = (b - 3328) >> 1;
        src = 208 + (b & 1);
      } else {
        row = (b >> 4) & 15;
        src = 16 * (b >> 8) + (b & 15);
      }
      const uint32_t byte = rg * 16 + row < rows ? block(row)[src] : 0u;
      v |= byte << (8 * t);
    }
  }
  *reinterpret_cast<uint32_t*>(dst + e * dst_stride + o) = v;
}

// Unit-decode probe of the generic kernels' register path (Unit::load +
// Unit::decode). grid (units per expert, experts).
template <int FMT>
__global__ void __launch_bounds__(64) moe_unit_unpack_kernel(Proj p, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x;
  const int e = blockIdx.y, rg = blockIdx.x / p.kb, kb = blockIdx.x - rg * p.kb;
  Unit<FMT> u;
  u.load(p, e, rg, kb, lane);
  u32x4 a[8];
  u.decode(a, lane);
  store_unit_frags(a, out + (int64_t)e * p.rows * p.k, p, rg, kb, lane,
                   [](int f, int jA) { return Unit<FMT>::xoff(f, jA); });
}

}  // namespace q6moe

using namespace q6moe;

extern "C" size_t q6moe_moe_table_bytes(int qtype, int64_t rows, int64_t width) {
  if (!expert_qtype(qtype) || rows < 1 || width < 1 || rows > (1 << 24) || width > (1 << 24) ||
      (block32_qtype(qtype) && width % 32))
    return 0;
  return (size_t)unit_table_bytes(qtype, rows, width);
}

extern "C" int q6moe_moe_pack(const uint8_t* raw, int qtype, int64_t experts, int64_t rows, int64_t width,
                              uint8_t* dst, void* stream) {
  Q6MOE_REQUIRE(raw && dst, "moe_pack: null pointer");
  Q6MOE_REQUIRE(expert_qtype(qtype), "moe_pack: qtype must be Q6_K, Q5_K, Q4_K, Q8_0 or Q5_1");
  Q6MOE_REQUIRE(!block32_qtype(qtype) || width % 32 == 0,
                "moe_pack: Q8_0 and Q5_1 rows must hold whole 32-value blocks");
  Q6MOE_REQUIRE(experts >= 1 && experts <= 65535 && rows >= 1 && width >= 1 && rows <= (1 << 24) &&
                    width <= (1 << 24),
                "moe_pack: bad shape");
  Q6MOE_REQUIRE(aligned(dst, 16), "moe_pack: dst must be 16-byte aligned");
  const int kbs = (int)cdiv(width, kQK);
  const int64_t bytes = unit_table_bytes(qtype, rows, width);
  const int64_t words = bytes / 4;
  const dim3 grid((unsigned)cdiv(words, 256), (unsigned)experts);
  if (qtype == Q6MOE_Q6_K)
    hipLaunchKernelGGL(moe_pack_kernel<FMT_Q6>, grid, dim3(256), 0, (hipStream_t)stream, raw, rows * kbs * 210,
                       (int)rows, kbs, kbs, dst, bytes, words);
  else if (qtype == Q6MOE_Q4_K)
    hipLaunchKernelGGL(moe_pack_kernel<FMT_Q4K>, grid, dim3(256), 0, (hipStream_t)stream, raw, rows * kbs * 144,
                       (int)rows, kbs, kbs, dst, bytes, words);
  else if (qtype == Q6MOE_Q5_K)
    hipLaunchKernelGGL(moe_pack_kernel<FMT_Q5K>, grid, dim3(256), 0, (hipStream_t)stream, raw, rows * kbs * 176,
                       (int)rows, kbs, kbs, dst, bytes, words);
  else if (qtype == Q6MOE_Q5_1)
    hipLaunchKernelGGL(moe_pack_kernel<FMT_Q51>, grid, dim3(256), 0, (hipStream_t)stream, raw,
                       rows * (width / 32) * 24, (int)rows, kbs, (int)(width / 32), dst, bytes, words);
  else
    hipLaunchKernelGGL(moe_pack_kernel<FMT_Q8>, grid, dim3(256), 0, (hipStream_t)stream, raw,
                       rows * (width / 32) * 34, (int)rows, kbs, (int)(width / 32), dst, bytes, words);
  return check_launch("moe_pack_kernel");
}

// e[i] = exp(-|x[i]|) and s[i] = sigmoid_acc(x[i]) for BF16 x: the values the
// SwiGLU epilogues and the shared-expert gate compute.
__global__ void __launch_bounds__(256) sigmoid_probe_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                            float* __restrict__ e, float* __restrict__ s) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = bf16_to_float(x[i]);
  e[i] = expf(-fabsf(v));
  s[i] = sigmoid_acc(v);
}

extern "C" int q6moe_sigmoid_probe(const uint16_t* x, int64_t n, float* e, float* s, void* stream) {
  Q6MOE_REQUIRE(x && e && s, "sigmoid_probe: null pointer");
  Q6MOE_REQUIRE(n >= 1 && n <= (int64_t)1 << 30, "sigmoid_probe: n must be in [1, 2^30]");
  Q6MOE_REQUIRE(aligned(x, 2) && aligned(e, 4) && aligned(s, 4), "sigmoid_probe: misaligned pointer");
  hipLaunchKernelGGL(sigmoid_probe_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, x, n,
                     e, s);
  return check_launch("sigmoid_probe_kernel");
}

extern "C" int q6moe_moe_unpack(const uint8_t* table, int qtype, int64_t experts, int64_t rows, int64_t width,
                                int64_t stride, int path, uint16_t* out, void* stream) {
  Q6MOE_REQUIRE(table && out, "moe_unpack: null pointer");
  Q6MOE_REQUIRE(expert_qtype(qtype), "moe_unpack: qtype must be Q6_K, Q5_K, Q4_K, Q8_0 or Q5_1");
  Q6MOE_REQUIRE(experts >= 1 && experts <= 65535 && rows >= 1 && width >= 1 && rows <= (1 << 24) &&
                    width <= (1 << 24) && (!block32_qtype(qtype) || width % 32 == 0),
                "moe_unpack: bad shape");
  Q6MOE_REQUIRE(path >= 0 && path <= 2, "moe_unpack: path must be 0 (generic), 1 (decode) or 2 (prefill)");
  Q6MOE_REQUIRE(path != 2 || pf_unpack_supported(fmt_of(qtype)),
                "moe_unpack: the prefill path decodes Q6_K, Q8_0, Q5_1 and Q4_K");
  const int64_t need = unit_table_bytes(qtype, rows, width);
  Q6MOE_REQUIRE(aligned(table, 16) && (experts == 1 || (stride >= need && stride % 16 == 0)),
                "moe_unpack: table must be 16-byte aligned with a stride covering one expert");
  const int64_t units = cdiv(rows, 16) * cdiv(width, kQK);
  Q6MOE_REQUIRE(units <= 0x7fffffff, "moe_unpack: too many units");
  q6moe_table t{qtype, table, experts == 1 ? need : stride, nullptr, 0};
  const Proj p = make_proj(t, (int)rows, (int)width);
  hipStream_t s = (hipStream_t)stream;
  const int fmt = fmt_of(qtype);
  const dim3 grid((unsigned)units, (unsigned)experts);
  if (path == 1) {
    launch_dec_unpack(fmt, p, (int)experts, out, s);
  } else if (path == 2) {
    launch_pf_unpack(fmt, p, (int)experts, out, s);
  } else if (fmt == FMT_Q6) {
    hipLaunchKernelGGL(moe_unit_unpack_kernel<FMT_Q6>, grid, dim3(64), 0, s, p, out);
  } else if (fmt == FMT_Q4K) {
    hipLaunchKernelGGL(moe_unit_unpack_kernel<FMT_Q4K>, grid, dim3(64), 0, s, p, out);
  } else if (fmt == FMT_Q5K) {
    hipLaunchKernelGGL(moe_unit_unpack_kernel<FMT_Q5K>, grid, dim3(64), 0, s, p, out);
  } else if (fmt == FMT_Q51) {
    hipLaunchKernelGGL(moe_unit_unpack_kernel<FMT_Q51>, grid, dim3(64), 0, s, p, out);
  } else {
    hipLaunchKernelGGL(moe_unit_unpack_kernel<FMT_Q8>, grid, dim3(64), 0, s, p, out);
  }
  return check_launch("moe_unpack");
}

extern "C" size_t q6moe_moe_workspace_size(int64_t tokens, int64_t top_k, int64_t experts, int64_t hidden,
                                           int64_t intermediate, int64_t shared_intermediate) {
  if (tokens < 1 || top_k < 1 || experts < 1 || hidden < 1 || intermediate < 1 || shared_intermediate < 0)
    return 0;
  const size_t pf = ws_layout(tokens, top_k, experts, hidden, intermediate, shared_intermediate, kPrefillTile,
                              false).total;
  const int64_t width = std::max(hidden, std::max(intermediate, shared_intermediate));
  if (!dec_supported(tokens, top_k, experts, width)) return pf;
  const size_t dec = ws_layout(tokens, top_k, experts, hidden, intermediate, shared_intermediate, kPrefillTile,
                               true).total;
  return pf > dec ? pf : dec;
}

// Scratch of q6moe_moe_forward_noalloc: the workspace regions of one call
// (routing tables, activations, expert outputs or contributions, shared-expert
// buffers) for callers that cannot allocate device memory. Each GPU holds its
// own copy for the life of the process. Host code uses the per-device address
// from hipGetSymbolAddress, never the array's name. Every call on a GPU shares
// that GPU's copy: calls that overlap on one GPU (other streams, other host
// threads) race. No region needs to start zeroed (each is written before it
// is read in a call), so nothing is cleared between calls.
constexpr size_t kStaticScratchBytes = Q6MOE_NOALLOC_SCRATCH_BYTES;
static_assert(kStaticScratchBytes == size_t(32) << 20, "32 MiB of static scratch per device");
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[kMaxScratchDevices];

// The current device's address of ``scratch``, looked up once per device with
// that device current.
static int static_scratch(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error(std::string("moe_forward_noalloc: hipGetDevice: ") + hipGetErrorString(err));
    return Q6MOE_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("moe_forward_noalloc: device index out of range");
    return Q6MOE_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      set_error(std::string("moe_forward_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
      return Q6MOE_ERR_HIP;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return Q6MOE_OK;
}

// The routed FFN on a given workspace (the caller's, or the static scratch).
static int moe_forward_impl(const q6moe_moe_args* a, void* workspace, size_t workspace_bytes, void* stream,
                            bool static_ws = false) {
  Q6MOE_REQUIRE(a->x && a->ids && a->weights && a->out && workspace, "moe_forward: null pointer");
  const int64_t B = a->tokens, K = a->top_k, E = a->experts, H = a->hidden, I = a->intermediate;
  Q6MOE_REQUIRE(B >= 1 && K >= 1 && E >= 1 && H >= 1 && I >= 1, "moe_forward: sizes must be positive");
  Q6MOE_REQUIRE(E <= kMaxExperts, "moe_forward: at most 1024 experts per call");
  Q6MOE_REQUIRE(K <= 32, "moe_forward: top_k must be at most 32");
  Q6MOE_REQUIRE(B * K <= (1 << 28) && H <= (1 << 24) && I <= (1 << 24), "moe_forward: problem too large");
  Q6MOE_REQUIRE(H % 8 == 0 && I % 8 == 0, "moe_forward: hidden and intermediate must be multiples of 8");
  Q6MOE_REQUIRE(aligned(a->x, 16) && aligned(a->out, 16) && aligned(workspace, 256),
                "moe_forward: x/out need 16-byte and workspace 256-byte alignment");
  Q6MOE_REQUIRE(a->gate.qtype == a->up.qtype && gate_up_qtype(a->gate.qtype) && expert_qtype(a->down.qtype),
                "moe_forward: gate and up must share Q6_K, Q5_K, Q4_K or Q8_0; down must be one of those or Q5_1");
  Q6MOE_REQUIRE(a->mode >= 0 && a->mode <= 2, "moe_forward: mode must be 0, 1 or 2");
  int rc;
  if ((rc = validate_table(a->gate, "gate", I, H, E)) || (rc = validate_table(a->up, "up", I, H, E)) ||
      (rc = validate_table(a->down, "down", H, I, E)))
    return rc;
  const int64_t Is = a->shared_gate.data ? a->shared_intermediate : 0;
  if (Is) {
    Q6MOE_REQUIRE(Is >= 1 && Is % 8 == 0 && Is <= (1 << 24), "moe_forward: shared_intermediate");
    Q6MOE_REQUIRE(a->shared_gate.qtype == a->gate.qtype && a->shared_up.qtype == a->gate.qtype &&
                      a->shared_down.qtype == a->down.qtype,
                  "moe_forward: the shared expert must use the routed experts' qtype");
    Q6MOE_REQUIRE(!(a->shared_router && a->shared_scale), "moe_forward: shared_router and shared_scale exclude each other");
    Q6MOE_REQUIRE(!a->shared_router || aligned(a->shared_router, 16), "moe_forward: shared_router needs 16-byte alignment");
    if ((rc = validate_table(a->shared_gate, "shared_gate", Is, H, 1)) ||
        (rc = validate_table(a->shared_up, "shared_up", Is, H, 1)) ||
        (rc = validate_table(a->shared_down, "shared_down", H, Is, 1)))
      return rc;
  }
  Q6MOE_REQUIRE(a->compute == 0 || a->compute == 1, "moe_forward: compute must be 0 (bf16) or 1 (int8_q8)");
  const bool w8 = a->compute == 1;
  Q6MOE_REQUIRE(!(w8 && a->mode == 1), "moe_forward: the int8_q8 policy runs on the grouped kernels (mode 0 or 2)");
  const int64_t width = std::max(H, std::max(I, Is));
  if (a->mode == 1 && !dec_supported(B, K, E, width)) {
    set_error("moe_forward: decode mode needs tokens <= 256, tokens*top_k <= 1024, experts <= 1024 and "
              "tokens*top_k*max(hidden, intermediate, shared_intermediate) < 2^30");
    return Q6MOE_ERR_INVALID;
  }
  // Mode 0: the decode-step kernels up to 64 tokens, unless the routing is
  // large (tokens x top-k x experts >= 2^17) and no shared expert rides along:
  // every decode-step wave repeats the routing over all entries and experts,
  // and there the grouped kernels (routing once) are faster. Measured on the
  // 512-expert top-10 layer: 16 tokens decode 141 us against grouped 158,
  // 32 tokens 245 against 230, 64 tokens 432 against 345; the 128-expert
  // top-8 layer at 64 tokens 125 against 124.
  const bool dec_auto = B <= 64 && (Is > 0 || B * K * E < (int64_t(1) << 17));
  const bool decode = !w8 && dec_supported(B, K, E, width) && (a->mode == 1 || (a->mode == 0 && dec_auto));
  const WsLayout L = ws_layout(B, K, E, H, I, Is, kPrefillTile, decode);
  if (workspace_bytes < L.total) {
    if (static_ws)
      set_error("moe_forward_noalloc: this call needs " + std::to_string(L.total) +
                " bytes of scratch; the static scratch holds " + std::to_string(kStaticScratchBytes) +
                " (use q6moe_moe_forward with a workspace)");
    else
      set_error("moe_forward: workspace too small (need " + std::to_string(L.total) + " bytes)");
    return Q6MOE_ERR_INVALID;
  }
  uint8_t* w = reinterpret_cast<uint8_t*>(workspace);
  MoeWs ws;
  ws.hdr = reinterpret_cast<int*>(w + L.hdr);
  ws.route_w = reinterpret_cast<float*>(w + L.route_w);
  ws.act = reinterpret_cast<uint16_t*>(w + L.act);
  ws.active = ws.act_off = ws.route_tok = ws.tok_pos = nullptr;
  ws.tile = nullptr;
  ws.ent_r = nullptr;
  ws.y = nullptr;
  if (!decode) {  // regions of the grouped path only
    ws.active = reinterpret_cast<int*>(w + L.active);
    ws.act_off = reinterpret_cast<int*>(w + L.act_off);
    ws.tile = reinterpret_cast<PfTile*>(w + L.tile);
    ws.ent_r = reinterpret_cast<float*>(w + L.ent_r);
    ws.route_tok = reinterpret_cast<int*>(w + L.route_tok);
    ws.tok_pos = reinterpret_cast<int*>(w + L.tok_pos);
    ws.y = reinterpret_cast<uint16_t*>(w + L.y);
  }
  ws.sh_act = Is ? reinterpret_cast<uint16_t*>(w + L.sh_act) : nullptr;
  ws.sh_y = Is ? reinterpret_cast<uint16_t*>(w + L.sh_y) : nullptr;

  hipStream_t s = (hipStream_t)stream;
  // Per-token shared-expert gate: the caller's, or computed here from the router.
  const uint16_t* sh_scale = a->shared_scale;
  if (Is && a->shared_router) {
    uint16_t* g = reinterpret_cast<uint16_t*>(w + L.sh_gate);
    hipLaunchKernelGGL(moe_shared_gate_kernel, dim3((unsigned)B), dim3(64), 0, s, a->x, a->shared_router, (int)H, g);
    if ((rc = check_launch("moe_shared_gate_kernel"))) return rc;
    sh_scale = g;
  }
  auto mark = [&](int i) {
    if (a->events && a->events[i]) (void)hipEventRecord((hipEvent_t)a->events[i], s);
  };
  const int fmt = fmt_of(a->gate.qtype), fmt_dn = fmt_of(a->down.qtype);
  // Generic (non-tiled) expert phases for the call's formats.
  auto phases = [&](const Proj& pg, const Proj& pu, const Proj& pd, const TokenSrc& src, int grid_x, int max_tok,
                    int inter, uint16_t* act_out, uint16_t* y_out, auto mk) {
    dispatch_formats(fmt, fmt_dn, [&](auto fg, auto fd) {
      launch_phases<decltype(fg)::value, decltype(fd)::value>(pg, pu, pd, src, grid_x, max_tok, a->x, (int)H, inter,
                                                              act_out, y_out, s, mk);
    });
  };
  if (decode) {
    mark(0);
    // up to kDecSharedTokens tokens the shared expert runs inside the decode launches
    const bool fused_shared = Is && B <= kDecSharedTokens;
    if (Is && !fused_shared) {
      TokenSrc dense{1, (int)B, nullptr, nullptr, nullptr, nullptr};
      const Proj sg = make_proj(a->shared_gate, (int)Is, (int)H), su = make_proj(a->shared_up, (int)Is, (int)H),
                 sd = make_proj(a->shared_down, (int)H, (int)Is);
      phases(sg, su, sd, dense, 1, (int)B, (int)Is, ws.sh_act, ws.sh_y, [](int) {});
      if ((rc = check_launch("moe shared expert kernels"))) return rc;
    }
    DecArgs D;
    D.gate = make_proj(a->gate, (int)I, (int)H);
    D.up = make_proj(a->up, (int)I, (int)H);
    D.down = make_proj(a->down, (int)H, (int)I);
    D.R = DecRoute{a->ids, a->weights, (int)B, (int)K, (int)E};
    D.T.hdr = ws.hdr;
    D.T.slot_e = reinterpret_cast<int*>(w + L.slot_e);
    D.T.slot_t0 = reinterpret_cast<int*>(w + L.slot_t0);
    D.T.slot_cnt = reinterpret_cast<int*>(w + L.slot_cnt);
    D.T.tok_n = reinterpret_cast<int*>(w + L.tok_n);
    D.T.route_w = ws.route_w;
    D.T.route_dst = reinterpret_cast<int*>(w + L.route_dst);
    D.x = a->x;
    D.H = (int)H;
    D.I = (int)I;
    D.max_slots = (int)(E < B * K ? E : B * K);
    D.act = ws.act;
    D.contrib = reinterpret_cast<float*>(w + L.contrib);
    D.flags = reinterpret_cast<uint64_t*>(w + L.flags);
    D.sh_y = ws.sh_y;
    D.sh_scale = sh_scale;
    D.out = a->out;
    D.S = DecShared{};
    if (fused_shared) {
      D.S.gate = make_proj(a->shared_gate, (int)Is, (int)H);
      D.S.up = make_proj(a->shared_up, (int)Is, (int)H);
      D.S.down = make_proj(a->shared_down, (int)H, (int)Is);
      D.S.is = (int)Is;
      D.S.act = ws.sh_act;
      D.S.y = ws.sh_y;
    }
    // events[1] and [2] take the gate/up kernel's own start and end timestamps
    D.gate_up_start = a->events ? a->events[1] : nullptr;
    D.after_gate_up = a->events ? a->events[2] : nullptr;
    D.after_down = a->events ? a->events[3] : nullptr;
    if ((rc = launch_moe_decode(fmt, fmt_dn, D, s))) return rc;
    rc = check_launch("moe decode kernels");
    mark(4);
    return rc;
  }
  mark(0);
  {
    static std::atomic<uint64_t> attr_done{0};
    // top_k <= 32, experts <= kMaxExperts: at most 64 KB of staged rows for
    // the count, 132 KB of staged rows, bitmaps and positions for the scatter
    const auto scatter_lds = [](int64_t k, int64_t e) { return (size_t)(3 * kChunk * k + e * (kChunkWords + 1)) * 4; };
    once_per_device(attr_done, [&] {
      (void)hipFuncSetAttribute((const void*)moe_route_count_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kChunk * 32 * 8);
      (void)hipFuncSetAttribute((const void*)moe_route_scatter_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)scatter_lds(32, kMaxExperts));
      (void)hipFuncSetAttribute((const void*)moe_route_small_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(scatter_lds(32, kMaxExperts) + kMaxExperts * 4));
      (void)hipFuncSetAttribute((const void*)moe_route_scan_scatter_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)scatter_lds(32, kMaxExperts));
    });
    const int nchunks = (int)cdiv(B, kChunk);
    int* chunk_cnt = reinterpret_cast<int*>(w + L.chunk_cnt);
    if (nchunks == 1) {
      // one chunk: the three passes in one launch (its counts and positions in LDS)
      const unsigned lanes = (unsigned)std::max<int64_t>(kChunk, cdiv(E, 64) * 64);
      hipLaunchKernelGGL(moe_route_small_kernel, dim3(1), dim3(lanes), scatter_lds(K, E) + (size_t)E * 4, s, a->ids,
                         a->weights, (int)B, (int)K, (int)E, (int)kPrefillTile, ws);
    } else {
      hipLaunchKernelGGL(moe_route_count_kernel, dim3(nchunks), dim3(kChunk), (size_t)kChunk * K * 8, s, a->ids,
                         a->weights, (int)B, (int)K, (int)E, ws, chunk_cnt);
      if (nchunks <= kFoldChunks) {
        // the scan folded into the scatter workgroups (up to 8192 tokens)
        const unsigned lanes = (unsigned)std::max<int64_t>(kChunk, cdiv(E, 64) * 64);
        hipLaunchKernelGGL(moe_route_scan_scatter_kernel, dim3(nchunks), dim3(lanes), scatter_lds(K, E), s, a->ids,
                           (int)B, (int)K, (int)E, nchunks, (int)kPrefillTile, ws, chunk_cnt);
      } else {
        hipLaunchKernelGGL(moe_route_scan_kernel, dim3(1), dim3((unsigned)cdiv(E, 64) * 64), 0, s, (int)E, nchunks,
                           (int)kPrefillTile, ws, chunk_cnt);
        hipLaunchKernelGGL(moe_route_scatter_kernel, dim3(nchunks), dim3(kChunk), scatter_lds(K, E), s, a->ids,
                           (int)B, (int)K, (int)E, nchunks, ws, chunk_cnt);
      }
    }
    if ((rc = check_launch("moe routing kernels"))) return rc;
  }

  TokenSrc routed{0, (int)B, ws.hdr, ws.active, ws.act_off, ws.route_tok};
  const int slots = (int)(E < B * K ? E : B * K);
  const Proj g = make_proj(a->gate, (int)I, (int)H), u = make_proj(a->up, (int)I, (int)H),
             d = make_proj(a->down, (int)H, (int)I);
  const int max_tokens = (int)B;  // an expert sees each token at most once
  // int8_q8 policy: the Q8_0 projections run W8A8 (compute.py:20-34)
  const bool w8_gu = w8 && fmt == FMT_Q8, w8_dn = w8 && fmt_dn == FMT_Q8;
  // The tiled MFMA kernels address token rows with 32-bit byte offsets.
  const bool rows32 = B * H * 2 < (1ll << 31) && B * K * I * 2 < (1ll << 31);
  const bool tiled_gu = !w8_gu && rows32 && pf_gate_up_supported(fmt, H, I);
  const bool tiled_dn = !w8_dn && rows32 && pf_down_supported(fmt_dn, H, I);
  const int max_tiles = (int)(E + B * K / kPrefillTile + 1);
  if ((tiled_gu || tiled_dn) && pf_tile_routes() != kPrefillTile) {
    set_error("moe_forward: prefill tile size mismatch");
    return Q6MOE_ERR_HIP;
  }
  // gate/up + SwiGLU
  if (w8_gu) {
    mark(1);
    int8_t* xq = reinterpret_cast<int8_t*>(w + L.xq);
    float* xq_s = reinterpret_cast<float*>(w + L.xq_s);
    launch_act_q8(a->x, B, (int)H, nullptr, xq, xq_s, s);
    launch_w8(true, g, u, routed, slots, 0, W8Src{xq, xq_s, (int)H}, ws.act, s);
    mark(2);
  } else if (tiled_gu) {
    // events[1] and [2] take the gate/up kernel's own start and end timestamps
    launch_moe_prefill_gate_up(fmt, g, u, ws, max_tiles, a->x, (int)B, (int)H, (int)I, s,
                               a->events ? a->events[1] : nullptr, a->events ? a->events[2] : nullptr);
  } else {
    mark(1);
    dispatch_format(fmt, [&](auto fg) {
      launch_gate_up<decltype(fg)::value>(g, u, routed, slots, max_tokens, a->x, (int)H, (int)I, ws.act, s);
    });
    mark(2);
  }
  // down projection
  if (w8_dn) {
    int8_t* aq = reinterpret_cast<int8_t*>(w + L.aq);
    float* aq_s = reinterpret_cast<float*>(w + L.aq_s);
    launch_act_q8(ws.act, B * K, (int)I, ws.hdr + 1, aq, aq_s, s);  // rows beyond the routes are skipped
    launch_w8(false, d, d, routed, slots, 1, W8Src{aq, aq_s, (int)I}, ws.y, s);
  } else if (tiled_dn) {
    launch_moe_prefill_down(fmt_dn, d, ws, max_tiles, (int)(B * K), (int)H, (int)I, s);
  } else {
    dispatch_format(fmt_dn, [&](auto fd) {
      launch_down<decltype(fd)::value>(d, routed, slots, max_tokens, ws.act, (int)H, (int)I, ws.y, s);
    });
  }
  if ((rc = check_launch("moe expert kernels"))) return rc;
  if (Is) {
    TokenSrc dense{1, (int)B, nullptr, nullptr, nullptr, nullptr};
    const Proj sg = make_proj(a->shared_gate, (int)Is, (int)H), su = make_proj(a->shared_up, (int)Is, (int)H),
               sd = make_proj(a->shared_down, (int)H, (int)Is);
    phases(sg, su, sd, dense, 1, (int)B, (int)Is, ws.sh_act, ws.sh_y, [](int) {});
    if ((rc = check_launch("moe shared expert kernels"))) return rc;
  }
  mark(3);
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)B, (unsigned)cdiv(H, 256 * 8)), dim3(256), 0, s,
                     ws.tok_pos, ws.route_w, ws.y, (int)K, (int)H, ws.sh_y, sh_scale, a->out);
  rc = check_launch("moe_combine_kernel");
  mark(4);
  return rc;
}

extern "C" int q6moe_moe_forward(const q6moe_moe_args* a, void* stream) {
  Q6MOE_REQUIRE(a, "moe_forward: null args");
  return moe_forward_impl(a, a->workspace, a->workspace_bytes, stream);
}

extern "C" int q6moe_moe_forward_noalloc(const q6moe_moe_args* a, void* stream) {
  Q6MOE_REQUIRE(a, "moe_forward_noalloc: null args");
  Q6MOE_REQUIRE(!a->workspace && a->workspace_bytes == 0,
                "moe_forward_noalloc: takes no workspace (workspace must be NULL and workspace_bytes 0)");
  void* ptr = nullptr;
  const int rc = static_scratch(&ptr);
  if (rc) return rc;
  return moe_forward_impl(a, ptr, kStaticScratchBytes, stream, true);
}

// Workspace of q6moe_q8_matmul: the quantised x (codes, FP32 scales).
static size_t q8_ws(int64_t m, int64_t k, size_t* scales_at) {
  const size_t codes = align256((size_t)(m * k));
  if (scales_at) *scales_at = codes;
  return codes + align256((size_t)(m * (k / 32) * 4));
}

extern "C" size_t q6moe_q8_matmul_workspace_size(int64_t m, int64_t k) {
  if (m < 1 || k < 32 || k % 32) return 0;
  return q8_ws(m, k, nullptr);
}

extern "C" int q6moe_q8_matmul(const uint16_t* x, int64_t m, int64_t k, const uint8_t* table, int64_t n, uint16_t* y,
                               void* workspace, size_t workspace_bytes, void* stream) {
  Q6MOE_REQUIRE(x && table && y && workspace, "q8_matmul: null pointer");
  Q6MOE_REQUIRE(m >= 1 && n >= 1 && k >= 32 && k % 32 == 0, "q8_matmul: need m, n >= 1 and k a multiple of 32");
  Q6MOE_REQUIRE(m <= (1 << 24) && n <= (1 << 24) && k <= (1 << 24), "q8_matmul: dimension too large");
  Q6MOE_REQUIRE(aligned(x, 16) && aligned(table, 16) && aligned(workspace, 256),
                "q8_matmul: x and table need 16-byte and workspace 256-byte alignment");
  size_t scales_at = 0;
  const size_t need = q8_ws(m, k, &scales_at);
  if (workspace_bytes < need) {
    set_error("q8_matmul: workspace too small (need " + std::to_string(need) + " bytes)");
    return Q6MOE_ERR_INVALID;
  }
  hipStream_t s = (hipStream_t)stream;
  int8_t* codes = reinterpret_cast<int8_t*>(workspace);
  float* scales = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + scales_at);
  launch_act_q8(x, m, (int)k, nullptr, codes, scales, s);
  q6moe_table t{Q6MOE_Q8_0, table, (int64_t)unit_table_bytes(Q6MOE_Q8_0, n, k), nullptr, 0};
  const Proj p = make_proj(t, (int)n, (int)k);
  TokenSrc dense{1, (int)m, nullptr, nullptr, nullptr, nullptr};
  launch_w8(false, p, p, dense, 1, 0, W8Src{codes, scales, (int)k}, y, s);
  return check_launch("q8_matmul kernels");
}
