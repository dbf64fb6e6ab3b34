// Decode attention over the paged INT8 KV cache: one query token per
// sequence against its cached tokens, with the dequant of read_quantized
// fused in, so the BF16 keys and values are never written to HBM. It is the
// core of the reference's decode step (kaggle/qwen38_tpu/attention_cache.py:
// 159-169 after read_quantized :71-81), with the same rounding points:
//
//   k, v   = RNE_bf16(f32(code) * f32(scale))          (per token and head)
//   raw    = RNE_bf16(sum_d q * k)                     (FP32 accumulation)
//   score  = RNE_bf16(f32(raw) / sqrt(D))
//   prob   = exp(score - max) / sum exp(score - max)   (FP32, numerics.softmax)
//   out    = RNE_bf16(sum_t RNE_bf16(prob) * v)        (FP32 accumulation)
//
// Three launches (the normalised probability is rounded before it weighs V,
// so the softmax statistics must be complete before the P.V pass):
//   1. attn_scores_kernel: per (256-token chunk, KV head, sequence), the
//      chunk's keys are dequantised into MFMA A operands (16 tokens x 32
//      channels per v_mfma_f32_16x16x32_bf16) against the group's query
//      heads as B operand; scores go to the workspace as BF16, and each
//      wave's maximum m_w and sum l_w of exp(score - m_w) over its 64 tokens.
//   2. attn_pv_kernel: per 2048-token chunk (8 waves, four 64-token tiles
//      each), wave h first merges head h's statistics over the attended
//      tokens, max = max_w m_w and sum = sum_w l_w exp(m_w - max) in a fixed
//      order; the workgroup forms RNE_bf16(prob) once per (head, token) in
//      LDS; each wave then runs P.V for its tiles, in turn, on MFMA with the
//      dequantised values as A operand (row = 8 channels apart, so a lane
//      dequantises the 8x8 code block it loaded straight into eight tiles'
//      operands) and the probabilities as B; the chunk's partial sums go to
//      the workspace.
//   3. attn_combine_kernel: partial sums over chunks in a fixed order, RNE.
//
// HBM-bound: the INT8 codes and scales of K and V are read once.
#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

constexpr int kAttnD = 128;      // head_dim
constexpr int kAttnR = 8;        // at most this many query heads per KV head
constexpr int kAttnChunk = 256;  // tokens per scores workgroup: 4 waves x 64
constexpr int kAttnWaveTok = 64;
constexpr int kPvWaves = 8;      // waves per P.V workgroup
constexpr int kPvThreads = kPvWaves * 64;
constexpr int kPvTiles = 4;      // 64-token tiles per P.V wave
constexpr int kPvChunk = kPvTiles * kPvThreads;  // tokens per P.V workgroup (one partial sum)

struct AttnParams {
  const uint16_t* q;                 // [B, Hq, D]
  const int8_t* kc;                  // [pages, P, KVH*D]
  const int8_t* vc;
  const float* ks;                   // [pages*P, KVH]
  const float* vs;
  const int32_t* table;              // [B, pps]
  const int32_t* len;                // [B]
  int64_t pool_pages;
  int pps, page, kvh, hq, r, cap, nchunks;  // nchunks: P.V chunks of kPvChunk tokens
  uint16_t* s;                       // [B, Hq, cap] BF16 scores
  float* wstats;                     // [B, Hq, cap / 64, 2]: per 64 tokens, max m_w and sum of exp(score - m_w)
  float* part;                       // [B, KVH, nchunks, kAttnR, D]
  uint16_t* out;                     // [B, Hq, D]
};

// Attended tokens of sequence b, clamped into [1, cap].
__device__ __forceinline__ int attn_len(const AttnParams& p, int b) {
  const int n = p.len[b];
  return n < 1 ? 1 : (n > p.cap ? p.cap : n);
}

// Page-table entry of token t0 of sequence b. The page index is clamped into
// the sequence's row, so the load is in bounds for any t0 and can be issued
// before the sequence length is known. A wave's 64 tokens t0 + [0, 64) (t0 a
// multiple of 64) lie in one page, since page_size is a multiple of 64: one
// table lookup per wave.
__device__ __forceinline__ int64_t attn_page(const AttnParams& p, int b, int t0) {
  const int pi = t0 / p.page;
  return p.table[(int64_t)b * p.pps + (pi < p.pps ? pi : p.pps - 1)];
}

// Pool row of token t0 on page pg, or -1 for an unmapped page (read as 0).
__device__ __forceinline__ int64_t attn_row(const AttnParams& p, int64_t pg, int t0) {
  return pg < 0 || pg >= p.pool_pages ? -1 : pg * p.page + t0 % p.page;
}

__global__ void __launch_bounds__(256) attn_scores_kernel(AttnParams p) {
  const int chunk = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = attn_len(p, b);
  const int t0 = chunk * kAttnChunk + wave * kAttnWaveTok;
  if (t0 >= n) return;
  const int col = lane & 15, g = lane >> 4;  // MFMA column (query head) and K group
  // B operand: query head kh*r + col, channels 32g + 8ks + [0, 8) of step ks
  u32x4 qb[4];
  {
    const bool live = col < p.r;
    const uint16_t* qr = p.q + ((int64_t)b * p.hq + kh * p.r + (live ? col : 0)) * kAttnD + 32 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qr + 8 * ks);
      qb[ks] = live ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const float kDiv = static_cast<float>(11.313708498984761);  // float32(128 ** 0.5) (attention_cache.py:163)
  const int64_t rowbytes = (int64_t)p.kvh * kAttnD;
  const int64_t base = attn_row(p, attn_page(p, b, t0), t0);
  // the wave's rows start at pool row base (wave-uniform); the lane adds its
  // token row col and channel group 32-bit offsets, row block rb adds 16 rows
  const int8_t* kw = p.kc + (base < 0 ? 0 : base) * rowbytes + kh * kAttnD;
  const float* sw = p.ks + (base < 0 ? 0 : base) * p.kvh + kh;
  const uint32_t lane_off = (uint32_t)col * (uint32_t)rowbytes + 32u * g;
  const uint32_t rb_off = 16u * (uint32_t)rowbytes;
  // A operand of row block rb: token t0 + 16rb + col, channels 32g + [0, 32);
  // the next block's loads are issued before this block is multiplied
  u32x4 cw[4][2];
  float scw[4];
  float sv[4][4];  // the lane's scores
  auto load_rb = [&](int rb) {
    const int t = t0 + 16 * rb + col;
    cw[rb][0] = cw[rb][1] = u32x4{0u, 0u, 0u, 0u};
    scw[rb] = 0.f;
    if (t < n && base >= 0) {
      const int8_t* src = kw + lane_off + rb * rb_off;
      cw[rb][0] = *reinterpret_cast<const u32x4*>(src);
      cw[rb][1] = *reinterpret_cast<const u32x4*>(src + 16);
      scw[rb] = sw[(16 * rb + col) * p.kvh];
    }
  };
  load_rb(0);
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    if (rb + 1 < 4) load_rb(rb + 1);
    const u32x4 c0 = cw[rb][0], c1 = cw[rb][1];
    const float sc = scw[rb];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint32_t w0 = ks < 2 ? c0[2 * ks] : c1[2 * ks - 4];
      const uint32_t w1 = ks < 2 ? c0[2 * ks + 1] : c1[2 * ks - 3];
      u32x4 a;
      a[0] = pack_bf16x2((float)(int8_t)w0 * sc, (float)(int8_t)(w0 >> 8) * sc);
      a[1] = pack_bf16x2((float)(int8_t)(w0 >> 16) * sc, (float)(int8_t)(w0 >> 24) * sc);
      a[2] = pack_bf16x2((float)(int8_t)w1 * sc, (float)(int8_t)(w1 >> 8) * sc);
      a[3] = pack_bf16x2((float)(int8_t)(w1 >> 16) * sc, (float)(int8_t)(w1 >> 24) * sc);
      acc = mfma16(a, qb[ks], acc);
    }
    // lane holds tokens t0 + 16rb + 4g + [0, 4) of query head col
    const int tt = t0 + 16 * rb + 4 * g;
#pragma unroll
    for (int v = 0; v < 4; ++v) sv[rb][v] = bf16_round(bf16_round(acc[v]) / kDiv);
    if (col < p.r) {
      uint16_t* dst = p.s + ((int64_t)b * p.hq + kh * p.r + col) * p.cap + tt;
      *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(sv[rb][0], sv[rb][1]), pack_bf16x2(sv[rb][2], sv[rb][3])};
    }
  }
  // The wave's statistics of head col over its attended tokens: the maximum
  // over the lane's scores and the four K groups (lanes col + 16g), then the
  // sum of exp(score - max) (hardware exponential: the sum only normalises,
  // and the P.V kernel's merge weighs it by an accurate exp) the same way.
  float m = -__builtin_inff();
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (t0 + 16 * rb + 4 * g + v < n) m = fmaxf(m, sv[rb][v]);
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  float l = 0.f;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (t0 + 16 * rb + 4 * g + v < n) l += __expf(sv[rb][v] - m);
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (g == 0 && col < p.r) {
    float* ws = p.wstats + (((int64_t)b * p.hq + kh * p.r + col) * (p.cap / kAttnWaveTok) + t0 / kAttnWaveTok) * 2;
    *reinterpret_cast<f32x2*>(ws) = f32x2{m, l};
  }
}

__global__ void __launch_bounds__(kPvThreads) __attribute__((amdgpu_waves_per_eu(4))) attn_pv_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t pr[kAttnR][kPvChunk];  // RNE_bf16(prob) [head][token]
  __shared__ float red[kPvWaves][kAttnR][kAttnD];                       // per-wave partial sums
  const int chunk = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c0 = chunk * kPvChunk;
  const int r16 = lane & 15, kg = lane >> 4;
  __shared__ f32x2 s_st[kAttnR];                                        // the heads' (max, sum)
  // The wave's page entries (tile i: tokens c0 + kPvThreads*i + 64*wave + [0, 64))
  // are read together with the length.
  int64_t pg[kPvTiles];
#pragma unroll
  for (int i = 0; i < kPvTiles; ++i) pg[i] = attn_page(p, b, c0 + kPvThreads * i + 64 * wave);
  const int n = attn_len(p, b);
  asm volatile("" ::: "memory");  // the loads above issue before the length is waited for
  if (c0 >= n) return;  // uniform over the workgroup
  const int nv = n - c0 < kPvChunk ? n - c0 : kPvChunk;
  // For the probability pass (thread t = tokens c0 + t + kPvThreads*i): the
  // chunk's scores of every head (token clamped into the sequence's length),
  // loaded together with the statistics below.
  const int t = threadIdx.x;
  uint16_t sc[kPvTiles][kAttnR];
#pragma unroll
  for (int i = 0; i < kPvTiles; ++i) {
    const int tt = t + kPvThreads * i;
    const int tc = c0 + (tt < nv ? tt : nv - 1);
#pragma unroll
    for (int h = 0; h < kAttnR; ++h)
      sc[i][h] = p.s[((int64_t)b * p.hq + kh * p.r + (h < p.r ? h : 0)) * p.cap + tc];
  }
  // The softmax statistics of head h < r, merged by wave h from the scores
  // kernel's per-64-token (m_w, l_w): lane i takes groups i, i + 64, ... in
  // order (the first 8 in one batch of loads), max over them and a fixed xor
  // tree, then sum of l_w exp(m_w - max) the same way; every workgroup of the
  // head computes the same values.
  float sm[kAttnR], sl[kAttnR];
  {
    const int nw = (n + kAttnWaveTok - 1) / kAttnWaveTok;
    const f32x2* wsh = reinterpret_cast<const f32x2*>(p.wstats) +
                       ((int64_t)b * p.hq + kh * p.r + (wave < p.r ? wave : 0)) * (p.cap / kAttnWaveTok);
    f32x2 wl[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int w = lane + 64 * u;
      wl[u] = wsh[w < nw ? w : nw - 1];
    }
    if (wave < p.r) {  // uniform over the wave
      float m = -__builtin_inff();
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (lane + 64 * u < nw) m = fmaxf(m, wl[u][0]);
      for (int w = lane + 512; w < nw; w += 64) m = fmaxf(m, wsh[w][0]);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      float l = 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (lane + 64 * u < nw) l += wl[u][1] * expf(wl[u][0] - m);
      for (int w = lane + 512; w < nw; w += 64) {
        const f32x2 v = wsh[w];
        l += v[1] * expf(v[0] - m);
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) l += __shfl_xor(l, off);
      if (lane == 0) s_st[wave] = f32x2{m, l};
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kAttnR; ++h) {
      const f32x2 v = s_st[h < p.r ? h : 0];
      sm[h] = v[0];
      sl[h] = v[1];
    }
  }
  // V codes of a tile: lane (r16, kg) reads channels 8*r16 + [0, 8) of the
  // wave's tokens 32s + 8kg + j (s = 0, 1; j = 0..7), all in the wave's page
  // (row 0 of the pool for an unmapped one); tokens from nv on and unmapped
  // pages are zeroed after the loads.
  const int64_t rowbytes = (int64_t)p.kvh * kAttnD;
  const uint32_t lane_off = (uint32_t)(8 * kg) * (uint32_t)rowbytes + 8u * r16;
  u32x2 wv[2][8];
  float sv[2][8];
  int64_t base = 0;
  auto load_tile = [&](int i) {
    base = attn_row(p, pg[i], c0 + kPvThreads * i + 64 * wave);
    const int8_t* vw = p.vc + (base < 0 ? 0 : base) * rowbytes + kh * kAttnD;
    const float* sw = p.vs + ((base < 0 ? 0 : base) + 8 * kg) * p.kvh + kh;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        wv[st][j] = *reinterpret_cast<const u32x2*>(vw + lane_off + (uint32_t)(32 * st + j) * (uint32_t)rowbytes);
        sv[st][j] = sw[(32 * st + j) * p.kvh];
      }
  };
  // the V operands of tokens from nv on, and of an unmapped page, are zero
  auto mask_tile = [&](int i) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = base >= 0 && kPvThreads * i + 64 * wave + 32 * st + 8 * kg + j < nv;
        wv[st][j] = ok ? wv[st][j] : u32x2{0u, 0u};
        sv[st][j] = ok ? sv[st][j] : 0.f;
      }
  };
  load_tile(0);  // the V codes' loads overlap the probability pass
  // 1. RNE_bf16(prob) of every (head, token) of the chunk, once; heads from r
  //    on are 0 (MFMA columns 8-15 take zero operands below)
#pragma unroll
  for (int i = 0; i < kPvTiles; ++i)
#pragma unroll
    for (int h = 0; h < kAttnR; ++h) {
      const int tt = t + kPvThreads * i;
      float q = 0.f;
      if (tt < nv && h < p.r) q = bf16_round(expf(bf16_to_float(sc[i][h]) - sm[h]) / sl[h]);
      pr[h][tt] = bf16_bits(q);
    }
  mask_tile(0);
  __syncthreads();
  // 2. out[h][d] over the wave's tokens as 8 tiles of v_mfma_f32_16x16x32_bf16:
  //    tile T has A[row r][k] = v[token 32s + k][channel 8r + T] (lane (r16, kg)
  //    dequantises byte T of its 8 tokens) and B[k][col h] = prob[h][token 32s + k];
  //    the wave's token tiles in order (a tile wholly past nv is skipped)
  f32x4 acc[8];
#pragma unroll
  for (int T = 0; T < 8; ++T) acc[T] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kPvTiles; ++i) {
    if (kPvThreads * i + 64 * wave >= nv) break;  // uniform over the wave
    if (i > 0) {  // the loads of a later tile wait for this wave's earlier MFMAs
      load_tile(i);
      mask_tile(i);
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      u32x4 bq = {0u, 0u, 0u, 0u};
      if (r16 < kAttnR) bq = *reinterpret_cast<const u32x4*>(&pr[r16][kPvThreads * i + 64 * wave + 32 * st + 8 * kg]);
#pragma unroll
      for (int T = 0; T < 8; ++T) {
        auto val = [&](int j) {
          const uint32_t w = T < 4 ? wv[st][j][0] : wv[st][j][1];
          return (float)(int8_t)(w >> (8 * (T & 3))) * sv[st][j];
        };
        u32x4 a;
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = pack_bf16x2(val(2 * q), val(2 * q + 1));
        acc[T] = mfma16(a, bq, acc[T]);
      }
    }
  }
  // 3. lane (h = r16, kg) holds out[h][8*(4kg + v) + T] = acc[T][v]; the
  //    waves' sums are added in wave order
  if (r16 < kAttnR) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int T = 0; T < 8; ++T) red[wave][r16][32 * kg + 8 * v + T] = acc[T][v];
  }
  __syncthreads();
  float* dst = p.part + (((int64_t)b * p.kvh + kh) * p.nchunks + chunk) * kAttnR * kAttnD;
  for (int o = threadIdx.x; o < kAttnR * kAttnD; o += kPvThreads) {
    const int h = o / kAttnD, d = o % kAttnD;
    float v = red[0][h][d];
#pragma unroll
    for (int w = 1; w < kPvWaves; ++w) v += red[w][h][d];
    dst[o] = v;
  }
}

// Eight thread groups per output channel each add a contiguous eighth of the
// chunks in chunk order; the eight group sums are then added in group order.
__global__ void __launch_bounds__(8 * kAttnD) attn_combine_kernel(AttnParams p) {
  __shared__ float red[8][kAttnD];
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x % kAttnD, grp = threadIdx.x / kAttnD;
  const int kh = h / p.r, hr = h % p.r;
  const int nc = (attn_len(p, b) + kPvChunk - 1) / kPvChunk;
  const int per = (nc + 7) / 8, cb = grp * per, ce = cb + per < nc ? cb + per : nc;
  const float* src = p.part + (((int64_t)b * p.kvh + kh) * p.nchunks) * kAttnR * kAttnD + hr * kAttnD + d;
  float v = 0.f;
  for (int c0 = cb; c0 < ce; c0 += 8) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = c0 + u < ce ? src[(int64_t)(c0 + u) * kAttnR * kAttnD] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (c0 + u < ce) v += x[u];
  }
  red[grp][d] = v;
  __syncthreads();
  if (grp == 0) {
    float t = red[0][d];
#pragma unroll
    for (int g = 1; g < 8; ++g)
      if (g * per < nc) t += red[g][d];
    p.out[((int64_t)b * p.hq + h) * kAttnD + d] = bf16_bits(t);
  }
}

struct AttnLayout {
  size_t s, wstats, part, total;
};

static size_t attn_align(size_t v) { return (v + 255) & ~(size_t)255; }

static AttnLayout attn_layout(int64_t B, int64_t hq, int64_t kvh, int64_t cap) {
  AttnLayout L;
  const int64_t nchunks = (cap + kPvChunk - 1) / kPvChunk;
  L.s = 0;
  L.wstats = attn_align(L.s + (size_t)B * hq * cap * 2);
  L.part = attn_align(L.wstats + (size_t)B * hq * (cap / kAttnWaveTok) * 2 * 4);
  L.total = attn_align(L.part + (size_t)B * kvh * nchunks * kAttnR * kAttnD * 4);
  return L;
}

}  // namespace q6moe

using namespace q6moe;

extern "C" size_t q6moe_attn_workspace_size(int64_t batch, int64_t query_heads, int64_t kv_heads,
                                            int64_t pages_per_seq, int64_t page_size) {
  if (batch < 1 || query_heads < 1 || kv_heads < 1 || pages_per_seq < 1 || page_size < 1) return 0;
  return attn_layout(batch, query_heads, kv_heads, pages_per_seq * page_size).total;
}

extern "C" int q6moe_kv_decode_attention(const q6moe_attn_args* a, void* stream) {
  Q6MOE_REQUIRE(a, "decode_attention: null args");
  Q6MOE_REQUIRE(a->q && a->k_codes && a->v_codes && a->k_scales && a->v_scales && a->page_table && a->lengths &&
                    a->out && a->workspace,
                "decode_attention: null pointer");
  Q6MOE_REQUIRE(a->head_dim == kAttnD, "decode_attention: head_dim must be 128");
  Q6MOE_REQUIRE(a->batch >= 1 && a->batch <= 65535 && a->kv_heads >= 1 && a->kv_heads <= 65535 &&
                    a->query_heads >= 1 && a->query_heads % a->kv_heads == 0 &&
                    a->query_heads / a->kv_heads <= kAttnR,
                "decode_attention: query_heads must be a multiple of kv_heads, at most 8 per KV head");
  Q6MOE_REQUIRE(a->page_size >= 64 && a->page_size % 64 == 0 && a->pages_per_seq >= 1 && a->pool_pages >= 1,
                "decode_attention: page_size must be a multiple of 64");
  const int64_t cap = a->pages_per_seq * a->page_size;
  Q6MOE_REQUIRE(cap <= (1 << 24) && a->pool_pages * a->page_size <= (1ll << 40),
                "decode_attention: cache too large");
  Q6MOE_REQUIRE(aligned(a->q, 16) && aligned(a->k_codes, 16) && aligned(a->v_codes, 16) && aligned(a->out, 4) &&
                    aligned(a->workspace, 256),
                "decode_attention: q/codes need 16-byte, out 4-byte and workspace 256-byte alignment");
  const AttnLayout L = attn_layout(a->batch, a->query_heads, a->kv_heads, cap);
  if (a->workspace_bytes < L.total) {
    set_error("decode_attention: workspace too small (need " + std::to_string(L.total) + " bytes)");
    return Q6MOE_ERR_INVALID;
  }
  AttnParams p;
  p.q = a->q;
  p.kc = a->k_codes;
  p.vc = a->v_codes;
  p.ks = a->k_scales;
  p.vs = a->v_scales;
  p.table = a->page_table;
  p.len = a->lengths;
  p.pool_pages = a->pool_pages;
  p.pps = (int)a->pages_per_seq;
  p.page = (int)a->page_size;
  p.kvh = (int)a->kv_heads;
  p.hq = (int)a->query_heads;
  p.r = (int)(a->query_heads / a->kv_heads);
  p.cap = (int)cap;
  p.nchunks = (int)((cap + kPvChunk - 1) / kPvChunk);
  uint8_t* w = reinterpret_cast<uint8_t*>(a->workspace);
  p.s = reinterpret_cast<uint16_t*>(w + L.s);
  p.wstats = reinterpret_cast<float*>(w + L.wstats);
  p.part = reinterpret_cast<float*>(w + L.part);
  p.out = a->out;
  hipStream_t s = (hipStream_t)stream;
  const dim3 chunks((unsigned)((cap + kAttnChunk - 1) / kAttnChunk), (unsigned)p.kvh, (unsigned)a->batch);
  const dim3 pv_chunks((unsigned)p.nchunks, (unsigned)p.kvh, (unsigned)a->batch);
  hipLaunchKernelGGL(attn_scores_kernel, chunks, dim3(256), 0, s, p);
  hipLaunchKernelGGL(attn_pv_kernel, pv_chunks, dim3(kPvThreads), 0, s, p);
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)p.hq, (unsigned)a->batch), dim3(8 * kAttnD), 0, s, p);
  return check_launch("decode_attention kernels");
}
