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
// Four launches (the normalised probability is rounded before it weighs V,
// so the softmax statistics must be complete before the P.V pass):
//   1. attn_scores_kernel: per (256-token chunk, KV head, sequence), the
//      chunk's keys are dequantised into MFMA A operands (16 tokens x 32
//      channels per v_mfma_f32_16x16x32_bf16) against the group's query
//      heads as B operand; scores go to the workspace as BF16.
//   2. attn_stats_kernel: per (sequence, query head), the maximum and the sum
//      of exp(score - max) over the attended tokens (fixed reduction order).
//   3. attn_pv_kernel: per chunk, the workgroup forms RNE_bf16(prob) once per
//      (token, head) in LDS, then each lane accumulates 8 heads x 8 channels
//      over token pairs with v_dot2_f32_bf16 (two tokens per instruction);
//      the chunk's partial sums go to the workspace.
//   4. attn_combine_kernel: partial sums over chunks in chunk order, RNE.
//
// HBM-bound: the INT8 codes and scales of K and V are read once.
#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

constexpr int kAttnD = 128;      // head_dim
constexpr int kAttnR = 8;        // at most this many query heads per KV head
constexpr int kAttnChunk = 256;  // tokens per workgroup: 4 waves x 64
constexpr int kAttnWaveTok = 64;

struct AttnParams {
  const uint16_t* q;                 // [B, Hq, D]
  const int8_t* kc;                  // [pages, P, KVH*D]
  const int8_t* vc;
  const float* ks;                   // [pages*P, KVH]
  const float* vs;
  const int32_t* table;              // [B, pps]
  const int32_t* len;                // [B]
  int64_t pool_pages;
  int pps, page, kvh, hq, r, cap, nchunks;
  uint16_t* s;                       // [B, Hq, cap] BF16 scores
  float* stats;                      // [B, Hq, 2]: max, sum
  float* part;                       // [B, KVH, nchunks, kAttnR, D]
  uint16_t* out;                     // [B, Hq, D]
};

// Attended tokens of sequence b, clamped into [1, cap].
__device__ __forceinline__ int attn_len(const AttnParams& p, int b) {
  const int n = p.len[b];
  return n < 1 ? 1 : (n > p.cap ? p.cap : n);
}

// Pool row of token t of sequence b, or -1 for an unmapped page (read as 0).
__device__ __forceinline__ int64_t attn_row(const AttnParams& p, int b, int t) {
  const int64_t pg = p.table[(int64_t)b * p.pps + t / p.page];
  return pg < 0 || pg >= p.pool_pages ? -1 : pg * p.page + t % p.page;
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
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    // A operand: token t (row col of the block), channels 32g + [0, 32)
    const int t = t0 + 16 * rb + col;
    const int64_t row = t < n ? attn_row(p, b, t) : -1;
    u32x4 c0 = {0u, 0u, 0u, 0u}, c1 = {0u, 0u, 0u, 0u};
    float sc = 0.f;
    if (row >= 0) {
      const int8_t* src = p.kc + row * rowbytes + kh * kAttnD + 32 * g;
      c0 = *reinterpret_cast<const u32x4*>(src);
      c1 = *reinterpret_cast<const u32x4*>(src + 16);
      sc = p.ks[row * p.kvh + kh];
    }
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
    if (col < p.r) {
      uint32_t o[2];
#pragma unroll
      for (int v = 0; v < 4; v += 2) {
        const float s0 = bf16_round(bf16_round(acc[v]) / kDiv);
        const float s1 = bf16_round(bf16_round(acc[v + 1]) / kDiv);
        o[v >> 1] = pack_bf16x2(s0, s1);
      }
      const int tt = t0 + 16 * rb + 4 * g;
      uint16_t* dst = p.s + ((int64_t)b * p.hq + kh * p.r + col) * p.cap + tt;
      *reinterpret_cast<u32x2*>(dst) = u32x2{o[0], o[1]};
    }
  }
}

// Sum of a 256-thread block in a fixed order (warp-level tree in LDS).
__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  red[threadIdx.x] = v;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) {
      const float a = red[threadIdx.x], c = red[threadIdx.x + off];
      red[threadIdx.x] = is_max ? fmaxf(a, c) : a + c;
    }
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(256) attn_stats_kernel(AttnParams p) {
  __shared__ float red[256];
  const int h = blockIdx.x, b = blockIdx.y;
  const int n = attn_len(p, b);
  const uint16_t* s = p.s + ((int64_t)b * p.hq + h) * p.cap;
  float m = -__builtin_inff();
  for (int t = threadIdx.x; t < n; t += 256) m = fmaxf(m, bf16_to_float(s[t]));
  m = block_reduce(m, red, true);
  float l = 0.f;
  for (int t = threadIdx.x; t < n; t += 256) l += expf(bf16_to_float(s[t]) - m);
  l = block_reduce(l, red, false);
  if (threadIdx.x == 0) {
    p.stats[((int64_t)b * p.hq + h) * 2] = m;
    p.stats[((int64_t)b * p.hq + h) * 2 + 1] = l;
  }
}

__global__ void __launch_bounds__(256) attn_pv_kernel(AttnParams p) {
  __shared__ uint32_t pp[kAttnChunk / 2][kAttnR];  // BF16 prob pairs (tokens 2m, 2m+1) per head
  __shared__ float red[4][kAttnR][kAttnD];         // per-wave partial sums
  const int chunk = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = attn_len(p, b);
  const int c0 = chunk * kAttnChunk;
  if (c0 >= n) return;  // uniform over the workgroup
  const int nv = n - c0 < kAttnChunk ? n - c0 : kAttnChunk;
  // 1. RNE_bf16(prob) of every (token, head) of the chunk, once
  {
    const int t = threadIdx.x;
    uint16_t* ph = reinterpret_cast<uint16_t*>(&pp[t >> 1][0]) + (t & 1);
#pragma unroll
    for (int h = 0; h < kAttnR; ++h) {
      float pr = 0.f;
      if (t < nv && h < p.r) {
        const int64_t hh = (int64_t)b * p.hq + kh * p.r + h;
        const float m = p.stats[hh * 2], l = p.stats[hh * 2 + 1];
        pr = bf16_round(expf(bf16_to_float(p.s[hh * p.cap + c0 + t]) - m) / l);
      }
      ph[2 * h] = bf16_bits(pr);
    }
  }
  __syncthreads();
  // 2. lane (channel group dg, token group tg): channels 8dg + [0, 8), token
  //    pairs m = 32*wave + 4i + tg (tokens 2m, 2m+1), i = 0..7
  const int dg = lane & 15, tg = lane >> 4;
  float acc[kAttnR][8];
#pragma unroll
  for (int h = 0; h < kAttnR; ++h)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[h][k] = 0.f;
  const int64_t rowbytes = (int64_t)p.kvh * kAttnD;
#pragma unroll 2
  for (int i = 0; i < 8; ++i) {
    const int m = 32 * wave + 4 * i + tg;
    if (2 * m >= nv) break;
    uint32_t w[2][2];
    float sc[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int t = c0 + 2 * m + e;
      const int64_t row = 2 * m + e < nv ? attn_row(p, b, t) : -1;
      w[e][0] = w[e][1] = 0u;
      sc[e] = 0.f;
      if (row >= 0) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(p.vc + row * rowbytes + kh * kAttnD + 8 * dg);
        w[e][0] = v[0];
        w[e][1] = v[1];
        sc[e] = p.vs[row * p.kvh + kh];
      }
    }
    // BF16 pairs (token 2m, token 2m+1) of channel k
    uint32_t vp[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int sh = 8 * (k & 3);
      const float a = (float)(int8_t)(w[0][k >> 2] >> sh) * sc[0];
      const float c = (float)(int8_t)(w[1][k >> 2] >> sh) * sc[1];
      vp[k] = pack_bf16x2(a, c);
    }
    const u32x4 pa = *reinterpret_cast<const u32x4*>(&pp[m][0]);
    const u32x4 pb = *reinterpret_cast<const u32x4*>(&pp[m][4]);
#pragma unroll
    for (int h = 0; h < kAttnR; ++h) {
      const uint32_t ph = h < 4 ? pa[h] : pb[h - 4];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        acc[h][k] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, vp[k]),
                                                     __builtin_bit_cast(bf16x2, ph), acc[h][k], false);
    }
  }
  // 3. sum the four token groups of each wave, then the four waves, in order
#pragma unroll
  for (int h = 0; h < kAttnR; ++h)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float v = acc[h][k];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][k] = v;
    }
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < kAttnR; ++h)
#pragma unroll
      for (int k = 0; k < 8; ++k) red[wave][h][8 * dg + k] = acc[h][k];
  }
  __syncthreads();
  float* dst = p.part + (((int64_t)b * p.kvh + kh) * p.nchunks + chunk) * kAttnR * kAttnD;
  for (int o = threadIdx.x; o < kAttnR * kAttnD; o += 256) {
    const int h = o / kAttnD, d = o % kAttnD;
    dst[o] = ((red[0][h][d] + red[1][h][d]) + red[2][h][d]) + red[3][h][d];
  }
}

__global__ void __launch_bounds__(kAttnD) attn_combine_kernel(AttnParams p) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int kh = h / p.r, hr = h % p.r;
  const int nc = (attn_len(p, b) + kAttnChunk - 1) / kAttnChunk;
  const float* src = p.part + (((int64_t)b * p.kvh + kh) * p.nchunks) * kAttnR * kAttnD + hr * kAttnD + d;
  float v = 0.f;
  for (int c = 0; c < nc; ++c) v += src[(int64_t)c * kAttnR * kAttnD];
  p.out[((int64_t)b * p.hq + h) * kAttnD + d] = bf16_bits(v);
}

struct AttnLayout {
  size_t s, stats, part, total;
};

static size_t attn_align(size_t v) { return (v + 255) & ~(size_t)255; }

static AttnLayout attn_layout(int64_t B, int64_t hq, int64_t kvh, int64_t cap) {
  AttnLayout L;
  const int64_t nchunks = (cap + kAttnChunk - 1) / kAttnChunk;
  L.s = 0;
  L.stats = attn_align(L.s + (size_t)B * hq * cap * 2);
  L.part = attn_align(L.stats + (size_t)B * hq * 2 * 4);
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
  p.nchunks = (int)((cap + kAttnChunk - 1) / kAttnChunk);
  uint8_t* w = reinterpret_cast<uint8_t*>(a->workspace);
  p.s = reinterpret_cast<uint16_t*>(w + L.s);
  p.stats = reinterpret_cast<float*>(w + L.stats);
  p.part = reinterpret_cast<float*>(w + L.part);
  p.out = a->out;
  hipStream_t s = (hipStream_t)stream;
  const dim3 chunks((unsigned)p.nchunks, (unsigned)p.kvh, (unsigned)a->batch);
  hipLaunchKernelGGL(attn_scores_kernel, chunks, dim3(256), 0, s, p);
  hipLaunchKernelGGL(attn_stats_kernel, dim3((unsigned)p.hq, (unsigned)a->batch), dim3(256), 0, s, p);
  hipLaunchKernelGGL(attn_pv_kernel, chunks, dim3(256), 0, s, p);
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)p.hq, (unsigned)a->batch), dim3(kAttnD), 0, s, p);
  return check_launch("decode_attention kernels");
}
