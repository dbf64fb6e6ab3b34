// INT8 KV-cache gather + dequant: out = RNE(f32(code) * f32(scale)).
//
// Replaces read_quantized / gather_scale_plane (kaggle/qwen38_tpu/attention_cache.py:46-81)
// for the reference's dense cache ([B, T, KVH*D] codes, BF16 scale plane
// [B*G, T]) and for a paged pool ([pages, P, KVH*D] codes, token-major FP32
// scales, per-sequence page tables). Token indices follow JAX gather rules:
// a negative index adds T, then the index is clamped into [0, T).
//
// HBM-bound: one thread moves 16 codes (one 16-byte load) and writes 16 BF16
// (two 16-byte non-temporal stores); a 256-thread block covers 256*16 channels.
#include "q6moe_api.h"
#include "q6moe_device.h"

namespace q6moe {

struct KvParams {
  const int8_t* codes;
  const void* scales;
  int scale_bf16;
  int scale_plane;
  const int32_t* table;
  int64_t pool_pages, pps, page;
  const int32_t* indices;
  int64_t batch, sel, cap, chans, groups, group;
  void* out;
  int out_bf16;
};

// Cache row of (sequence b, token t) or -1 for an unmapped page.
__device__ __forceinline__ int64_t kv_row(const KvParams& p, int64_t b, int64_t s, int64_t* tok) {
  int64_t t = p.indices ? (int64_t)p.indices[b * p.sel + s] : s;
  if (t < 0) t += p.cap;
  t = t < 0 ? 0 : (t >= p.cap ? p.cap - 1 : t);
  *tok = t;
  if (!p.table) return b * p.cap + t;
  const int64_t pg = p.table[b * p.pps + t / p.page];
  if (pg < 0 || pg >= p.pool_pages) return -1;
  return pg * p.page + t % p.page;
}

__device__ __forceinline__ float kv_scale(const KvParams& p, int64_t b, int64_t t, int64_t row, int64_t g) {
  const int64_t idx = p.scale_plane ? (b * p.groups + g) * p.cap + t : row * p.groups + g;
  return p.scale_bf16 ? bf16_to_float(reinterpret_cast<const uint16_t*>(p.scales)[idx])
                      : reinterpret_cast<const float*>(p.scales)[idx];
}

// Vector path: chans % 16 == 0, group % 16 == 0, 16-byte aligned rows.
__global__ void __launch_bounds__(256) kv_read_vec_kernel(KvParams p, int64_t units) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int64_t per_row = p.chans / 16;
  const int64_t rs = u / per_row;  // (b, s) flattened
  const int64_t c = (u % per_row) * 16;
  const int64_t b = rs / p.sel, s = rs % p.sel;
  int64_t t;
  const int64_t row = kv_row(p, b, s, &t);
  u32x4 codes = {0u, 0u, 0u, 0u};
  float sc = 0.f;
  if (row >= 0) {
    codes = ld16_stream(p.codes + row * p.chans + c);
    sc = kv_scale(p, b, t, row, c / p.group);
  }
  if (p.out_bf16) {
    u32x4 o0, o1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = codes[i];
      const float v0 = (float)(int8_t)(w & 0xff) * sc, v1 = (float)(int8_t)((w >> 8) & 0xff) * sc;
      const float v2 = (float)(int8_t)((w >> 16) & 0xff) * sc, v3 = (float)(int8_t)(w >> 24) * sc;
      if (i < 2) {
        o0[2 * i] = pack_bf16x2(v0, v1);
        o0[2 * i + 1] = pack_bf16x2(v2, v3);
      } else {
        o1[2 * (i - 2)] = pack_bf16x2(v0, v1);
        o1[2 * (i - 2) + 1] = pack_bf16x2(v2, v3);
      }
    }
    uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + rs * p.chans + c;
    __builtin_nontemporal_store(o0, reinterpret_cast<u32x4*>(o));
    __builtin_nontemporal_store(o1, reinterpret_cast<u32x4*>(o + 8));
  } else {
    float* o = reinterpret_cast<float*>(p.out) + rs * p.chans + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = codes[i];
      f32x4 v = {(float)(int8_t)(w & 0xff) * sc, (float)(int8_t)((w >> 8) & 0xff) * sc,
                 (float)(int8_t)((w >> 16) & 0xff) * sc, (float)(int8_t)(w >> 24) * sc};
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(o + 4 * i));
    }
  }
}

// Scalar path for any shape: one thread per output element.
__global__ void kv_read_scalar_kernel(KvParams p, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t rs = i / p.chans, c = i % p.chans;
  const int64_t b = rs / p.sel, s = rs % p.sel;
  int64_t t;
  const int64_t row = kv_row(p, b, s, &t);
  float v = 0.f;
  if (row >= 0) v = (float)p.codes[row * p.chans + c] * kv_scale(p, b, t, row, c / p.group);
  if (p.out_bf16)
    reinterpret_cast<uint16_t*>(p.out)[i] = bf16_bits(v);
  else
    reinterpret_cast<float*>(p.out)[i] = v;
}

}  // namespace q6moe

using namespace q6moe;

extern "C" int q6moe_kv_read(const q6moe_kv_args* a, void* stream) {
  Q6MOE_REQUIRE(a, "kv_read: null args");
  Q6MOE_REQUIRE(a->codes && a->scales && a->out, "kv_read: null pointer");
  Q6MOE_REQUIRE(a->batch >= 1 && a->selected >= 1 && a->kv_heads >= 1 && a->head_dim >= 1,
                "kv_read: batch, selected, kv_heads and head_dim must be positive");
  const int64_t chans = a->kv_heads * a->head_dim;
  Q6MOE_REQUIRE(a->group >= 1 && chans % a->group == 0, "kv_read: group must divide kv_heads*head_dim");
  Q6MOE_REQUIRE(a->scale_dtype == Q6MOE_BF16 || a->scale_dtype == Q6MOE_F32, "kv_read: scale dtype");
  Q6MOE_REQUIRE(a->out_dtype == Q6MOE_BF16 || a->out_dtype == Q6MOE_F32, "kv_read: out dtype");
  Q6MOE_REQUIRE(a->scale_layout == 0 || a->scale_layout == 1, "kv_read: scale layout");
  KvParams p;
  p.codes = a->codes;
  p.scales = a->scales;
  p.scale_bf16 = a->scale_dtype == Q6MOE_BF16;
  p.scale_plane = a->scale_layout == 0;
  p.table = a->page_table;
  p.pool_pages = a->pool_pages;
  p.pps = a->pages_per_seq;
  p.page = a->page_size;
  p.indices = a->indices;
  p.batch = a->batch;
  p.sel = a->selected;
  p.chans = chans;
  p.group = a->group;
  p.groups = chans / a->group;
  p.out = a->out;
  p.out_bf16 = a->out_dtype == Q6MOE_BF16;
  if (a->page_table) {
    Q6MOE_REQUIRE(a->pages_per_seq >= 1 && a->page_size >= 1 && a->pool_pages >= 1,
                  "kv_read: paged cache needs pages_per_seq, page_size, pool_pages >= 1");
    Q6MOE_REQUIRE(a->scale_layout == 1, "kv_read: paged cache uses token-major scales");
    p.cap = a->pages_per_seq * a->page_size;
  } else {
    Q6MOE_REQUIRE(a->capacity >= 1, "kv_read: capacity must be positive");
    p.cap = a->capacity;
  }
  Q6MOE_REQUIRE(a->indices || a->selected <= p.cap, "kv_read: selected exceeds capacity without indices");
  hipStream_t s = (hipStream_t)stream;
  const int64_t total = a->batch * a->selected * chans;
  const bool vec = chans % 16 == 0 && a->group % 16 == 0 && aligned(a->codes, 16) && aligned(a->out, 16);
  if (vec) {
    const int64_t units = total / 16;
    hipLaunchKernelGGL(kv_read_vec_kernel, dim3((unsigned)cdiv(units, 256)), dim3(256), 0, s, p, units);
  } else {
    hipLaunchKernelGGL(kv_read_scalar_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, p, total);
  }
  return check_launch("kv_read");
}
