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

// Cache row of (sequence b, token t) or -1 for an unmapped page. Idx is the
// integer type of the index arithmetic (32-bit when every offset fits).
template <typename Idx>
__device__ __forceinline__ Idx kv_row(const KvParams& p, Idx b, Idx s, Idx* tok) {
  const Idx cap = (Idx)p.cap;
  int64_t t64 = p.indices ? (int64_t)p.indices[(int64_t)b * p.sel + s] : (int64_t)s;
  if (t64 < 0) t64 += p.cap;
  t64 = t64 < 0 ? 0 : (t64 >= p.cap ? p.cap - 1 : t64);
  const Idx t = (Idx)t64;
  *tok = t;
  if (!p.table) return b * cap + t;
  const Idx page = (Idx)p.page;
  const int64_t pg = p.table[(int64_t)b * p.pps + t / page];
  if (pg < 0 || pg >= p.pool_pages) return (Idx)-1;
  return (Idx)pg * page + t % page;
}

template <typename Idx>
__device__ __forceinline__ float kv_scale(const KvParams& p, Idx b, Idx t, Idx row, Idx g) {
  const Idx groups = (Idx)p.groups;
  const Idx idx = p.scale_plane ? (b * groups + g) * (Idx)p.cap + t : row * groups + g;
  return p.scale_bf16 ? bf16_to_float(reinterpret_cast<const uint16_t*>(p.scales)[idx])
                      : reinterpret_cast<const float*>(p.scales)[idx];
}

// Vector path: chans % 16 == 0, group % 16 == 0, 16-byte aligned rows.
template <typename Idx>
__global__ void __launch_bounds__(256) kv_read_vec_kernel(KvParams p, int64_t units) {
  const int64_t u64 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u64 >= units) return;
  const Idx u = (Idx)u64;
  const Idx per_row = (Idx)(p.chans / 16);
  const Idx rs = u / per_row;  // (b, s) flattened
  const Idx c = (u - rs * per_row) * 16;
  const Idx sel = (Idx)p.sel;
  const Idx b = rs / sel, s = rs - b * sel;
  Idx t;
  const Idx row = kv_row<Idx>(p, b, s, &t);
  u32x4 codes = {0u, 0u, 0u, 0u};
  float sc = 0.f;
  if (row != (Idx)-1) {
    codes = ld16_stream(p.codes + (int64_t)row * p.chans + c);
    sc = kv_scale<Idx>(p, b, t, row, c / (Idx)p.group);
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
    uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + (int64_t)rs * p.chans + c;
    __builtin_nontemporal_store(o0, reinterpret_cast<u32x4*>(o));
    __builtin_nontemporal_store(o1, reinterpret_cast<u32x4*>(o + 8));
  } else {
    float* o = reinterpret_cast<float*>(p.out) + (int64_t)rs * p.chans + c;
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
  const int64_t row = kv_row<int64_t>(p, b, s, &t);
  float v = 0.f;
  if (row >= 0) v = (float)p.codes[row * p.chans + c] * kv_scale<int64_t>(p, b, t, row, c / p.group);
  if (p.out_bf16)
    reinterpret_cast<uint16_t*>(p.out)[i] = bf16_bits(v);
  else
    reinterpret_cast<float*>(p.out)[i] = v;
}

// ---------------------------------------------------------------------------
// Quantise and write (quantize / write_quantized, attention_cache.py:15-43).
// One thread per (row, group): max|g|, the scale, then the group's codes.
// ---------------------------------------------------------------------------
struct KvQuant {
  const void* x;
  int x_bf16;
  int64_t chans, group, groups;
  int scale_bf16;
};

__device__ __forceinline__ float kv_x(const KvQuant& q, int64_t i) {
  return q.x_bf16 ? bf16_to_float(reinterpret_cast<const uint16_t*>(q.x)[i])
                  : reinterpret_cast<const float*>(q.x)[i];
}

// Quantise group g of row r into codes (chans-strided destination) and
// return the stored scale value (FP32 holding the BF16 or FP32 scale).
__device__ __forceinline__ float kv_quant_group(const KvQuant& q, int64_t r, int64_t g, int8_t* dst) {
  const int64_t base = r * q.chans + g * q.group;
  float m = 0.f;
  for (int64_t c = 0; c < q.group; ++c) m = fmaxf(m, fabsf(kv_x(q, base + c)));
  float scale = m / 127.f;
  if (q.scale_bf16) scale = bf16_round(scale);
  const float divisor = scale == 0.f ? 1.f : scale;
  for (int64_t c = 0; c < q.group; ++c) {
    float v = __builtin_rintf(kv_x(q, base + c) / divisor);
    v = fminf(fmaxf(v, -127.f), 127.f);
    dst[c] = (int8_t)(int)v;
  }
  return scale;
}

__device__ __forceinline__ void kv_store_scale(void* scales, int bf16, int64_t idx, float v) {
  if (bf16)
    reinterpret_cast<uint16_t*>(scales)[idx] = bf16_bits(v);
  else
    reinterpret_cast<float*>(scales)[idx] = v;
}

__global__ void __launch_bounds__(256) kv_quantize_kernel(KvQuant q, int64_t rows, int8_t* codes, void* scales) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * q.groups) return;
  const int64_t r = i / q.groups, g = i % q.groups;
  const float s = kv_quant_group(q, r, g, codes + r * q.chans + g * q.group);
  kv_store_scale(scales, q.scale_bf16, i, s);
}

struct KvWrite {
  int8_t* codes;
  void* scales;
  int scale_plane;
  const int32_t* table;
  int64_t pool_pages, pps, page, cap;
  const int32_t* indices;
  const uint8_t* active;
};

__global__ void __launch_bounds__(256) kv_write_kernel(KvQuant q, KvWrite w, int64_t batch) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= batch * q.groups) return;
  const int64_t b = i / q.groups, g = i % q.groups;
  if (w.active && !w.active[b]) return;
  int64_t t = w.indices[b];
  if (t < 0) t += w.cap;
  if (t < 0 || t >= w.cap) return;  // out-of-bounds scatter updates are dropped
  int64_t row = b * w.cap + t;
  if (w.table) {
    const int64_t pg = w.table[b * w.pps + t / w.page];
    if (pg < 0 || pg >= w.pool_pages) return;
    row = pg * w.page + t % w.page;
  }
  const float s = kv_quant_group(q, b, g, w.codes + row * q.chans + g * q.group);
  const int64_t idx = w.scale_plane ? (b * q.groups + g) * w.cap + t : row * q.groups + g;
  kv_store_scale(w.scales, q.scale_bf16, idx, s);
}

// gather_scale_plane (kaggle/qwen38_tpu/attention_cache.py:46-68): plane
// [B*G, T] (2- or 4-byte values, copied bitwise), indices [B, S] (negative adds
// T, then clamp, as a JAX gather) -> out [B, S, G]. One thread per output.
template <typename V>
__global__ void __launch_bounds__(256)
    kv_gather_scales_kernel(const V* __restrict__ plane, const int32_t* __restrict__ idx, int64_t sel,
                            int64_t groups, int64_t time, int64_t n, V* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t g = i % groups, bs = i / groups, b = bs / sel;
  int64_t t = idx[bs];
  if (t < 0) t += time;
  t = t < 0 ? 0 : (t >= time ? time - 1 : t);
  out[i] = plane[(b * groups + g) * time + t];
}

}  // namespace q6moe

using namespace q6moe;

extern "C" int q6moe_kv_gather_scales(const void* plane, int plane_dtype, const int32_t* indices, int64_t batch,
                                      int64_t selected, int64_t groups, int64_t time, void* out, void* stream) {
  Q6MOE_REQUIRE(plane && indices && out, "kv_gather_scales: null pointer");
  Q6MOE_REQUIRE(plane_dtype == Q6MOE_BF16 || plane_dtype == Q6MOE_F32, "kv_gather_scales: plane must be BF16 or F32");
  Q6MOE_REQUIRE(batch >= 1 && selected >= 0 && groups >= 1 && time >= 1, "kv_gather_scales: bad shape");
  const int64_t n = batch * selected * groups;
  if (n == 0) return Q6MOE_OK;
  const dim3 grid((unsigned)cdiv(n, 256));
  if (plane_dtype == Q6MOE_BF16)
    hipLaunchKernelGGL(kv_gather_scales_kernel<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const uint16_t*>(plane), indices, selected, groups, time, n,
                       reinterpret_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(kv_gather_scales_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const float*>(plane), indices, selected, groups, time, n,
                       reinterpret_cast<float*>(out));
  return check_launch("kv_gather_scales_kernel");
}

extern "C" int q6moe_kv_quantize(const void* x, int x_dtype, int64_t rows, int64_t chans, int64_t group,
                                 int8_t* codes, void* scales, int scale_dtype, void* stream) {
  Q6MOE_REQUIRE(x && codes && scales, "kv_quantize: null pointer");
  Q6MOE_REQUIRE(rows >= 1 && chans >= 1 && group >= 1 && chans % group == 0,
                "kv_quantize: rows, chans must be positive and group must divide chans");
  Q6MOE_REQUIRE(x_dtype == Q6MOE_BF16 || x_dtype == Q6MOE_F32, "kv_quantize: x dtype");
  Q6MOE_REQUIRE(scale_dtype == Q6MOE_BF16 || scale_dtype == Q6MOE_F32, "kv_quantize: scale dtype");
  KvQuant q{x, x_dtype == Q6MOE_BF16, chans, group, chans / group, scale_dtype == Q6MOE_BF16};
  const int64_t n = rows * q.groups;
  hipLaunchKernelGGL(kv_quantize_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, q,
                     rows, codes, scales);
  return check_launch("kv_quantize");
}

extern "C" int q6moe_kv_write(const q6moe_kv_write_args* a, void* stream) {
  Q6MOE_REQUIRE(a, "kv_write: null args");
  Q6MOE_REQUIRE(a->x && a->codes && a->scales && a->indices, "kv_write: null pointer");
  Q6MOE_REQUIRE(a->batch >= 1 && a->kv_heads >= 1 && a->head_dim >= 1,
                "kv_write: batch, kv_heads and head_dim must be positive");
  const int64_t chans = a->kv_heads * a->head_dim;
  Q6MOE_REQUIRE(a->group >= 1 && chans % a->group == 0, "kv_write: group must divide kv_heads*head_dim");
  Q6MOE_REQUIRE(a->x_dtype == Q6MOE_BF16 || a->x_dtype == Q6MOE_F32, "kv_write: x dtype");
  Q6MOE_REQUIRE(a->scale_dtype == Q6MOE_BF16 || a->scale_dtype == Q6MOE_F32, "kv_write: scale dtype");
  Q6MOE_REQUIRE(a->scale_layout == 0 || a->scale_layout == 1, "kv_write: scale layout");
  KvWrite w;
  w.codes = a->codes;
  w.scales = a->scales;
  w.scale_plane = a->scale_layout == 0;
  w.table = a->page_table;
  w.pool_pages = a->pool_pages;
  w.pps = a->pages_per_seq;
  w.page = a->page_size;
  w.indices = a->indices;
  w.active = a->active;
  if (a->page_table) {
    Q6MOE_REQUIRE(a->pages_per_seq >= 1 && a->page_size >= 1 && a->pool_pages >= 1,
                  "kv_write: paged cache needs pages_per_seq, page_size, pool_pages >= 1");
    Q6MOE_REQUIRE(a->scale_layout == 1, "kv_write: paged cache uses token-major scales");
    w.cap = a->pages_per_seq * a->page_size;
  } else {
    Q6MOE_REQUIRE(a->capacity >= 1, "kv_write: capacity must be positive");
    w.cap = a->capacity;
  }
  KvQuant q{a->x, a->x_dtype == Q6MOE_BF16, chans, a->group, chans / a->group, a->scale_dtype == Q6MOE_BF16};
  const int64_t n = a->batch * q.groups;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, q, w,
                     a->batch);
  return check_launch("kv_write");
}

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
    // 32-bit index arithmetic when every element offset and cache row fits
    const int64_t rows = a->page_table ? a->pool_pages * a->page_size : a->batch * p.cap;
    const bool small = total < (1ll << 31) && rows * chans < (1ll << 31) &&
                       a->batch * p.groups * p.cap < (1ll << 31);
    if (small)
      hipLaunchKernelGGL(kv_read_vec_kernel<uint32_t>, dim3((unsigned)cdiv(units, 256)), dim3(256), 0, s, p, units);
    else
      hipLaunchKernelGGL(kv_read_vec_kernel<int64_t>, dim3((unsigned)cdiv(units, 256)), dim3(256), 0, s, p, units);
  } else {
    hipLaunchKernelGGL(kv_read_scalar_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, p, total);
  }
  return check_launch("kv_read");
}
