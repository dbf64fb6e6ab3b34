// Router: FP32 softmax of the logits -> top_k -> weights divided by their sum
// -> inactive rows zeroed -> RNE to BF16 (kaggle/qwen38_tpu/math.py:277-281,
// routes_and_shared without the shared expert; numerics.py:48-51 softmax).
//
// One wave per token row, up to 1024 experts (S = 4 logits per lane up to 256
// experts, 16 above). The softmax
// sum and the top-k selection are wave reductions in a fixed order; top_k
// picks the largest probability, the lower expert id on ties (jax.lax.top_k),
// one selection round per k; the selected probabilities are summed in
// selection order.
#include "moe_common.h"
#include "q6moe_api.h"

namespace q6moe {

constexpr int kRouterMaxExperts = kMaxExperts;
constexpr int kRouterMaxTopK = 32;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int S>
__global__ void __launch_bounds__(256) router_topk_kernel(const float* __restrict__ logits, int B, int E, int K,
                                                          const uint8_t* __restrict__ active,
                                                          int32_t* __restrict__ ids, uint16_t* __restrict__ wts) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const float* x = logits + (int64_t)row * E;
  // expert of slot q of this lane: lane + 64q
  float v[S];
  float m = -__builtin_inff();
#pragma unroll
  for (int q = 0; q < S; ++q) {
    const int e = lane + 64 * q;
    v[q] = e < E ? x[e] : -__builtin_inff();
    m = fmaxf(m, v[q]);
  }
  m = wave_max(m);
  float part = 0.f;
#pragma unroll
  for (int q = 0; q < S; ++q) {
    v[q] = lane + 64 * q < E ? expf(v[q] - m) : 0.f;
    part += v[q];
  }
  const float total = wave_sum(part);
  float pr[S];
#pragma unroll
  for (int q = 0; q < S; ++q) pr[q] = lane + 64 * q < E ? v[q] / total : -1.f;  // probabilities are >= 0
  // top_k: one round per selection; (probability desc, id asc)
  float sel_p = 0.f, sum = 0.f;
  int sel_e = 0;
  for (int k = 0; k < K; ++k) {
    float bp = -2.f;
    int be = 1 << 30;
#pragma unroll
    for (int q = 0; q < S; ++q)
      if (pr[q] > bp) {  // slots ascend in id, so the first maximum has the lowest id
        bp = pr[q];
        be = lane + 64 * q;
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float op = __shfl_xor(bp, off);
      const int oe = __shfl_xor(be, off);
      if (op > bp || (op == bp && oe < be)) {
        bp = op;
        be = oe;
      }
    }
    // retire the selected expert on its lane
#pragma unroll
    for (int q = 0; q < S; ++q)
      if (lane + 64 * q == be) pr[q] = -1.f;
    sum += bp;  // selection order, FP32
    if (lane == k) {
      sel_p = bp;
      sel_e = be;
    }
  }
  if (lane < K) {
    const bool on = !active || active[row];
    const float w = on ? sel_p / sum : 0.f;
    ids[(int64_t)row * K + lane] = sel_e;
    wts[(int64_t)row * K + lane] = bf16_bits(w);
  }
}

}  // namespace q6moe

using namespace q6moe;

extern "C" int q6moe_route_topk(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                                const uint8_t* active, int32_t* ids, uint16_t* weights, void* stream) {
  Q6MOE_REQUIRE(logits && ids && weights, "route_topk: null pointer");
  Q6MOE_REQUIRE(tokens >= 1 && tokens <= (1 << 26) && experts >= 1 && experts <= kRouterMaxExperts,
                "route_topk: 1 <= experts <= 1024");
  Q6MOE_REQUIRE(top_k >= 1 && top_k <= experts && top_k <= kRouterMaxTopK, "route_topk: 1 <= top_k <= min(experts, 32)");
  const dim3 grid((unsigned)((tokens + 3) / 4));
  if (experts <= 256)
    hipLaunchKernelGGL(router_topk_kernel<4>, grid, dim3(256), 0, (hipStream_t)stream, logits, (int)tokens,
                       (int)experts, (int)top_k, active, ids, weights);
  else
    hipLaunchKernelGGL(router_topk_kernel<kRouterMaxExperts / 64>, grid, dim3(256), 0, (hipStream_t)stream, logits,
                       (int)tokens, (int)experts, (int)top_k, active, ids, weights);
  return check_launch("route_topk kernel");
}
