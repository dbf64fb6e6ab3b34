/*
 * q6moe -- C ABI of the MI355X (gfx950) packed-weight expert matmul and the
 * Q8 KV-cache gather. Plain pointers and sizes only; every device pointer is
 * HIP device memory and ``stream`` is a hipStream_t (NULL = default stream).
 *
 * Conventions
 *  - Every entry point returns 0 on success or a negative Q6MOE_ERR_* code;
 *    q6moe_last_error() then holds a message (thread-local).
 *  - Launches are stream-ordered and asynchronous; nothing synchronises.
 *  - No entry point allocates device memory: scratch space is the caller's
 *    ``workspace`` (size from the matching *_workspace_size query).
 *  - Results are deterministic: no floating-point atomics anywhere.
 *  - BF16 values are passed as uint16 bit patterns.
 *
 * Reference interfaces replaced (paths relative to the reference tree of
 * AhmadSaeedZaidi/data-synth-tpu):
 *  - q6moe_q6_matmul      kaggle/packed_q6/kernel.py:98-148  (q6_matmul)
 *  - q6moe_q6_decode      kaggle/packed_q6/kernel.py:44-62   (decode_tile, whole matrix)
 *  - q6moe_q6_pack        kaggle/packed_q6/layout.py:49-90   (pack_q6, on device)
 *  - q6moe_gguf_decode    kaggle/glm53_offload/gguf_quant.py:180-216 (dequantize_rows)
 *  - q6moe_moe_forward    kaggle/qwen38_tpu/experts.py:17-140 (expert_parallel's fn)
 *                         kaggle/qwen38_tpu/grouped_experts.py:21-163
 *  - q6moe_q8_matmul      kaggle/qwen38_tpu/compute.py:20-34    (q8_matmul, W8A8)
 *  - q6moe_kv_read        kaggle/qwen38_tpu/attention_cache.py:71-81 (read_quantized)
 *                         kaggle/qwen38_tpu/attention_cache.py:46-68 (gather_scale_plane)
 *  - q6moe_kv_quantize    kaggle/qwen38_tpu/attention_cache.py:15-23 (quantize)
 *  - q6moe_kv_write       kaggle/qwen38_tpu/attention_cache.py:26-43 (write_quantized)
 */
#ifndef Q6MOE_H
#define Q6MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q6MOE_OK 0
#define Q6MOE_ERR_INVALID (-1)     /* bad argument: shapes, sizes, alignment, dtype */
#define Q6MOE_ERR_HIP (-2)         /* a HIP runtime call or launch failed */
#define Q6MOE_ERR_UNSUPPORTED (-3) /* valid request this build does not implement */

/* dtype codes */
#define Q6MOE_F32 0
#define Q6MOE_BF16 1

/* GGUF tensor types (values of GGMLQuantizationType) */
#define Q6MOE_GGUF_F32 0
#define Q6MOE_GGUF_F16 1
#define Q6MOE_Q4_0 2
#define Q6MOE_Q4_1 3
#define Q6MOE_Q5_0 6
#define Q6MOE_Q5_1 7
#define Q6MOE_Q8_0 8
#define Q6MOE_Q4_K 12
#define Q6MOE_Q5_K 13
#define Q6MOE_Q6_K 14
#define Q6MOE_IQ4_NL 20
#define Q6MOE_GGUF_BF16 30

/* Library version (major*10000 + minor*100 + patch). */
int q6moe_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* q6moe_last_error(void);

/*
 * y[M, N] = x[M, K] @ decode(W)^T, BF16 operands, FP32 accumulation.
 * Replaces q6_matmul (kaggle/packed_q6/kernel.py:98-148).
 *   x       BF16 [M, ldx], row-major, K <= ldx
 *   data    SoA plane, ceil(N/64)*ceil(K/256)*13312 bytes (layout q6_k_soa_n64_k256_v1)
 *   scales  FP16 scale plane of the same layout (>= ceil(N/64)*ceil(K/256)*128 bytes)
 *   y       [M, ldy] of y_dtype (Q6MOE_F32 as the reference returns, or Q6MOE_BF16 = RNE)
 * Columns of x beyond K are treated as zero (the reference zero-pads x).
 */
int q6moe_q6_matmul(const uint16_t* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* data,
                    const uint8_t* scales, int64_t n, void* y, int y_dtype, int64_t ldy,
                    void* stream);

/*
 * Whole-matrix decode of a packed projection to BF16 [N, ldo] (first K columns).
 * Bit-exact RNE_bf16((d*sc)*code) (kaggle/packed_q6/kernel.py:44-62).
 */
int q6moe_q6_decode(const uint8_t* data, const uint8_t* scales, int64_t n, int64_t k,
                    uint16_t* out, int64_t ldo, void* stream);

/*
 * GGUF Q6_K rows [N, ceil(K/256), 210] -> SoA planes (kaggle/packed_q6/layout.py:49-90).
 * data: ceil(N/64)*KB*13312 bytes; scales: the 512-byte-padded plane, fully written
 * (padding and rows >= N are zero). Does not validate d (the host packer does).
 */
int q6moe_q6_pack(const uint8_t* raw, int64_t n, int64_t k, uint8_t* data, uint8_t* scales,
                  void* stream);

/*
 * dequantize_rows(raw, qtype, width) on device for every type the reference decodes:
 * Q6_K, Q5_K, Q4_K, Q8_0 (kaggle/glm53_offload/gguf_quant.py:180-216), Q4_0, Q4_1,
 * Q5_0, Q5_1, IQ4_NL (kaggle/qwen38_tpu/quant.py:15-55) and F32, F16, BF16:
 * raw [rows, ceil(width/vals), bytes] (any byte alignment)
 * -> out [rows, width] as FP32 or BF16 (RNE of the FP32 value).
 */
int q6moe_gguf_decode(const uint8_t* raw, int qtype, int64_t rows, int64_t width, void* out,
                      int out_dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Routed SwiGLU expert FFN (expert_parallel / grouped_expert_parallel).     */
/* ------------------------------------------------------------------------ */

/*
 * Expert tables of the routed FFN are unit-major, packed once from the GGUF
 * tables the reference keeps per expert ([E, bytes_per_expert] of raw GGUF
 * rows; kaggle/qwen38_tpu/parallel.py:40-87). Formats: Q6_K, Q5_K, Q4_K and
 * Q8_0 for gate/up; those or Q5_1 for down, in any pair. A unit is 16 output
 * rows x one 256-wide K block (Q6_K 3360 bytes, Q5_K 2816, Q4_K 2304, Q8_0
 * 4352, Q5_1 3072; rows and missing 32-value blocks padded with zeros); an
 * expert's units run [row group][K block]. K-quant units hold the rows' block
 * bytes in 16-byte chunks (Q6_K bit-planar: the same 6-bit codes, sub-scales
 * and FP16 scales, rearranged per decoding lane); Q8_0 and Q5_1 units hold each
 * lane's codes per 64-column chunk and then the rows' block scales (maps in
 * csrc/moe_common.h and csrc/q6moe_device.h). The repack is lossless, so
 * decoded values are those of the GGUF rows.
 */
size_t q6moe_moe_table_bytes(int qtype, int64_t rows, int64_t width); /* per expert; 0 if invalid */

/* raw [experts][rows][ceil(width/256)][210, 176 or 144] (Q6_K, Q5_K, Q4_K) or
   [experts][rows][ceil(width/32)][34 or 24] (Q8_0, Q5_1) -> dst [experts][table bytes]
   (dst 16-byte aligned). No counterpart call in the reference, whose matmul
   reads GGUF bytes directly; this is its one-time load-side preparation. */
int q6moe_moe_pack(const uint8_t* raw, int qtype, int64_t experts, int64_t rows, int64_t width,
                   uint8_t* dst, void* stream);

/*
 * Bit-exact decode probe of unit-major expert tables: table (expert e at
 * table + e * stride) -> out BF16 [experts, rows, width], each weight
 * RNE_bf16 of its GGUF value (kaggle/glm53_offload/gguf_quant.py:111-173,
 * the values dequantize_rows(..., dtype=bfloat16) gives; a Q6_K weight whose
 * code is 32 decodes to +0 whatever the sign of d*sc). ``path`` picks the
 * decoder the MoE kernels use: 0 the generic kernels' register decode, 1 the
 * decode-step kernels' LDS-staged decode, 2 the prefill kernels' whole-block
 * decode (Q6_K only). No counterpart call in the reference: it is the
 * unit-major analogue of q6moe_q6_decode, for tests of the decoders.
 */
int q6moe_moe_unpack(const uint8_t* table, int qtype, int64_t experts, int64_t rows, int64_t width,
                     int64_t stride, int path, uint16_t* out, void* stream);

/*
 * Sigmoid probe: for n BF16 inputs x, e[i] = exp(-|x[i]|) and s[i] = the FP32
 * sigmoid that the routed FFN's SwiGLU and the shared-expert gate compute,
 * where(x >= 0, 1, e) / (1 + e) (kaggle/qwen38_tpu/numerics.py:42-45), on the
 * given stream. No counterpart call in the reference: it is for tests of that
 * formula (the quotient is the correctly rounded one of the same e).
 */
int q6moe_sigmoid_probe(const uint16_t* x, int64_t n, float* e, float* s, void* stream);

/* Weight tables of one projection for all experts. */
typedef struct q6moe_table {
  int qtype;                /* gate/up: Q6MOE_Q6_K, _Q5_K, _Q4_K or _Q8_0; down: those or Q6MOE_Q5_1 */
  const uint8_t* data;      /* unit-major table of expert e at data + e * data_stride */
  int64_t data_stride;      /* bytes between experts (>= q6moe_moe_table_bytes, multiple of 16) */
  const uint8_t* scales;    /* unused (NULL): the scales live in the units */
  int64_t scale_stride;     /* unused (0) */
} q6moe_table;

typedef struct q6moe_moe_args {
  q6moe_table gate, up, down;  /* gate/up: [I rows, H], down: [H rows, I] per expert */
  int64_t experts;             /* E, 1..1024 (the reference model's layer has 512) */
  int64_t hidden;              /* H */
  int64_t intermediate;        /* I */
  const uint16_t* x;           /* BF16 [B, H] */
  const int32_t* ids;          /* [B, top_k]; ids outside [0, E) are ignored */
  const uint16_t* weights;     /* BF16 [B, top_k]; zero means no route */
  int64_t tokens;              /* B */
  int64_t top_k;               /* k */
  /* optional always-on shared expert (gate/up [Is, H], down [H, Is]); data == NULL: none */
  q6moe_table shared_gate, shared_up, shared_down;
  int64_t shared_intermediate; /* Is */
  const uint16_t* shared_scale;/* optional BF16 [B] per-token gate of the shared output; NULL = 1 */
  uint16_t* out;               /* BF16 [B, H] */
  void* workspace;             /* >= q6moe_moe_workspace_size(...) bytes, 256-byte aligned */
  size_t workspace_bytes;
  /* kernel family: 0 the decode-step kernels up to 64 tokens where they apply (and, without
     a shared expert, tokens*top_k*E < 2^17), else the grouped ones; 1 the decode-step kernels (B <= 256, B*top_k <= 1024, E <= 1024 and
     B*top_k*max(H, I, Is) < 2^30, else Q6MOE_ERR_INVALID); 2 the grouped-GEMM (prefill)
     kernels, tiled on the matrix cores for Q6_K with H and I multiples of 256 */
  int mode;
  /* optional profiling: NULL, or Q6MOE_MOE_EVENTS hipEvent_t handles recorded on ``stream``
     before routing, after routing, after gate/up, after down, after the combine; on the
     decode-step and tiled prefill paths the second and third take the gate/up kernel's own
     start and end timestamps (hipExtLaunchKernel), so that their difference is its duration */
  void* const* events;
  /* optional BF16 [H] shared-expert router (kaggle/qwen38_tpu/math.py:283): the shared
     output is scaled per token by RNE(sigmoid(RNE(x . shared_router))), computed on the
     device; NULL: shared_scale (or 1) is used. Not both. */
  const uint16_t* shared_router;
  /* expert compute policy (kaggle/qwen38_tpu/experts.py:85-101): 0 "bf16" (decoded BF16 weights,
     FP32 accumulation); 1 "int8_q8": projections whose table is Q8_0 run W8A8 as q8_matmul does
     (kaggle/qwen38_tpu/compute.py:20-34), on the grouped kernels (mode 0 or 2) */
  int compute;
} q6moe_moe_args;

#define Q6MOE_MOE_EVENTS 5

/*
 * Router (routes_and_shared's routing, kaggle/qwen38_tpu/math.py:277-281): FP32
 * softmax of logits [B, E] (E <= 1024), top_k (k <= 32; larger probability
 * first, lower expert id on ties), weights divided by their FP32 sum in
 * selection order, rows with active[b] == 0 zeroed (active NULL: all active),
 * RNE to BF16. Writes ids int32 [B, k] and weights BF16 [B, k]: the ids and
 * weights q6moe_moe_forward takes.
 */
int q6moe_route_topk(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                     const uint8_t* active, int32_t* ids, uint16_t* weights, void* stream);

size_t q6moe_moe_workspace_size(int64_t tokens, int64_t top_k, int64_t experts, int64_t hidden,
                                int64_t intermediate, int64_t shared_intermediate);

int q6moe_moe_forward(const q6moe_moe_args* args, void* stream);

/*
 * q6moe_moe_forward without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. args->workspace must
 * be NULL and args->workspace_bytes 0: the call uses the library's static
 * per-device scratch of Q6MOE_NOALLOC_SCRATCH_BYTES (32 MiB, held by each GPU
 * the library runs on until the process ends) and allocates nothing. Calls
 * whose regions (q6moe_moe_workspace_size of their shape) exceed it are
 * rejected with Q6MOE_ERR_INVALID. Every call on a GPU shares that GPU's
 * scratch: calls that overlap on one GPU (several streams or host threads)
 * race; serialise them.
 */
#define Q6MOE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int q6moe_moe_forward_noalloc(const q6moe_moe_args* args, void* stream);

/*
 * W8A8 projection of the int8_q8 policy, q8_matmul (kaggle/qwen38_tpu/compute.py:20-34):
 * y BF16 [m, n] = RNE(sum over 32-value groups g of (f32(sum_k xq[:, g, k] * w[:, g, k]) *
 * xs[:, g]) * d[:, g]) with x BF16 [m, k] quantised per row and group (xs = max|x| / 127,
 * xq = clip(rint(x / (xs ? xs : 1)), -127, 127)) and w, d the INT8 codes and FP16 scales of
 * a Q8_0 table [n rows, k] in the unit-major layout (q6moe_moe_pack, one expert), on the
 * INT8 matrix cores. k a multiple of 32; workspace >= q6moe_q8_matmul_workspace_size(m, k).
 */
size_t q6moe_q8_matmul_workspace_size(int64_t m, int64_t k);
int q6moe_q8_matmul(const uint16_t* x, int64_t m, int64_t k, const uint8_t* table, int64_t n, uint16_t* y,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* INT8 KV cache gather + dequant (read_quantized).                         */
/* ------------------------------------------------------------------------ */

typedef struct q6moe_kv_args {
  const int8_t* codes;      /* dense: [B, T, KVH*D]; paged: [pages, page_size, KVH*D] */
  const void* scales;       /* see scale_layout */
  int scale_dtype;          /* Q6MOE_BF16 (reference) or Q6MOE_F32 */
  int scale_layout;         /* 0: plane [B*G, T] (reference); 1: token-major [rows, G] */
  const int32_t* page_table;/* NULL: dense cache; else [B, pages_per_seq] */
  int64_t pool_pages;       /* pages in the pool; table entries outside [0, pool_pages) read as 0 */
  int64_t pages_per_seq;
  int64_t page_size;
  const int32_t* indices;   /* NULL: tokens 0..S-1; else [B, S] (negative adds T, then clamp) */
  int64_t batch;            /* B */
  int64_t selected;         /* S */
  int64_t capacity;         /* T (dense) -- paged: pages_per_seq * page_size */
  int64_t kv_heads;
  int64_t head_dim;
  int64_t group;            /* channels per scale; divides KVH*D */
  void* out;                /* [B, S, KVH*D] */
  int out_dtype;            /* Q6MOE_BF16 or Q6MOE_F32 (compute_cast target) */
} q6moe_kv_args;

int q6moe_kv_read(const q6moe_kv_args* args, void* stream);

/*
 * gather_scale_plane (kaggle/qwen38_tpu/attention_cache.py:46-68): the scale
 * plane [B*G, T] (BF16 or F32, values copied bitwise) at token indices [B, S]
 * (a negative index adds T, then the index is clamped into [0, T)) ->
 * out [B, S, G] of the plane's dtype.
 */
int q6moe_kv_gather_scales(const void* plane, int plane_dtype, const int32_t* indices, int64_t batch,
                           int64_t selected, int64_t groups, int64_t time, void* out, void* stream);

/*
 * INT8 block quantisation of KV rows (quantize, kaggle/qwen38_tpu/attention_cache.py:15-23):
 * x [rows, chans] (BF16 or F32 values) in groups of ``group`` channels ->
 * codes int8 [rows, chans] and scales [rows, chans/group]. With a BF16 scale,
 * scale = RNE_bf16(max|g| / 127) and the rounded scale is the divisor; with an
 * F32 scale the FP32 quotient is both. An all-zero group stores scale 0 and
 * divides by 1. codes = clip(rint(g / divisor), -127, 127).
 */
int q6moe_kv_quantize(const void* x, int x_dtype, int64_t rows, int64_t chans, int64_t group,
                      int8_t* codes, void* scales, int scale_dtype, void* stream);

/*
 * write_quantized (kaggle/qwen38_tpu/attention_cache.py:26-43): quantise row b of x
 * (one new token per sequence) and store its codes at token slot indices[b] of the
 * dense cache [B, T, KVH*D] (page_table NULL) or of the paged pool [pages, P, KVH*D],
 * and its scales in the plane [B*G, T] (scale_layout 0, dense only) or token-major
 * [rows, G] (scale_layout 1). Rows with active[b] == 0 are left unchanged. A slot
 * index below zero adds T; slots outside [0, T) and unmapped pages are not written
 * (JAX scatter drops out-of-bounds updates).
 */
typedef struct q6moe_kv_write_args {
  const void* x;            /* [B, KVH*D] */
  int x_dtype;              /* Q6MOE_BF16 or Q6MOE_F32 */
  int8_t* codes;            /* dense: [B, T, KVH*D]; paged: [pages, page_size, KVH*D] */
  void* scales;             /* see scale_layout */
  int scale_dtype;          /* Q6MOE_BF16 (reference) or Q6MOE_F32 */
  int scale_layout;         /* 0: plane [B*G, T]; 1: token-major [rows, G] */
  const int32_t* page_table;/* NULL: dense cache; else [B, pages_per_seq] */
  int64_t pool_pages;
  int64_t pages_per_seq;
  int64_t page_size;
  const int32_t* indices;   /* [B] token slot per row */
  const uint8_t* active;    /* [B] nonzero: write the row; NULL: every row */
  int64_t batch;            /* B */
  int64_t capacity;         /* T (dense) -- paged: pages_per_seq * page_size */
  int64_t kv_heads;
  int64_t head_dim;
  int64_t group;            /* channels per scale; divides KVH*D */
} q6moe_kv_write_args;

int q6moe_kv_write(const q6moe_kv_write_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Decode attention over the paged INT8 KV cache.                           */
/* ------------------------------------------------------------------------ */

/*
 * The core of the reference's decode attention step (kaggle/qwen38_tpu/
 * attention_cache.py:159-169: scores of the query against read_quantized keys,
 * RNE to BF16, divided by sqrt(D), RNE; numerics.softmax over the attended
 * tokens; RNE_bf16(prob) times read_quantized values with FP32 accumulation;
 * RNE to BF16), with the dequant fused in: no BF16 copy of K or V is written.
 * Replaces read_quantized(k), read_quantized(v) and the two einsums around
 * the softmax for one query token per sequence; the output gate and the out
 * projection stay with the caller. Paged cache, FP32 scale per token and KV
 * head (group = head_dim), head_dim 128, up to 8 query heads per KV head.
 * The reference's mask ``indices <= lengths`` is lengths[b] = position + 1
 * attended tokens here (tokens 0 .. lengths[b]-1; clamped into [1, capacity]).
 */
typedef struct q6moe_attn_args {
  const uint16_t* q;          /* BF16 [B, Hq, 128] */
  const int8_t* k_codes;      /* [pool_pages, page_size, KVH*128] */
  const int8_t* v_codes;
  const float* k_scales;      /* FP32 [pool_pages*page_size, KVH] */
  const float* v_scales;
  const int32_t* page_table;  /* [B, pages_per_seq]; entries outside [0, pool_pages) read as 0 */
  const int32_t* lengths;     /* [B] attended tokens */
  int64_t batch, query_heads, kv_heads, head_dim, pool_pages, pages_per_seq, page_size;
  uint16_t* out;              /* BF16 [B, Hq, 128] */
  void* workspace;            /* >= q6moe_attn_workspace_size(...) bytes, 256-byte aligned */
  size_t workspace_bytes;
} q6moe_attn_args;

size_t q6moe_attn_workspace_size(int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t pages_per_seq,
                                 int64_t page_size);
int q6moe_kv_decode_attention(const q6moe_attn_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q6MOE_H */
