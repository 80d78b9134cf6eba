/*
 * alloy_amd — C ABI of the MI355X (gfx950) quantized-weight matmul library.
 *
 * Drop-in boundary for Alloy's quantized-linear operator surface.  Each named
 * entry point replaces one `torch.ops.alloy.*` custom op of the reference
 * (schemas at packages/alloy-torch/src/alloy_torch/custom_ops.py, cited per
 * function below); the Python package binds these through ctypes and registers
 * the same op names.
 *
 * Conventions
 *   - Every pointer is a DEVICE pointer owned by the caller; the library never
 *     allocates device memory.  Its only state is a per-process cache of device
 *     attributes (CU count per device; resident workgroups per device, kernel and
 *     launch shape), filled on first use under a mutex, and the static scratch
 *     array of alloy_gguf_moe_routed_noalloc; results never depend on earlier calls.
 *   - `stream` is a hipStream_t (NULL = default stream); all work is enqueued on
 *     it, asynchronously.  Calls are reentrant; concurrent calls on different
 *     streams do not interact.
 *   - Outputs are fully overwritten (no pre-zeroing needed).  Results are
 *     deterministic: no floating-point atomics anywhere.
 *   - Row-major everywhere: activations x[M,K], output y[M,N], weight row n
 *     holds K elements.  Weight buffers must be 16-byte aligned.
 *   - On failure a status != ALLOY_OK is returned and alloy_last_error() holds a
 *     thread-local message.  Status -> Python exception mapping mirrors the
 *     reference's validation (packages/alloy-server/src/alloy_server/gguf/quant.py:81-105,
 *     230-249; packages/alloy-server/src/alloy_server/mlx/quant.py:88-109).
 */
#ifndef ALLOY_AMD_H
#define ALLOY_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  ALLOY_OK = 0,
  ALLOY_E_SHAPE = 1,       /* ValueError: shape / divisibility */
  ALLOY_E_DTYPE = 2,       /* TypeError: unsupported dtype code */
  ALLOY_E_ALIGN = 3,       /* ValueError: pointer alignment */
  ALLOY_E_UNSUPPORTED = 4, /* NotImplementedError: unsupported format / size */
  ALLOY_E_HIP = 5,         /* RuntimeError: HIP launch / runtime failure */
  ALLOY_E_ARG = 6          /* ValueError: bad argument (null pointer, bad enum) */
} alloy_status;

typedef enum {
  ALLOY_FMT_Q8_0 = 0,      /* GGUF wire blocks, 34 B / 32 weights */
  ALLOY_FMT_Q5_0 = 1,      /* GGUF wire blocks, 22 B / 32 weights */
  ALLOY_FMT_Q4_K = 2,      /* GGUF wire blocks, 144 B / 256 weights */
  ALLOY_FMT_Q6_K = 3,      /* GGUF wire blocks, 210 B / 256 weights */
  ALLOY_FMT_MLX_Q4 = 4,    /* MLX affine 4-bit: qweight u8[N,K/2], fp16 scales/biases [N,K/gs] */
  ALLOY_FMT_Q8_0_SPLIT = 5,/* reference loader layout: int8 qweight[N,K] + fp16 scales[N,K/32] */
  ALLOY_FMT_Q5_0_SPLIT = 6 /* reference loader layout: u8 qweight[N,K/2] + u8 qhigh[N,K/2] + fp16 scales[N,K/32] */
} alloy_format;

typedef enum { ALLOY_DT_F32 = 0, ALLOY_DT_F16 = 1 } alloy_dtype;

/* Gate activation of the fused gated pair: silu(v) = v / (1 + exp(-v)); gelu in the
 * tanh form 0.5 v (1 + tanh(clamp(sqrt(2/pi) (v + 0.044715 v^3), -10, 10)))
 * (packages/alloy-metal/src/alloy/_compiler/trace/__init__.py:432-450). */
typedef enum { ALLOY_ACT_SILU = 0, ALLOY_ACT_GELU_TANH = 1 } alloy_act;

typedef enum {
  ALLOY_PATH_AUTO = 0,      /* M==1 -> GEMV (v_dot2); M<=16 -> MFMA GEMV; else MFMA GEMM */
  ALLOY_PATH_GEMV = 1,      /* v_dot2 GEMV, one x row per grid row (any M) */
  ALLOY_PATH_GEMV_MFMA = 2, /* MFMA GEMV, 16 x rows per column tile (any M) */
  ALLOY_PATH_GEMM = 3       /* MFMA GEMM with fp16-in-LDS dequant (any M) */
} alloy_path;

/*
 * Generic quantized matmul: y[M,N] = x[M,K] @ dequant(w)[N,K]^T.
 *   w, scales, biases, aux: the format's buffers (unused ones may be NULL):
 *     GGUF wire formats: w = blocks[N, K/QK*block_bytes]
 *     MLX_Q4:            w = qweight, scales, biases, group_size
 *     Q8_0_SPLIT:        w = qweight (int8), scales
 *     Q5_0_SPLIT:        w = qweight, aux = qhigh, scales
 *   `opts` packs launch knobs for tuning (0 = automatic): bits 0-11 threads per
 *   row of the v_dot2 GEMV (multiple of 16, 16..256), bits 12-27 its grid cap,
 *   bits 28-31 MFMA GEMV row groups, bits 32-35 rows of weights in flight per
 *   thread of the v_dot2 GEMV (2, 3 or 4; for the LDS-staged rows at M = 1: 1 the
 *   four-row tile, 2 / 4 the tile ring with two / four tiles in flight), bits 36-39
 *   the kernel variant (0 automatic).  GEMV: 1 register ring with an LDS row
 *   combine, 2 LDS-staged row tiles, 3 wave rows with buffer loads and DPP
 *   reductions, 4 rows staged through LDS by aligned 16-byte loads (Q6_K, Q5_0,
 *   Q8_0, Q4_K wire blocks).  MFMA GEMV
 *   (M <= 16): 1 16x16x32 tiles, 5 Q4_K 4x4x4 broadcast tiles, 6 Q4_K x-stationary
 *   tiles, 7 x-stationary tiles of any format that has them, 8 x-stationary tiles
 *   with the weights dequantised to fp16 before the MFMA (Q4_K, Q6_K, MLX), 9 the
 *   LDS-staged rows of variant 4 for up to 8 rows of x.  GEMM: 1 generic
 *   128x128 tiles, 4 / 5 / 6 / 7 / 8 Q4_K tiles of 256x256 / 128x256 / 128x128 /
 *   64x256 / 64x128; bits 40-43 K splits for such a forced Q4_K tile (dividing K/256
 *   with at least two super-blocks each; needs a workspace of splits*M*N*4 bytes,
 *   else unsplit).
 * No reference counterpart as a single op: the reference dispatches per format
 * (packages/alloy-torch/src/alloy_torch/ops/linalg.py:346-739); the named entry
 * points below are the per-op replacements and all route here.
 */
alloy_status alloy_qmm(alloy_format fmt, const void* w, const void* aux, const void* scales,
                       const void* biases, int32_t group_size, const void* x, alloy_dtype x_dtype,
                       void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                       alloy_path path, int64_t opts, void* stream);

/*
 * alloy_qmm with a caller workspace: when the Q4_K prefill GEMM would leave CUs idle
 * (few output tiles, e.g. M = 512), or an M <= 16 product on the x-stationary kernels
 * has few row tiles over a long K, K is split into S slices whose fp32 partial
 * products go to ws (S*M*N*4 bytes, 16-byte aligned; y 16-byte aligned for fp32
 * output, 8-byte for fp16; M*N a multiple of 4) and are summed in slice order
 * (deterministic).  ws = NULL or too small: no split.  alloy_gemm_workspace_bytes()
 * returns the bytes the plan wants for this shape (0 when it does not split).  No
 * reference counterpart (the reference has no K split); for callers that can
 * provide scratch memory.
 */
int64_t alloy_gemm_workspace_bytes(alloy_format fmt, int64_t M, int64_t N, int64_t K);
alloy_status alloy_qmm_ws(alloy_format fmt, const void* w, const void* aux, const void* scales,
                          const void* biases, int32_t group_size, const void* x, alloy_dtype x_dtype,
                          void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                          alloy_path path, int64_t opts, void* ws, int64_t ws_bytes, void* stream);

/* torch.ops.alloy.gguf_q4_k_mm(activations, blocks) — custom_ops.py:47-49 */
alloy_status alloy_gguf_q4_k_mm(const void* x, alloy_dtype x_dtype, const void* blocks, void* y,
                                alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* torch.ops.alloy.gguf_q6_k_mm(activations, packed_weights) — custom_ops.py:96 */
alloy_status alloy_gguf_q6_k_mm(const void* x, alloy_dtype x_dtype, const void* packed_weights,
                                void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                                void* stream);

/* torch.ops.alloy.gguf_q8_0_mm(activations, qweight, scales) — custom_ops.py:104
 * (the reference's split layout: int8 qweight[N,K], fp16 scales[N,K/32]) */
alloy_status alloy_gguf_q8_0_mm(const void* x, alloy_dtype x_dtype, const void* qweight,
                                const void* scales, void* y, alloy_dtype y_dtype, int64_t M,
                                int64_t N, int64_t K, void* stream);

/* torch.ops.alloy.gguf_q5_0_mm(activations, qweight, qhigh, scales) — custom_ops.py:86-88
 * (the reference's split layout, packages/alloy-server/src/alloy_server/gguf/quant.py:414-494) */
alloy_status alloy_gguf_q5_0_mm(const void* x, alloy_dtype x_dtype, const void* qweight,
                                const void* qhigh, const void* scales, void* y,
                                alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                                void* stream);

/* Raw GGUF wire-block Q8_0 / Q5_0 (the blob as stored in a .gguf file).  The
 * reference repacks these at load (gguf/quant.py:414-521); these read the blob
 * directly.  Same math as alloy_gguf_q8_0_mm / alloy_gguf_q5_0_mm. */
alloy_status alloy_gguf_q8_0_blocks_mm(const void* x, alloy_dtype x_dtype, const void* blocks,
                                       void* y, alloy_dtype y_dtype, int64_t M, int64_t N,
                                       int64_t K, void* stream);
alloy_status alloy_gguf_q5_0_blocks_mm(const void* x, alloy_dtype x_dtype, const void* blocks,
                                       void* y, alloy_dtype y_dtype, int64_t M, int64_t N,
                                       int64_t K, void* stream);

/* torch.ops.alloy.mlx_q4_mm(activations, qweight, scales, biases) — custom_ops.py:72-74.
 * group_size = 2*qweight_cols / scales_cols (packages/alloy-torch/src/alloy_torch/ops/linalg.py:509-511);
 * this build requires group_size % 32 == 0. */
alloy_status alloy_mlx_q4_mm(const void* x, alloy_dtype x_dtype, const void* qweight,
                             const void* scales, const void* biases, int32_t group_size, void* y,
                             alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Dequantisation probe: rows [row0, row0+nrows) of the weight decoded to
 * out[nrows, K] as fp32 (out_dtype F32: exact values, bit-identical to the
 * reference decode) or fp16 (F16: round-to-nearest-even of those values — the
 * operand the MFMA paths feed).  Replaces the decode half of the reference's
 * embedding ops (custom_ops.py:67-69, 83-85, 89-91, 97-99, 103; quant.py:811-884, 1165-1270, 2804-2830).
 */
alloy_status alloy_dequant(alloy_format fmt, const void* w, const void* aux, const void* scales,
                           const void* biases, int32_t group_size, void* out,
                           alloy_dtype out_dtype, int64_t row0, int64_t nrows, int64_t N,
                           int64_t K, void* stream);

/*
 * MoE router — moe_router_topk (packages/alloy-metal/src/alloy/std/moe.py:31-79):
 * per token the top_k largest logits (descending, ties to the lowest index) and a
 * softmax over those k.  logits f32[T,E] -> idx i32[T,top_k], weights f32[T,top_k].
 */
alloy_status alloy_moe_router_topk(const float* logits, int32_t* idx, float* weights, int64_t T,
                                   int32_t E, int32_t top_k, void* stream);

/* Workspace bytes alloy_mlx_moe_routed needs for (T, E, top_k, H, I). */
size_t alloy_moe_workspace_bytes(int64_t T, int32_t E, int32_t top_k, int64_t H, int64_t I);

/*
 * Routed-expert MoE block over MLX 4-bit experts — the MLX-weight counterpart of
 * torch.ops.alloy.gguf_moe_routed (custom_ops.py:63-66; handler
 * packages/alloy-torch/src/alloy_torch/ops/moe.py:110-249):
 *   router top-k -> per routed (token, slot): h = silu(G_e x) * (U_e x)
 *   -> y[t] = sum_s w[t,s] * (D_e h), summed in slot order.
 *   hidden f16[T,H]; router_logits f32[T,E]
 *   gate_up: qweight u8[E, 2I, H/2] (rows [0:I] gate, [I:2I] up), scales/biases f16[E, 2I, H/gs]
 *   down:    qweight u8[E, H, I/2],  scales/biases f16[E, H, I/gs]
 *   y f32[T,H].  workspace: >= alloy_moe_workspace_bytes(...) bytes, 256-B aligned.
 */
alloy_status alloy_mlx_moe_routed(const void* hidden, const float* router_logits,
                                  const void* gu_qweight, const void* gu_scales,
                                  const void* gu_biases, const void* dn_qweight,
                                  const void* dn_scales, const void* dn_biases,
                                  int32_t group_size, int32_t E, int32_t top_k, int64_t T,
                                  int64_t H, int64_t I, void* workspace, size_t workspace_bytes,
                                  float* y, void* stream);

/*
 * Quantized embedding lookup — the reference's gguf_q4_k_embedding,
 * gguf_q6_k_embedding, gguf_q8_0_embedding, gguf_q5_0_embedding, mlx_q4_embedding
 * (custom_ops.py:67-69, 83-85, 89-91, 97-99, 103; kernels
 * packages/alloy-metal/src/alloy/std/quant.py:811-884, 1165-1270, 2804-2830):
 * out[i, :] = the exact fp32 decode of weight row ids[i] (K values), for n_ids ids
 * (int32, or int64 when ids_int64); an id outside [0, N) gives a zero row.  The
 * weight buffers are passed as for alloy_qmm; out is f32[n_ids, K], 16-byte aligned.
 */
alloy_status alloy_embedding(alloy_format fmt, const void* w, const void* aux, const void* scales,
                             const void* biases, int32_t group_size, const void* ids, int32_t ids_int64,
                             int64_t n_ids, int64_t N, int64_t K, float* out, void* stream);

/*
 * Batched projections: n weight matrices of one format and K against the same
 * activations, y[i][M, N[i]] = x dequant(w[i])^T — the reference's batched_*_mm ops
 * (custom_ops.py:50-52, 75-78, 92-95, 100-102, 105-106; handler
 * packages/alloy-torch/src/alloy_torch/ops/linalg.py:555-682, which row-concatenates
 * the weights into one matrix).  Here nothing is copied: for M = 1 one launch per
 * group of up to 8 matrices serves all of them (each workgroup reads one matrix);
 * otherwise each matrix runs as alloy_qmm.  Host arrays of n device pointers
 * (aux / scales / biases arrays may be NULL when the format has none); outputs are
 * separate contiguous [M, N[i]] buffers.
 */
alloy_status alloy_qmm_batched(alloy_format fmt, int32_t n, const void* const* w, const void* const* aux,
                               const void* const* scales, const void* const* biases, const int64_t* N,
                               int32_t group_size, const void* x, alloy_dtype x_dtype, void* const* y,
                               alloy_dtype y_dtype, int64_t M, int64_t K, void* stream);

/*
 * Fused gated pair y[M,N] = act(x G^T) * (x U^T) over two weight matrices of one
 * format (each passed like alloy_qmm's w / aux / scales / biases) — the reference's
 * *_silu / *_gelu ops (custom_ops.py:53-58, 79-82, 108-111; kernels
 * packages/alloy-metal/src/alloy/std/quant.py:356-759, 1456-1940, 2833-2887).
 * With K % 256 == 0, K <= 4096, N <= 8192 and fp16 x, for Q4_K at 4 <= M <= 16 or
 * M >= 2 and M * N > 6144, and for MLX (power-of-two group size <= 256) at M <= 16, one
 * launch reads both matrices and applies the activation in its epilogue and no
 * workspace is needed; otherwise the two products go to fp32 workspace buffers and a
 * combine kernel writes y.  workspace: >=
 * alloy_glu_workspace_bytes(...) bytes, 256-byte aligned (may be NULL when that is 0).
 */
size_t alloy_glu_workspace_bytes(alloy_format fmt, int64_t M, int64_t N, int64_t K, int32_t group_size,
                                 alloy_dtype x_dtype);
alloy_status alloy_qmm_glu(alloy_format fmt, alloy_act act, const void* gate_w, const void* gate_aux,
                           const void* gate_scales, const void* gate_biases, const void* up_w,
                           const void* up_aux, const void* up_scales, const void* up_biases,
                           int32_t group_size, const void* x, alloy_dtype x_dtype, void* y,
                           alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream);
/* gguf_q4_k_silu / gguf_q4_k_gelu(activations, gate_blocks, up_blocks) — custom_ops.py:53-58 */
alloy_status alloy_gguf_q4_k_silu(const void* x, alloy_dtype x_dtype, const void* gate_blocks,
                                  const void* up_blocks, void* y, alloy_dtype y_dtype, int64_t M, int64_t N,
                                  int64_t K, void* workspace, size_t workspace_bytes, void* stream);
alloy_status alloy_gguf_q4_k_gelu(const void* x, alloy_dtype x_dtype, const void* gate_blocks,
                                  const void* up_blocks, void* y, alloy_dtype y_dtype, int64_t M, int64_t N,
                                  int64_t K, void* workspace, size_t workspace_bytes, void* stream);
/* mlx_q4_silu(activations, gate_qweight, gate_scales, gate_biases, up_qweight, up_scales,
 * up_biases) — custom_ops.py:79-82 */
alloy_status alloy_mlx_q4_silu(const void* x, alloy_dtype x_dtype, const void* gate_qweight,
                               const void* gate_scales, const void* gate_biases, const void* up_qweight,
                               const void* up_scales, const void* up_biases, int32_t group_size, void* y,
                               alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K, void* workspace,
                               size_t workspace_bytes, void* stream);
/* gguf_q8_0_silu(activations, gate_qweight, gate_scales, up_qweight, up_scales) — custom_ops.py:108-111 */
alloy_status alloy_gguf_q8_0_silu(const void* x, alloy_dtype x_dtype, const void* gate_qweight,
                                  const void* gate_scales, const void* up_qweight, const void* up_scales,
                                  void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routed-expert MoE block over GGUF experts — torch.ops.alloy.gguf_moe_routed
 * (custom_ops.py:59-66; handler packages/alloy-torch/src/alloy_torch/ops/moe.py:110-249;
 * containers packages/alloy-server/src/alloy_server/models/qwen3_5.py:232-343):
 *   same routing and composition as alloy_mlx_moe_routed, with
 *   gate_up_blocks u8[E, 2I, (H/256)*144] native Q4_K (rows [0:I] gate, [I:2I] up),
 *   down_qweight   u8[E, H, (I/256)*210] Q6_K.
 *   hidden f16[T,H]; router_logits f32[T,E]; y f32[T,H].  H and I multiples of 256
 *   (ALLOY_E_SHAPE otherwise, as the reference's containers require), at most 4096
 *   (ALLOY_E_UNSUPPORTED).  workspace: >= alloy_moe_workspace_bytes(...) bytes.
 */
alloy_status alloy_gguf_moe_routed(const void* hidden, const float* router_logits,
                                   const void* gate_up_blocks, const void* down_qweight, int32_t E,
                                   int32_t top_k, int64_t T, int64_t H, int64_t I, void* workspace,
                                   size_t workspace_bytes, float* y, void* stream);

/*
 * gguf_moe_routed without a workspace argument.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same computation, routing and
 * results as alloy_gguf_moe_routed; the workspace is a library-owned static device
 * array of ALLOY_MOE_NOALLOC_SCRATCH_BYTES on each GPU (held until the process
 * ends).  A shape whose alloy_moe_workspace_bytes(T, E, top_k, H, I) exceeds it
 * returns ALLOY_E_UNSUPPORTED (at H = 2048, I = 768, top_k = 8: T <= 256).  All calls
 * on one GPU share the array: calls that overlap (other streams) race and must be
 * serialized by the caller.  Calls no hipMalloc / hipFree.
 */
#define ALLOY_MOE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
alloy_status alloy_gguf_moe_routed_noalloc(const void* hidden, const float* router_logits,
                                           const void* gate_up_blocks, const void* down_qweight, int32_t E,
                                           int32_t top_k, int64_t T, int64_t H, int64_t I, float* y,
                                           void* stream);

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* alloy_last_error(void);
/* Library version string. */
const char* alloy_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ALLOY_AMD_H */
