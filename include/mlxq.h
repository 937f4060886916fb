/*
 * mlxq -- MI355X (gfx950) quantized-weight hot path, C ABI.
 *
 * Drop-in boundary for the device arithmetic that SceneWorks/mlx-llm reaches
 * through MLX (group-wise affine quantize / dequantize / quantized_matmul) and
 * for its pure-Rust GGUF block dequantizer.  Each entry point names the
 * reference call it replaces (paths relative to the reference crate root).
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers owned by the caller; the library
 *     allocates nothing on these paths.  Work is enqueued asynchronously on
 *     `stream` (a hipStream_t; NULL = the default stream); the caller
 *     synchronizes before reading results.
 *   - Row-major layouts.  Weights use the Hugging Face `[out, in]` layout:
 *     W is [N, K]; x is [M, K]; y is [M, N] (quantized_matmul transpose=true).
 *   - Packed codes: wq is uint32 [N, K*bits/32]; element k of a row sits in
 *     word k/(32/bits) at bits [(k%(32/bits))*bits, +bits) (LSB first).
 *     scales/biases are [N, K/group_size] in the weight dtype.
 *   - bf16 / f16 values are passed as their 16-bit patterns.
 *   - Every function returns an mlxq_status.  On failure, mlxq_last_error()
 *     returns a message for the calling thread.
 *   - Calls are reentrant per stream.  The qmatmul workspace (below) must not
 *     be shared by calls that can run concurrently.
 */
#ifndef MLXQ_H
#define MLXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The reference maps errors to crate::error::Error
 * (src/error.rs:11-42): MLXQ_ERR_UNSUPPORTED -> Error::Unsupported,
 * MLXQ_ERR_DEVICE -> Error::Mlx, everything else -> Error::Msg. */
typedef enum {
  MLXQ_OK = 0,
  MLXQ_ERR_INVALID = 1,      /* null pointer, negative size, bad enum value */
  MLXQ_ERR_SHAPE = 2,        /* K % group_size != 0, n % block_elems != 0  */
  MLXQ_ERR_UNSUPPORTED = 3,  /* bits / group_size / GGUF tag / dtype       */
  MLXQ_ERR_SHORT_BUFFER = 4, /* GGUF data shorter than the blocks need     */
  MLXQ_ERR_WORKSPACE = 5,    /* qmatmul workspace missing or too small     */
  MLXQ_ERR_DEVICE = 6        /* HIP runtime / launch failure               */
} mlxq_status;

/* Element types for the `dtype` arguments. */
typedef enum {
  MLXQ_F32 = 0,
  MLXQ_F16 = 1,
  MLXQ_BF16 = 2
} mlxq_dtype;

/* Kernel choice for mlxq_qmatmul_algo. */
typedef enum {
  MLXQ_ALGO_AUTO = 0, /* qmv for M <= 32, qmm above (what mlxq_qmatmul does) */
  MLXQ_ALGO_QMV = 1,  /* decode GEMV, any M <= 32                             */
  MLXQ_ALGO_QMM = 2,  /* LDS-dequant bf16 MFMA GEMM, any M                    */
  MLXQ_ALGO_QMM_LIB = 3 /* dequantize into the workspace, then hipBLASLt's bf16
                           GEMM (needs mlxq_qmatmul_workspace_size bytes at a
                           shape where MLXQ_ALGO_AUTO takes it; see there)      */
} mlxq_algo;

/* Message for the last failing call on this thread ("" if none). */
const char* mlxq_last_error(void);
/* Library version string. */
const char* mlxq_version(void);

/* Reads the MLXQ_* kernel-override environment variables (tuning and tests:
 * force a GEMV kernel or a tile configuration) again.  No counterpart in the
 * reference.  The dispatch reads them once, on first use, never per call, so
 * a process that changes them calls this afterwards. */
int mlxq_reload_overrides(void);

/* ------------------------------------------------------------------ */
/* Affine group-wise quantization                                      */
/* ------------------------------------------------------------------ */

/* Replaces mlx_rs::ops::quantize(w, group_size, bits) reached from
 * QuantizedLinear::quantize (src/primitives/quant.rs:38-53, call at :44),
 * itself called by Projection::load_with_bias (src/primitives/projection.rs:57-71),
 * quantize-on-load (src/models/llama.rs:97) and the snapshot requant
 * (src/snapshot.rs:100-107).
 * w: [rows, cols] in `dtype` (MLXQ_F32 or MLXQ_BF16); scales/biases are
 * written in the same dtype.  bits in {4, 8}; group_size in {32, 64, 128}. */
int mlxq_quantize(const void* w, int dtype, int64_t rows, int64_t cols,
                  int group_size, int bits, uint32_t* wq, void* scales,
                  void* biases, void* stream);

/* Replaces mlx_rs::ops::dequantize reached from
 * QuantizedLinear::dequantize_weight (src/primitives/quant.rs:73-81).
 * out[r, c] = scale * q + bias, computed in f32 and stored in `dtype`. */
int mlxq_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                    int dtype, int64_t rows, int64_t cols, int group_size,
                    int bits, void* out, void* stream);

/* ------------------------------------------------------------------ */
/* Quantized matmul                                                    */
/* ------------------------------------------------------------------ */

/* Bytes of device workspace mlxq_qmatmul may use for this shape: nonzero
 * for batched decode (2 <= M <= 32, group size 64; also calls of 33..64
 * rows, run as 32-row decode calls) and for prefill shapes with too few
 * output tiles to fill the GPU (e.g. M = 512, 4096 -> 4096: 4 x M x N x 4
 * bytes), where the kernel splits K across workgroups and a second kernel
 * adds the f32 partial sums in slice order.  At prefill shapes where it is
 * measured faster (gate/up-like from M = 512, square from 1024, down-like
 * from 1024 / 2048 (Q4 / Q8), k/v-like from 2048) the size is instead that
 * of the whole weight dequantized to bf16 (N x K x 2 bytes) plus 32 MiB for
 * hipBLASLt: the call dequantizes into the workspace and runs hipBLASLt's
 * bf16 GEMM (MLXQ_ALGO_QMM_LIB).
 * The workspace must be 256-byte aligned; its contents need no
 * initialisation and are scratch after a call.  With no or too small a
 * workspace the call still succeeds on the fused / unsplit kernels. */
int mlxq_qmatmul_workspace_size(int64_t M, int64_t N, int64_t K,
                                int group_size, int bits, size_t* bytes);

/* Replaces mlx_rs::ops::quantized_matmul(x, w, scales, Some(biases),
 * transpose=true, group_size, bits) plus the optional dense bias add, i.e.
 * QuantizedLinear::forward (src/primitives/quant.rs:56-70), reached from
 * Projection::forward (src/primitives/projection.rs:93-98).
 * y[m, n] = sum_k x[m, k] * (scale*q + bias)[n, k]  (+ bias_vec[n])
 * x, scales, biases, bias_vec (nullable, [N]) and y are bf16; accumulation is
 * f32.  M >= 1 rows of activations (decode: M = batch; prefill: M = tokens). */
int mlxq_qmatmul(const void* x, int64_t M, const uint32_t* wq,
                 const void* scales, const void* biases, const void* bias_vec,
                 int64_t N, int64_t K, int group_size, int bits, void* y,
                 void* workspace, size_t workspace_bytes, void* stream);

/* mlxq_qmatmul with an explicit kernel choice (mlxq_algo).  MLX makes the
 * same qmv/qmm choice internally from M. */
int mlxq_qmatmul_algo(const void* x, int64_t M, const uint32_t* wq,
                      const void* scales, const void* biases,
                      const void* bias_vec, int64_t N, int64_t K,
                      int group_size, int bits, void* y, void* workspace,
                      size_t workspace_bytes, int algo, void* stream);

/* mlxq_qmatmul for callers that cannot allocate or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same kernels and results as
 * mlxq_qmatmul with a workspace, except where mlxq_qmatmul would take the
 * library GEMM (some shapes above 512 rows; it needs a workspace of the
 * whole dequantized weight and a hipBLASLt handle, which allocates): there
 * the qmm kernel runs instead (or 32-row decode calls when K does not suit
 * it).  So for M > 32: 33..64 rows run as 32-row decode calls, gate/up-like
 * shapes at 65..128 rows on the 64-row streaming form, the others on qmm
 * (mlxq_qmatmul_route with noalloc = 1 names the route).  The split-K
 * partial sums live in a fixed library scratch array in device
 * memory (mlxq_qmatmul_noalloc_max_scratch() bytes, 64 MiB, held by every
 * device the library runs on until the process ends); nothing is allocated.
 * A shape whose workspace size exceeds the scratch returns
 * MLXQ_ERR_WORKSPACE before any launch (e.g. a 4096 -> 128256 lm_head at
 * M = 32: 16 x M x N x 4 bytes).
 * All calls on one device share its scratch: calls that can overlap in time
 * on one device (two streams, two threads) race and must be serialized by
 * the caller. */
int mlxq_qmatmul_noalloc(const void* x, int64_t M, const uint32_t* wq,
                         const void* scales, const void* biases,
                         const void* bias_vec, int64_t N, int64_t K,
                         int group_size, int bits, void* y, void* stream);

/* The kernels a call of mlxq_qmatmul_algo (noalloc = 0, with a workspace
 * of workspace_bytes) or of mlxq_qmatmul_noalloc (noalloc = 1) with these
 * sizes would launch, as a NUL-terminated " + "-separated list of kernel
 * names with their template arguments (e.g. "qmm_kernel<4, 64, 8, 2>",
 * "tile::qmv_stream_kernel<8, 64, 2, 8, 4, 2, false> + ...", a library GEMM
 * as "hipBLASLt GEMM"), into buf.  The library's own dispatch runs with
 * every launch suppressed, so the answer is the route the call takes, for
 * labels, measurement bookkeeping and tests.  Launches nothing and touches
 * no device memory, but needs the device (the dispatch queries occupancy and
 * the kernel names come from the runtime).  No counterpart in the
 * reference. */
int mlxq_qmatmul_route(int64_t M, int64_t N, int64_t K, int group_size,
                       int bits, size_t workspace_bytes, int algo,
                       int noalloc, char* buf, size_t buf_len);

/* Size in bytes of mlxq_qmatmul_noalloc's scratch array. */
size_t mlxq_qmatmul_noalloc_max_scratch(void);

/* One projection of a fused decode call (mlxq_qmatmul_fused). */
typedef struct {
  const uint32_t* wq;    /* [N, K*bits/32] packed codes                     */
  const void* scales;    /* [N, K/group_size] bf16                          */
  const void* biases;    /* [N, K/group_size] bf16                          */
  const void* bias;      /* [N] bf16 dense bias, or NULL                    */
  const void* residual;  /* [M, N] bf16, or NULL: y = bf16(r + bf16(x W^T)) */
  void* y;               /* [M, N] bf16 output                              */
  int64_t N;
} mlxq_projection;

/* Decode-step fusion of the layer chain around the projections
 * (src/models/llama.rs:689-735): one launch computes
 *   x' = rms_norm(x, norm_weight, eps)          if norm_weight != NULL
 *        (nn.rs:35-37, as mlxq_rms_norm),
 *   x' = repeat_kv(x, kv_heads, head_dim, groups) if groups > 1
 *        (attention.rs:45-55; x rows then hold K/groups values),
 *   x' = x                                      otherwise,
 * and then, for nproj <= 3 projections of the same x' (q, k, v at
 * llama.rs:806-812), y_i = x' W_i^T (+ bias_i) (+ residual_i: the residual
 * add of llama.rs:729-733, rounded as add(r, bf16(x' W^T))).
 * swiglu != 0 (nproj == 2): y_0 = silu(x' W_0^T) * (x' W_1^T) with the
 * rounding of mlxq_silu_mul (llama.rs:1040-1045).
 * Results equal the unfused sequence of mlxq_rms_norm / mlxq_repeat_kv /
 * mlxq_qmatmul / mlxq_add / mlxq_silu_mul up to f32 summation order.
 * Covers: 1 <= M <= 4 (K*bits/8 % 64 == 0), every form, SwiGLU only with a
 * norm; 5 <= M <= 32, group size 64: multi-projection / head repeat /
 * residual forms where K is one tile slice (Q4 K = 4096, Q8 K = 2048 or
 * 4096), SwiGLU without a norm on gate/up-like shapes (N * K >= 2^25,
 * K < N), the residual / multi-projection forms otherwise.  Other shapes
 * and forms (e.g. a norm above 4 rows) return MLXQ_ERR_UNSUPPORTED before
 * any launch, and the caller issues the unfused calls.  No workspace, no
 * allocation. */
int mlxq_qmatmul_fused(const void* x, int64_t M, int64_t K,
                       const void* norm_weight, float eps, int kv_heads,
                       int head_dim, int groups, const mlxq_projection* proj,
                       int nproj, int swiglu, int group_size, int bits,
                       void* stream);

/* The end of a decoder layer and the start of the next
 * (src/models/llama.rs:729-733 residual add after down_proj, then :698
 * input_layernorm of the next layer):
 *   sum_out = bf16(residual + bf16(x W^T (+ bias_vec))),
 *   y       = rms_norm(sum_out, norm_weight, eps)   (as mlxq_rms_norm).
 * Results equal mlxq_qmatmul followed by mlxq_add_rms_norm bit for bit.  At
 * 5 <= M <= 32 where mlxq_qmatmul splits K, the split sum, the residual and
 * the norm run in one second launch (one workgroup per row) instead of two;
 * other shapes run the unfused calls.  workspace / workspace_bytes as for
 * mlxq_qmatmul (mlxq_qmatmul_workspace_size).  residual, norm_weight,
 * sum_out and y are bf16 ([M, N], [N], [M, N], [M, N]), 16-byte aligned;
 * N % 8 == 0; sum_out may not alias residual. */
int mlxq_qmatmul_add_rms_norm(const void* x, int64_t M, const uint32_t* wq,
                              const void* scales, const void* biases,
                              const void* bias_vec, int64_t N, int64_t K,
                              int group_size, int bits, const void* residual,
                              const void* norm_weight, float eps,
                              void* sum_out, void* y, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ */
/* Decode layer chain around the projections (bf16, MLX rounding points) */
/* ------------------------------------------------------------------ */

/* Replaces mlx_rs::fast::rms_norm reached from primitives::nn::rms_norm
 * (src/primitives/nn.rs:35-37), applied before q/k/v and gate/up
 * (src/models/llama.rs:698,728) and before lm_head (:596).
 * x, y: [rows, dim] bf16; weight: [dim] bf16; dim % 8 == 0.
 * y = bf16(weight * bf16(x * 1/sqrt(mean(x^2) + eps))), sums in f32. */
int mlxq_rms_norm(const void* x, const void* weight, int64_t rows, int64_t dim,
                  float eps, void* y, void* stream);

/* Replaces silu(gate) followed by multiply(gate, up) in LlamaMlp::forward
 * (src/models/llama.rs:1040-1045; silu at src/primitives/nn.rs:50-52).
 * n bf16 elements (n % 8 == 0):
 * y = bf16(bf16(g * bf16(1/(1+exp(-g)))) * u). */
int mlxq_silu_mul(const void* gate, const void* up, int64_t n, void* y,
                  void* stream);

/* Replaces the residual add(x, attn) / add(h, ffn)
 * (src/models/llama.rs:729-733): y = bf16(a + b), n % 8 == 0. */
int mlxq_add(const void* a, const void* b, int64_t n, void* y, void* stream);

/* The residual add that ends a layer followed by the RMSNorm that starts
 * the next one (src/models/llama.rs:729-733 then :698, or the final norm
 * at :596), in one launch: sum = bf16(a + b) as mlxq_add, y =
 * rms_norm(sum, weight, eps) as mlxq_rms_norm.  a, b, sum, y: [rows, dim]
 * bf16, dim % 8 == 0.  sum may be a or b (in-place residual update); y may
 * not alias a, b or sum. */
int mlxq_add_rms_norm(const void* a, const void* b, const void* weight,
                      int64_t rows, int64_t dim, float eps, void* sum,
                      void* y, void* stream);

/* Replaces repeat_kv (src/primitives/attention.rs:45-55) for one position:
 * x [rows, kv_heads, head_dim] -> y [rows, kv_heads*groups, head_dim], output
 * head h = KV head h / groups.  head_dim % 8 == 0. */
int mlxq_repeat_kv(const void* x, int64_t rows, int kv_heads, int head_dim,
                   int groups, void* y, void* stream);

/* ------------------------------------------------------------------ */
/* GGUF block dequantization                                           */
/* ------------------------------------------------------------------ */

/* GgmlType::from_tag + GgmlType::block (src/gguf/dequant.rs:85-141):
 * (elements per block, bytes per block) for a GGUF type tag.  Host only. */
int mlxq_gguf_block(uint32_t tag, int64_t* elems, int64_t* bytes);

/* tensor_byte_len (src/gguf/dequant.rs:144-153).  Host only. */
int mlxq_gguf_tensor_byte_len(uint32_t tag, int64_t n, int64_t* bytes);

/* Replaces gguf::dequant::dequantize(tag, data, n) (src/gguf/dequant.rs:156-211),
 * called by gguf::convert (src/gguf/convert.rs:132).  data: device bytes of
 * n/elems blocks (data_len >= the blocks' bytes); out: n values in out_dtype
 * (MLXQ_F32: bit-exact with the reference; MLXQ_BF16: that f32 value rounded
 * to nearest-even, as convert.rs:156 does).  Device tags: F32, F16, BF16,
 * Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS,
 * and the grid types IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M
 * (dequant.rs:505-719): every type the reference decodes. */
int mlxq_gguf_dequantize(uint32_t tag, const void* data, int64_t data_len,
                         int64_t n, int out_dtype, void* out, void* stream);

/* Fused on-device convert of one projection weight, replacing for a GGUF
 * tensor with a projection key the host chain of convert
 * (src/gguf/convert.rs:131 dequantize, :133-137 q/k un-permute via
 * permute_inverse_qk :232-256, :156 cast to bf16) and the snapshot writer's
 * requant (:176 -> src/snapshot.rs:100-107 -> quant.rs:44).
 * data: device bytes of the [rows, cols] GGUF tensor (tags as
 * mlxq_gguf_dequantize); permute_heads > 0 un-permutes rows with that head
 * count (llama q: num_heads, k: num_kv_heads), 0 leaves them.  Output: MLX
 * affine wq [rows, cols*bits/32], bf16 scales/biases [rows, cols/group_size],
 * bit-identical with mlxq_gguf_dequantize(BF16) -> row gather ->
 * mlxq_quantize(BF16), with no intermediate tensor. */
int mlxq_gguf_requantize(uint32_t tag, const void* data, int64_t data_len,
                         int64_t rows, int64_t cols, int permute_heads,
                         int group_size, int bits, uint32_t* wq, void* scales,
                         void* biases, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MLXQ_H */
