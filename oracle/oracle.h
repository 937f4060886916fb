/*
 * CPU oracle for the quantized-weight hot path.  TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / the CPU baseline.  The product
 * path (libmlxq.so) never links it.
 *
 * Every function restates the reference's algorithm and cites the
 * /root/reference file:line it follows.  Pinning of each function (what checks
 * it against something other than itself) is listed next to it.
 */
#ifndef MLXQ_ORACLE_H
#define MLXQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded inputs: SplitMix64 (src/primitives/sampler.rs:33-60) ----
 * pinned: published SplitMix64 outputs for seed 0 (tests/test_oracle.py). */
uint64_t orc_splitmix64_next(uint64_t* state);
float orc_splitmix64_next_f32(uint64_t* state); /* (u64>>40)/2^24, sampler.rs:57-59 */
/* n draws of N(mean, std) via Box-Muller in f64, rounded to f32.
 * pinned: sample mean/variance and moments (tests/test_oracle.py). */
void orc_gen_normal_f32(uint64_t seed, float mean, float std, float* out, size_t n);

/* ---- scalar conversions ----
 * f16 -> f32 is exact (`half::f16::to_f32`, dequant.rs:222-225).
 * pinned: exhaustive over all 65536 f16 patterns against numpy.float16. */
float orc_f16_to_f32(uint16_t h);
/* f32 -> f16 round-to-nearest-even (used only to build GGUF blocks).
 * pinned: exhaustive sweep against numpy.float16 casts. */
uint16_t orc_f32_to_f16(float f);
/* f32 -> bf16 round-to-nearest-even (MLX `as_dtype(bf16)`, convert.rs:156).
 * pinned: against torch bfloat16 casts over special values and random bits. */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);

/* ---- GGUF geometry (dequant.rs:85-153) ----
 * returns 0 ok, 3 unsupported tag, 2 bad element count. */
int orc_gguf_block(uint32_t tag, int64_t* elems, int64_t* bytes);
int orc_gguf_tensor_byte_len(uint32_t tag, int64_t n, int64_t* bytes);
/* dequant.rs:156-211: returns 0 ok, 3 unsupported, 2 n not a multiple,
 * 4 data shorter than needed.  Every type the reference decodes: F32, F16,
 * BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL,
 * IQ4_XS and the grid types IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S,
 * IQ1_M (dequant.rs:505-719).
 * pinned (grid types): the reference's known answers (dequant.rs:877-955),
 * the codebooks' structure and closed forms of single-bit changes
 * (tests/test_oracle_iq.py). */
int orc_gguf_dequantize(uint32_t tag, const uint8_t* data, int64_t data_len,
                        int64_t n, float* out);
/* ksigns_iq2xs entry i (i < 128): i with bit 7 = parity of i. */
uint8_t orc_ksigns_iq2xs(int i);
/* Codebook `table` (0 IQ2_XXS, 1 IQ2_XS, 2 IQ2_S, 3 IQ3_XXS, 4 IQ3_S,
 * 5 IQ1_S): entry i into *entry (if non-null); returns the table size, -1
 * for a bad table or index. */
int orc_iq_grid(int table, int i, uint64_t* entry);

/* ---- GGUF block producers (NOT in the reference; llama.cpp block layouts
 * restated from the public ggml format so tests have realistic blocks).
 * Only the validity of the bytes matters; parity is judged on dequant.
 * pinned: produce -> orc_gguf_dequantize round trip stays within the format's
 * quantization error (tests/test_oracle.py). */
int orc_gguf_quantize(uint32_t tag, const float* x, int64_t n, uint8_t* out);

/* ---- MLX group-wise affine quantization (quant.rs:38-53 -> mlx quantize,
 * MLX 0.31.2 CPU backend semantics).  dtype: 0 = f32 input and f32
 * scales/biases, 2 = bf16 input (uint16 bits) and bf16 scales/biases.
 * wq is [rows, cols*bits/32] uint32, LSB-first packing along cols.
 * pinned: affine-grid invariants + quant.rs:91-107 round trip (tests). */
int orc_affine_quantize(int dtype, const void* w, int64_t rows, int64_t cols,
                        int group_size, int bits, uint32_t* wq, void* scales,
                        void* biases);
/* w = scale*q + bias in f32, stored in dtype (quant.rs:73-81). */
int orc_affine_dequantize(int dtype, const uint32_t* wq, const void* scales,
                          const void* biases, int64_t rows, int64_t cols,
                          int group_size, int bits, void* out);
/* y[m,n] = sum_k x[m,k] * (s*q+b)[n,k] in f64 (quant.rs:56-70 with
 * transpose=true); x is bf16 bits; s/b bf16 bits; y f64.
 * pinned: against a dense float64 numpy matmul of orc_affine_dequantize. */
int orc_qmatmul_f64(const uint16_t* x, int64_t M, const uint32_t* wq,
                    const uint16_t* scales, const uint16_t* biases,
                    int64_t N, int64_t K, int group_size, int bits,
                    double* y);
/* Same product, f32 accumulation, OpenMP over N: the timed CPU baseline
 * ("port" of the reference's dequant-on-the-fly CPU path). */
int orc_qmatmul_f32(const uint16_t* x, int64_t M, const uint32_t* wq,
                    const uint16_t* scales, const uint16_t* biases,
                    int64_t N, int64_t K, int group_size, int bits,
                    float* y, int threads);
/* OpenMP-parallel GGUF dequant over blocks for the CPU baseline timing. */
int orc_gguf_dequantize_mt(uint32_t tag, const uint8_t* data, int64_t data_len,
                           int64_t n, float* out, int threads);

/* ---- decode layer chain (bf16 in/out, MLX rounding points) ----
 * rms_norm: src/primitives/nn.rs:35-37; silu_mul: src/models/llama.rs:1040-1045;
 * add: llama.rs:729-733; repeat_kv: src/primitives/attention.rs:45-55.
 * pinned: closed forms, scipy's expit, torch's bf16 casts and the
 * reference's repeat_kv known answer (tests/test_oracle.py). */
int orc_rms_norm_bf16(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t dim,
                      float eps, uint16_t* y);
int orc_silu_mul_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* y);
int orc_add_bf16(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* y);
int orc_repeat_kv(const uint16_t* x, int64_t rows, int kv_heads, int head_dim, int groups,
                  uint16_t* y);

#ifdef __cplusplus
}
#endif
#endif
