/*
 * rsllm_oracle.h — CPU restatement of rsLLM's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the parity oracle and the CPU baseline
 * (kind "port"). It is linked only by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg. The product library (rsllm_amd) never links
 * or calls it.
 *
 * Every function restates one reference function; the citation is given
 * beside each declaration (paths relative to the rsLLM source tree).
 * Status codes use the same numbering as include/rsllm_hip.h so that error
 * behaviour can be compared one-to-one.
 */
#ifndef RSLLM_ORACLE_H
#define RSLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_SHAPE_MISMATCH = 1,        /* backend-cpu/src/error.rs:12 */
    ORC_NOT_BLOCK_ALIGNED = 2,     /* backend-cpu/src/error.rs:18-25 */
    ORC_NON_FINITE_INPUT = 3,      /* backend-cpu/src/error.rs:33 */
    ORC_DEQUANT_SIZE_MISMATCH = 5, /* rsllm-gguf/src/error.rs:71-76 */
    ORC_UNSUPPORTED_DEQUANT = 6,   /* rsllm-gguf/src/error.rs:80 */
    ORC_PANIC = 9                  /* the reference would panic (e.g. row_len == 0) */
};

/* GgmlType ids, rsllm-gguf/src/tensor.rs:26-85 */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 8,
    ORC_Q2_K = 10, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15,
    ORC_IQ2_XXS = 16, ORC_BF16 = 30
};

/* Detail of the last error on this thread (sizes of NotBlockAligned /
 * DequantSizeMismatch). */
void orc_last_detail(size_t *a, size_t *b);

/* half::f16::to_f32 (half 2.7.1), call sites rsllm-gguf/src/dequant/q4_k.rs:53-54. */
float orc_f16_to_f32(uint16_t h);

/* GgmlType::block_elements / block_bytes, rsllm-gguf/src/tensor.rs:128-184.
 * Returns 0 for ids this oracle does not know. */
uint32_t orc_block_elements(uint32_t dtype);
uint32_t orc_block_bytes(uint32_t dtype);

/* q4_k_scale_min, rsllm-gguf/src/dequant/mod.rs:48-58 */
void orc_q4k_scale_min(int j, const uint8_t q[12], uint8_t *sc, uint8_t *m);

/* dequant_q4_k  rsllm-gguf/src/dequant/q4_k.rs:35-92
 * dequant_q6_k  rsllm-gguf/src/dequant/q6_k.rs:34-102
 * dequant_q8_0  rsllm-gguf/src/dequant/q8_0.rs:25-63
 * dequant_q4_0  rsllm-gguf/src/dequant/q4_0.rs:44-64 */
int orc_dequant_q4_k(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_q6_k(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_q8_0(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_q4_0(const uint8_t *src, size_t src_len, float *dst, size_t n);
/* dequant_q2_k     rsllm-gguf/src/dequant/q2_k.rs:39-98
 * dequant_iq2_xxs  rsllm-gguf/src/dequant/iq2_xxs.rs:47-113 (codebook
 * iq2_xxs/tables.rs; orc_iq2xxs_grid(i) returns entry i as a u64) */
int orc_dequant_q2_k(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_iq2_xxs(const uint8_t *src, size_t src_len, float *dst, size_t n);
uint64_t orc_iq2xxs_grid(int i);
/* dequant_q4_1  rsllm-gguf/src/dequant/q4_0.rs:66-104
 * dequant_q5_k  rsllm-gguf/src/dequant/q5_k.rs:34-94
 * dequant_q8_k  rsllm-gguf/src/dequant/q8_k.rs:32-70 */
int orc_dequant_q4_1(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_q5_k(const uint8_t *src, size_t src_len, float *dst, size_t n);
int orc_dequant_q8_k(const uint8_t *src, size_t src_len, float *dst, size_t n);

/* dequant_to_f32, rsllm-gguf/src/dequant/mod.rs:69-85: every arm (F32,
 * F16, BF16, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, Q8_0, Q2_K, Q8_K, IQ2_XXS); the
 * rest report ORC_UNSUPPORTED_DEQUANT. */
int orc_dequant_to_f32(uint32_t dtype, const uint8_t *src, size_t src_len, float *dst, size_t n);

/* matmul_quant_f32, rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119.
 * Threads: one task per token (parallel.rs:37-54); n_threads == 0 means
 * min(n_tok, online cores). allow_q6k != 0 runs the same algorithm for Q6_K,
 * which the reference's dtype guard (:57-64) rejects. */
int orc_matmul_quant_f32(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                         const float *x, size_t x_len, size_t n_tok, size_t in_dim,
                         size_t out_dim, uint32_t dtype, int allow_q6k, int n_threads);

/* The same arithmetic restricted to output rows [row0, row1) of every token;
 * used to time a bounded sample of a large matrix. */
int orc_matmul_quant_f32_rows(float *out, const uint8_t *w, const float *x, size_t n_tok,
                              size_t in_dim, size_t out_dim, uint32_t dtype, size_t row0,
                              size_t row1, int n_threads);

/* quantize_q8_0_activation  rsllm-backend-cpu/src/ops/q8_0.rs:42-88
 * quantize_q8_0_batch       rsllm-backend-cpu/src/ops/q8_0.rs:95-129
 * dot_q8_0_row_scalar       rsllm-backend-cpu/src/ops/q8_0.rs:163-193
 * matmul_q8_0_batch         rsllm-backend-cpu/src/ops/q8_0.rs:217-263 */
int orc_quantize_q8_0_activation(const float *x, size_t n, int8_t *xq, size_t xq_len,
                                 float *scale, size_t scale_len);
int orc_quantize_q8_0_batch(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                            float *scale, size_t scale_len, size_t n_tok, size_t in_dim);
float orc_dot_q8_0_row_scalar(const uint8_t *row, const int8_t *xq, const float *xscale,
                              size_t in_dim);
int orc_matmul_q8_0_batch(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                          const int8_t *xq, size_t xq_len, const float *xscale,
                          size_t xscale_len, size_t n_tok, size_t in_dim, size_t out_dim,
                          int n_threads);

/* sigmoid / silu / swiglu, rsllm-backend-cpu/src/ops/scalar.rs:57-86 */
float orc_sigmoid(float x);
float orc_silu(float x);
/* apply_swiglu_clamp, rsllm-models/src/dsv4/moe.rs:515-531 (in place) */
void orc_swiglu_clamp(float *h_gate, float *h_up, size_t n, float c);

/* Routed-expert composition: accumulate_moe_outputs moe.rs:648-707 with
 * apply_expert_swiglu moe.rs:479-502 and apply_swiglu_clamp moe.rs:515-531,
 * every matmul going through orc_matmul_quant_f32 (n_tok = 1, as the
 * reference calls it). Experts are slices of stacked blobs
 * (StackedExperts::expert moe.rs:69-108): expert e of `gate` starts at
 * e * n_ff * row_bytes(n_embd).
 * out [n_tok x n_embd] is ACCUMULATED into (the caller pre-clears it). */
int orc_moe_routed(float *out, const float *x, size_t n_tok, size_t n_embd, size_t n_ff,
                   const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                   uint32_t dtype_gate_up, uint32_t dtype_down, size_t n_expert,
                   const int32_t *ids, const float *weights, size_t k, float clamp);

/* matmul_weight_f32, rsllm-models/src/dsv4/weight.rs:113-169. dtype ORC_F32:
 * w holds out_dim * in_dim f32 values (w_len in bytes), naive sequential dot
 * (:148-158); otherwise orc_matmul_quant_f32 (allow_q6k as there) with every
 * non-panic error reported as ORC_SHAPE_MISMATCH (:160-167). Errors of
 * this function itself: detail a = 10 (out), 11 (x), 12 (weight_f32),
 * 13 (quant). */
int orc_matmul_weight_f32(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                          const float *x, size_t x_len, size_t n_tok, size_t in_dim,
                          size_t out_dim, uint32_t dtype, int allow_q6k);

/* matmul_grouped_lora_down, weight.rs:209-266, with grouped_weight_slice
 * :271-323: per group g, gather x columns, matmul_weight_f32 on the g-th
 * [rank x group_dim] slice, scatter into out. Errors (all ORC_SHAPE_MISMATCH,
 * detail a): 20 (x), 21 (out), 22 (slice f32), 23 (slice alignment),
 * 24 (slice quant), or matmul_weight_f32's; detail b = the failing group.
 * As in the reference, groups before a failing one are already written. */
int orc_matmul_grouped_lora_down(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                                 const float *x, size_t x_len, size_t n_tok, size_t n_groups,
                                 size_t group_dim, size_t rank, uint32_t dtype, int allow_q6k);

/* apply_shared_expert, rsllm-models/src/dsv4/moe.rs:422-455 with
 * apply_expert_swiglu :479-502 (one expert through every token; out is
 * overwritten). Each matrix is a WeightBlob of its own dtype (ORC_F32 or a
 * quant type). Errors: ORC_SHAPE_MISMATCH detail a = 30 (x), 31 (out), or
 * orc_matmul_weight_f32's with detail b = 0 / 1 / 2 for gate / up / down. */
int orc_apply_shared_expert(float *out, size_t out_len, const float *x, size_t x_len,
                            const uint8_t *gate, size_t gate_len, uint32_t dt_gate,
                            const uint8_t *up, size_t up_len, uint32_t dt_up,
                            const uint8_t *down, size_t down_len, uint32_t dt_down, size_t n_tok,
                            size_t n_embd, size_t n_ff, float clamp);

/* Online core count (what rayon's global pool would size itself to). */
int orc_num_cores(void);

#ifdef __cplusplus
}
#endif
#endif
