// Host-side launchers of the gfx950 kernels. Every launcher enqueues on the
// given stream and returns the launch status; shapes are validated by the
// C-ABI layer (abi.hip) before any launcher is called.
#pragma once

#include "common.h"

namespace rsllm_hip {

inline size_t block_elems_of(uint32_t t) {
    switch (t) {
    case T_F32: case T_F16: case T_BF16: return 1;
    case T_Q4_0: case T_Q4_1: case T_Q8_0: return 32;
    case T_Q2_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_Q8_K: case T_IQ2_XXS: return 256;
    default: return 0;
    }
}

inline size_t block_bytes_of(uint32_t t) {
    switch (t) {
    case T_F32: return 4;
    case T_F16: case T_BF16: return 2;
    case T_Q4_0: return 18;
    case T_Q4_1: return 20;
    case T_Q8_0: return 34;
    case T_Q2_K: return 84;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_Q8_K: return 292;
    case T_IQ2_XXS: return 66;
    default: return 0;
    }
}

inline size_t row_bytes_of(uint32_t t, size_t in_dim) {
    const size_t be = block_elems_of(t);
    return be ? in_dim / be * block_bytes_of(t) : 0;
}

// dequant.hip
hipError_t launch_dequant(uint32_t dtype, const uint8_t *src, float *dst, size_t n_elems,
                          hipStream_t s);
// GGUF rows -> device layout (dst must not alias src, except for Q4_K).
hipError_t launch_prepare(uint32_t dtype, const uint8_t *src, uint8_t *dst, size_t rows,
                          size_t in_dim, hipStream_t s);
// The same over n_blocks consecutive blocks. The layout packs 8 blocks per
// super-tile from the first block on (the last one may be shorter), so a
// matrix converted in pieces that start on multiples of 8 blocks, at the
// same byte offsets, is byte-identical to the matrix converted whole.
hipError_t launch_prepare_blocks(uint32_t dtype, const uint8_t *src, uint8_t *dst,
                                 size_t n_blocks, hipStream_t s);
// Formats whose device layout differs from the GGUF bytes.
inline bool layout_converted(uint32_t t) {
    return t == T_Q6_K || t == T_Q8_0 || t == T_Q4_0 || t == T_Q2_K || t == T_IQ2_XXS;
}

// gemv.hip: y[t, o] = sum_i W[o, i] x[t, i] for t < n_tok, W (w_bytes bytes)
// in device layout. Batch 1 is one launch that quantises x in LDS; 5..32
// tokens of Q4_K / Q6_K and 9..32 of Q8_0 run on the matrix cores
// (gemv_mfma.hip); more than 32 tokens (prefill) of Q4_K run the prefill GEMM
// (prefill.hip), of Q6_K / Q8_0 the matrix-core GEMV in 32-token chunks;
// other batches run the activation pre-pass, then the GEMV. `xq_scratch`
// must hold gemv_work_bytes(dtype, n_tok, in_dim, out_dim) bytes.
hipError_t launch_gemv(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                       uint8_t *xq_scratch, float *y, int n_tok, int in_dim, int out_dim,
                       hipStream_t s);
size_t gemv_scratch_bytes(uint32_t dtype, int n_tok, int in_dim);
// Scratch launch_gemv needs for this call (>= gemv_scratch_bytes; the MFMA
// path for 2..32 tokens keeps f16 activations there).
size_t gemv_work_bytes(uint32_t dtype, int n_tok, int in_dim, int out_dim);

// gemv.hip, caller chain (weight.rs:113-266): f32 weights
// (WeightBlob::F32) and quantized rows with strided / grouped x and y:
// y[t * y_stride + r] = sum_i W[r, i] x[t * x_stride + (r / rows_per_group)
// * in_dim + i], x_dim = n_groups * in_dim values of x per token.
// launch_gemv_rows (weights in the whole matrix's device layout; tokens in
// chunks of up to 8, one pass over the weights each) returns
// hipErrorNotSupported when one group's x is too long for LDS
// (gemv_rows_fits is false).
hipError_t launch_gemv_f32(const float *w, const float *x, float *y, int n_tok, int in_dim,
                           int out_dim, int x_dim, int x_stride, int y_stride, int rows_per_group,
                           hipStream_t s);
hipError_t launch_gemv_rows(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            float *y, int n_tok, int in_dim, int out_dim, int x_dim, int x_stride,
                            int y_stride, int rows_per_group, hipStream_t s);
bool gemv_rows_fits(uint32_t dtype, int in_dim);
// Two matrices of `rows` rows and in_dim columns (device layouts of their
// own, w_bytes each) on one x [n_tok x in_dim]: y[t * y_stride + r] for
// r < rows from w0, y[t * y_stride + rows + r] from w1. Same token chunks
// and hipErrorNotSupported as launch_gemv_rows.
hipError_t launch_gemv_pair(uint32_t dtype, const uint8_t *w0, const uint8_t *w1, size_t w_bytes,
                            const float *x, float *y, int n_tok, int in_dim, int rows,
                            int y_stride, hipStream_t s);

// gemv_mfma.hip: the same product for 5..32 tokens of Q4_K / Q6_K (9..32 of
// Q8_0) on the matrix cores (weights dequantised to f16 once, tokens as the
// MFMA's N).
bool gemv_mfma_supported(uint32_t dtype, int n_tok, int in_dim, int out_dim);
size_t gemv_mfma_scratch_bytes(uint32_t dtype, int n_tok, int in_dim, int out_dim);
hipError_t launch_gemv_mfma(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            uint8_t *scratch, float *y, int n_tok, int in_dim, int out_dim,
                            hipStream_t s);
// The two halves of launch_gemv: the activation pre-pass (format-specific
// int8 two-limb layout) and the GEMV on pre-quantised activations.
hipError_t launch_quantize_x(uint32_t dtype, const float *x, uint8_t *xq, int n_tok, int in_dim,
                             hipStream_t s);
hipError_t launch_gemv_prequant(uint32_t dtype, const uint8_t *w, size_t w_bytes,
                                const uint8_t *xq, float *y, int n_tok, int in_dim, int out_dim,
                                hipStream_t s);

// Grouped GEMV for routed experts (gemv.hip): slots sorted by expert,
// expert e owns slots [off[e], off[e+1]) (off on the device, n_expert + 1
// entries). For each slot s: y_m[s * out_dim + o] = sum_i W_m[e][o, i] *
// x~[row(s), i], m = 0 (w0 -> y0) and, when w1 is given, m = 1 (w1 -> y1);
// W_m[e] starts at w_m + e * w_stride (device layout); row(s) = tok[s], or s
// when tok is null; xq holds the activation limbs of those rows
// (launch_quantize_x layout, xq_bytes bytes). Workgroup row y of the grid
// (grid_experts rows) serves expert act[y] when y < *n_act.
hipError_t launch_gemv_grouped(uint32_t dtype, const uint8_t *w0, const uint8_t *w1,
                               size_t w_stride, const uint8_t *xq, size_t xq_bytes,
                               const int *off, const int *tok, const int *act, const int *n_act,
                               int grid_experts, float *y0, float *y1, int in_dim, int out_dim,
                               hipStream_t s);
// launch_quantize_x applied to silu(min(g, c)) * clamp(u, -c, c) of the
// first min(n_rows, off[n_expert]) rows of hg, hu ([n_rows x n]).
hipError_t launch_quantize_swiglu(uint32_t dtype, const float *hg, const float *hu, float clamp,
                                  uint8_t *xq, int n_rows, int n, const int *off, int n_expert,
                                  hipStream_t s);

// gemv_mfma.hip, routed experts on the matrix cores (Q4_K, Q6_K or Q8_0
// gate/up and down; n_embd and n_ff multiples of 256). Slots sorted by
// expert as launch_gemv_grouped's (off: n_expert + 1 entries on the device,
// slot_tok: the token of each sorted slot, n_pairs = n_tok * k bounding the
// slot count). Writes hg, hu [slot x n_ff] (gate and up of
// x[slot_tok[slot]]) and yd [slot x n_embd] (down of the clamped SwiGLU of
// hg, hu). The batches: each active expert's sorted slots cut into runs of
// up to mfg_width(n_pairs, n_expert) (experts ascending, runs in slot
// order), *n_bat of them, as k_moe_scan lists them; at most
// mfg_max_batches(n_pairs, n_expert, width). With `route` (calls of up to
// kRoute1Pairs pairs) the first launch also runs the one-workgroup routing
// that writes off, slot_tok, slot_of, the active experts and the batches;
// without it the caller has routed. `scratch` holds
// moe_mfma_scratch_bytes(n_pairs, n_expert, n_embd, n_ff) bytes: the batch
// list and its count first (mfg_batch_bytes; bat, n_bat point there), then
// the activation images.
constexpr int kMfgBatch = 16;
struct MfgBatch {
    int first, count, expert, pad;
};
struct MoeRoute1Args;
// Batch width of the grouped routed-expert route: 8 slots (the packed
// 8-column kernel) when the experts average at most 8 slots, else 16.
inline int mfg_width(int n_pairs, int n_expert) {
    return (long long)n_pairs <= 8LL * n_expert ? 8 : kMfgBatch;
}
inline int mfg_max_batches(int n_pairs, int n_expert, int width) {
    return (n_pairs + width - 1) / width + (n_pairs < n_expert ? n_pairs : n_expert);
}
inline size_t mfg_batch_bytes(int n_pairs, int n_expert, int width) {
    return ((size_t)mfg_max_batches(n_pairs, n_expert, width) * sizeof(MfgBatch) + 255) / 256 * 256 +
           256;
}
bool moe_mfma_supported(uint32_t dt_gu, uint32_t dt_d, int n_embd, int n_ff);
// the images' byte offsets fit 32 bits
bool moe_mfma_fits(int n_pairs, int n_embd, int n_ff);
size_t moe_mfma_scratch_bytes(int n_pairs, int n_expert, int n_embd, int n_ff);
hipError_t launch_moe_mfma(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                           const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                           int n_tok, const MoeRoute1Args *route, const int *off,
                           const int *slot_tok, MfgBatch *bat, int *n_bat, int n_pairs,
                           int n_expert, float *hg, float *hu, float *yd, uint8_t *scratch,
                           int n_embd, int n_ff, float clamp, hipStream_t s);

// gemv_mfma.hip, matmul_grouped_lora_down on the matrix cores: y[t *
// y_stride + g * R + r] = sum_i W[g R + r, i] x[t * x_stride + g * D + i]
// for a stacked Q4_K / Q6_K / Q8_0 matrix of G * R rows (device layout as
// one matrix, w_bytes < 4 GiB), 9 or more tokens, D a multiple of 256, R of
// 64, G * R >= 1024 (lora_mfma_supported). `scratch` holds
// lora_mfma_scratch_bytes(n_tok, D, G) bytes. hipErrorNotSupported outside
// those shapes.
bool lora_mfma_supported(uint32_t dtype, int n_tok, int D, int G, int R);
size_t lora_mfma_scratch_bytes(int n_tok, int D, int G);
hipError_t launch_lora_mfma(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            int x_stride, float *y, int y_stride, uint8_t *scratch, int n_tok,
                            int D, int G, int R, hipStream_t s);

// prefill.hip: out[t, o] = sum_i deq(W)[o, i] * x[t, i] for a raw GGUF Q4_K
// weight W [out_dim x in_dim] and bf16 activations x [n_tok x in_dim]
// (n_tok x out_dim fp32 output, overwritten). `scratch` holds
// prefill_scratch_bytes(n_tok, in_dim, out_dim) bytes (scaled f16
// activations, per-token scales, and the partial sums of a call whose K is
// split across workgroups).
size_t prefill_scratch_bytes(int n_tok, int in_dim, int out_dim);
hipError_t launch_prefill_q4k(const uint8_t *w, size_t w_bytes, const uint16_t *x_bf16,
                              uint8_t *scratch, float *out, int n_tok, int in_dim, int out_dim,
                              hipStream_t s);
// The same GEMM on f32 activations x [n_tok x in_dim] (16-byte aligned; w
// 16-byte aligned) for a Q4_K weight (GGUF bytes) or a Q8_0 weight (device
// layout), in_dim a multiple of 256: each element of x rounded once to f16
// after the per-token 2^e scaling. Same scratch.
hipError_t launch_prefill_f32(uint32_t dtype, const uint8_t *w, const float *x, uint8_t *scratch,
                              float *out, int n_tok, int in_dim, int out_dim, hipStream_t s);

// moe.hip: routed experts (accumulate_moe_outputs). Expert e of gate/up is
// at gate/up + e * gu_stride, of down at down + e * d_stride (device
// layout); ids, wts: [n_tok x k] on the device; out [n_tok x n_embd] is
// accumulated into. `scratch` holds moe_scratch_bytes(...) bytes.
size_t moe_scratch_bytes(uint32_t dt_gu, uint32_t dt_d, int n_tok, int k, int n_expert,
                         int n_embd, int n_ff);
hipError_t launch_moe(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                      const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                      const int *ids, const float *wts, float *out, uint8_t *scratch, int n_tok,
                      int k, int n_expert, int n_embd, int n_ff, float clamp, hipStream_t s);

// moe.hip, shared expert: elementwise clamped SwiGLU a = silu(min(g, c)) *
// clamp(u, -c, c) (no clamp when c <= 1e-6).
hipError_t launch_swiglu(const float *g, const float *u, float *a, size_t n, float c,
                         hipStream_t s);
// a[t * n + i] = SwiGLU(h[t * 2n + i], h[t * 2n + n + i]) (gate and up side
// by side per token, as launch_gemv_pair writes them).
hipError_t launch_swiglu_pair(const float *h, float *a, int n_tok, int n, float c, hipStream_t s);

// q8_int8.hip: the Q8_0 int8-activation path. launch_q8_quantize writes
// xq [n_tok x blocks x 32] int8 and scale [n_tok x blocks] (blocks =
// ceil(in_dim / 32)) and ORs 1 into *status (if non-null) when a token has
// a non-finite input. launch_q8_int8_matmul: out [n_tok x out_dim] from Q8_0
// weights in the device layout (w_bytes bytes) and those activations.
hipError_t launch_q8_quantize(const float *x, int8_t *xq, float *scale, int n_tok, int in_dim,
                              int *status, hipStream_t s);
hipError_t launch_q8_int8_matmul(const uint8_t *w, size_t w_bytes, const int8_t *xq,
                                 const float *xscale, float *out, int n_tok, int in_dim,
                                 int out_dim, hipStream_t s);

// Largest weight tensor the buffer-addressed kernels accept (offsets are
// 32-bit).
constexpr size_t kMaxWeightBytes = 0xFFFFFF00u;

// Fill n floats with zero (used for in_dim == 0; no hipMemset so the call
// stays capturable into a graph).
hipError_t launch_fill_zero(float *y, size_t n, hipStream_t s);

}  // namespace rsllm_hip
