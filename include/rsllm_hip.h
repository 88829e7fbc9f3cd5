/*
 * rsllm_hip.h — C ABI of the MI355X (gfx950) quantized mat-vec / mat-mul
 * backend for rsLLM.
 *
 * Each entry point replaces one function of the reference's CPU path
 * (citations: paths relative to the rsLLM tree, crates/<crate>/src/...).
 * Arguments keep the reference's meaning and order; slices become
 * (pointer, length) pairs so the same length checks can run here, in the
 * same order, with the same error classes.
 *
 * Two flavours:
 *   - host-pointer entry points: synchronous drop-ins for the Rust functions
 *     (buffers are caller-owned host memory; `out` is valid on return);
 *   - `_dev` entry points: device pointers, enqueued on the caller's
 *     hipStream_t, no host synchronisation.
 *
 * Weights in device memory are in the "device layout" written by
 * rsllm_hip_prepare_weights_dev: for Q4_K it is the GGUF byte stream
 * itself; Q6_K / Q8_0 / Q4_0 / Q2_K / IQ2_XXS matrices are regrouped into
 * 8-block super-tiles of the same total size (see
 * rsllm_hip_prepare_weights_dev).
 *
 * Thread safety: every entry point may be called from any thread, as
 * CpuBackend (backend-cpu/src/lib.rs:42-45) may. Process state (device
 * ordinal, the registry of device copies) is guarded by a mutex, and the
 * registry is a hash map keyed by host address. Each calling thread gets its
 * own stream and host<->device staging for the host-pointer entry points.
 * The kernels' device workspace belongs to a stream: one set per (device,
 * stream), used by every call enqueued on that stream and locked while a
 * call enqueues, so calls on different streams never share workspace and
 * threads sharing a stream take turns. A call that uses a registered or
 * model-resident tensor holds a reference to its device memory until it has
 * synchronised, so a release on another thread never frees memory under it.
 * Device pointers a caller obtained itself (rsllm_hip_model_tensor) are the
 * caller's to keep alive: release a model only after work using them ends.
 */
#ifndef RSLLM_HIP_H
#define RSLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque stream handle: a hipStream_t (NULL = the default stream). */
typedef void *rsllm_hip_stream_t;

/* Status codes. 1..4 mirror rsllm_backend_cpu::Error
 * (backend-cpu/src/error.rs:7-43), 5..6 mirror rsllm_gguf::Error's
 * dequant variants (rsllm-gguf/src/error.rs:69-80). */
typedef enum rsllm_hip_status {
    RSLLM_HIP_OK = 0,
    RSLLM_HIP_ERR_SHAPE_MISMATCH = 1,        /* Error::ShapeMismatch(&str) */
    RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED = 2,     /* Error::NotBlockAligned{what,actual,block} */
    RSLLM_HIP_ERR_NON_FINITE_INPUT = 3,      /* Error::NonFiniteInput(&str) */
    RSLLM_HIP_ERR_UNSUPPORTED_TIER = 4,      /* Error::UnsupportedTier(&str) */
    RSLLM_HIP_ERR_DEQUANT_SIZE_MISMATCH = 5, /* Error::DequantSizeMismatch{src_bytes,expected_bytes} */
    RSLLM_HIP_ERR_UNSUPPORTED_DEQUANT = 6,   /* Error::UnsupportedDequant(name) */
    RSLLM_HIP_ERR_DEVICE = 7,                /* a HIP runtime call failed (no reference counterpart) */
    RSLLM_HIP_ERR_INVALID_ARGUMENT = 8,      /* NULL pointer with nonzero length, or a shape the
                                                reference would panic on (row_len == 0 in
                                                parallel.rs:44) */
    RSLLM_HIP_ERR_UNIMPLEMENTED = 10         /* a call the reference accepts but this backend
                                                does not serve (e.g. the Q4_K-only prefill entry
                                                given another dtype) */
} rsllm_hip_status;

/* GgmlType ids (rsllm-gguf/src/tensor.rs:26-85) used by this ABI. */
enum {
    RSLLM_GGML_F32 = 0, RSLLM_GGML_F16 = 1, RSLLM_GGML_Q4_0 = 2, RSLLM_GGML_Q4_1 = 3,
    RSLLM_GGML_Q8_0 = 8, RSLLM_GGML_Q2_K = 10, RSLLM_GGML_Q4_K = 12, RSLLM_GGML_Q5_K = 13,
    RSLLM_GGML_Q6_K = 14, RSLLM_GGML_Q8_K = 15, RSLLM_GGML_IQ2_XXS = 16, RSLLM_GGML_BF16 = 30
};

/* Details of the last error on the calling thread.
 * what/actual/block: NotBlockAligned (error.rs:18-25);
 * src_bytes/expected_bytes: DequantSizeMismatch (gguf error.rs:71-76). */
typedef struct rsllm_hip_error_detail {
    int32_t status;
    const char *message; /* the reference's message text where it has one */
    const char *what;
    size_t actual, block;
    size_t src_bytes, expected_bytes;
} rsllm_hip_error_detail;

void rsllm_hip_last_error(rsllm_hip_error_detail *out);

/* No reference counterpart; a diagnostic: the number of device allocations
 * (hipMalloc) the library has made in this process so far (workspace sets,
 * staging, registered tensors, model arenas). It only grows. */
uint64_t rsllm_hip_device_allocations(void);

/* Backend handle analogue: CpuBackend::new (backend-cpu/src/lib.rs:50-53)
 * plus device choice. Optional; the first call of any entry point performs
 * it with device 0. */
int rsllm_hip_init(int device_ordinal);

/* BackendCapability analogue (rsllm-cal/src/lib.rs:62-75,
 * backend-cpu/src/capability.rs:119-131). */
typedef struct rsllm_hip_capability {
    const char *backend; /* "rocm" */
    const char *arch;    /* "gfx950" */
    int q4k_matmul, q6k_matmul, q8_0_matmul, q2k_matmul, iq2xxs_matmul, fp8_kv_cache;
} rsllm_hip_capability;
void rsllm_hip_capability_get(rsllm_hip_capability *out);

/* ---- quantized matmul --------------------------------------------------- */

/* matmul_quant_f32 (backend-cpu/src/ops/quant_matmul.rs:45-119).
 * out[t*out_dim + o] = sum_i deq(W)[o, i] * x[t*in_dim + i]; `out` is
 * overwritten. Validation order as :57-92: dtype, in_dim % block,
 * weights_len, x_len, out_len. Accepted dtypes: Q4_K, Q2_K, IQ2_XXS, Q4_0,
 * Q8_0 (the reference's guard), and Q6_K (a deliberate superset: the
 * reference's guard rejects Q6_K). `tier` is
 * accepted and ignored, as the reference ignores it (:55).
 * Weights are uploaded for this call unless the same (pointer, length,
 * dtype, in_dim) was registered with rsllm_hip_register_weights. */
int rsllm_hip_matmul_quant_f32(float *out, size_t out_len, const uint8_t *weights,
                               size_t weights_len, const float *x, size_t x_len, size_t n_tok,
                               size_t in_dim, size_t out_dim, uint32_t dtype, uint32_t tier);

/* Device-pointer matmul_quant_f32: same validation; `weights` in device
 * layout; enqueued on `stream`. */
int rsllm_hip_matmul_quant_f32_dev(float *out, size_t out_len, const uint8_t *weights,
                                   size_t weights_len, const float *x, size_t x_len,
                                   size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                   rsllm_hip_stream_t stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (work under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc): rsllm_hip_matmul_quant_f32_dev with the same arguments,
 * validation and results, whose activation workspace is a static array of
 * RSLLM_HIP_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends)
 * instead of memory the library allocates; the call itself allocates and
 * frees nothing. A call whose workspace would exceed that size (many tokens
 * of a long row) returns RSLLM_HIP_ERR_INVALID_ARGUMENT. Every call on one
 * GPU shares its array and leaves its contents behind: calls that overlap in
 * time on one GPU (two streams, or two threads) race on it, so enqueue them
 * on one stream. */
#define RSLLM_HIP_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
int rsllm_hip_matmul_quant_f32_dev_noalloc(float *out, size_t out_len, const uint8_t *weights,
                                           size_t weights_len, const float *x, size_t x_len,
                                           size_t n_tok, size_t in_dim, size_t out_dim,
                                           uint32_t dtype, rsllm_hip_stream_t stream);

/* Activations pre-quantised for the GEMV kernels, for callers that reuse one
 * x across several weight matrices of the same dtype and in_dim (e.g. an
 * FFN's gate and up projections) or time the GEMV alone. No reference
 * counterpart: matmul_quant_f32 takes f32 x directly. x is re-expressed per
 * 16-element group as s * (256 h + l) with int8 limbs (about 16 bits
 * relative to the group's largest element) in a dtype-specific lane-major
 * layout of rsllm_hip_xq_bytes(dtype, n_tok, in_dim) bytes.
 * rsllm_hip_matmul_prequant_dev is rsllm_hip_matmul_quant_f32_dev with xq in
 * place of x (same validation, x_len replaced by xq_len). The products are
 * the same; the summation order can differ from the one-shot call's kernel,
 * so the two agree to a few ulp, not bit for bit. */
size_t rsllm_hip_xq_bytes(uint32_t dtype, size_t n_tok, size_t in_dim);
int rsllm_hip_quantize_x_dev(uint32_t dtype, const float *x, size_t x_len, size_t n_tok,
                             size_t in_dim, uint8_t *xq, size_t xq_len, rsllm_hip_stream_t stream);
int rsllm_hip_matmul_prequant_dev(float *out, size_t out_len, const uint8_t *weights,
                                  size_t weights_len, const uint8_t *xq, size_t xq_len,
                                  size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                  rsllm_hip_stream_t stream);

/* ---- weights residency ----------------------------------------------------
 * The reference borrows weights from the GGUF mmap for the life of the
 * GgufFile (rsllm-gguf/src/file.rs:81-97, models/src/dsv4/loader.rs:199-216).
 * Registering uploads a tensor once (converted to the device layout);
 * later host-pointer calls with the same (pointer, length, dtype, in_dim)
 * use the device copy. Release removes every registered tensor; the device
 * copy of one that a call on another thread is using is freed when that call
 * ends. */
int rsllm_hip_register_weights(const uint8_t *weights, size_t weights_len, uint32_t dtype,
                               size_t in_dim);
int rsllm_hip_release_weights(void);

/* No reference counterpart (the reference has no streams): frees the device
 * workspace the library keeps for `stream` on the current device, for a
 * caller about to destroy that stream. Work still enqueued there finishes
 * first (hipFree waits for the device); a later call on the stream makes a
 * new set. hipStreamPerThread names a different stream in each thread, so
 * each thread that passes it gets a set of its own, and releasing it frees
 * only the calling thread's set. */
int rsllm_hip_stream_release(rsllm_hip_stream_t stream);

/* ---- whole-model residency ---------------------------------------------------
 * No single reference function: this replaces keeping weights only in the
 * GGUF mmap (GgufFile::open, rsllm-gguf/src/file.rs:81-97; tensor_bytes
 * :181-187; resolve_blob, models/src/dsv4/loader.rs:199-216) when the
 * matmuls run on the GPU. The caller lists every tensor once, after opening
 * the file:
 *   name    TensorInfo::name;
 *   data    GgufFile::tensor_bytes (host memory, e.g. inside the mmap);
 *   len     its byte length;
 *   dtype   TensorInfo::raw_type (GgmlType id);
 *   in_dim  row length (shape[0]) for tensors used as matmul weights (F32 or
 *           a matmul format), else 0.
 * rsllm_hip_model_upload copies all of them into one device allocation, in
 * list order (each 256-byte aligned, so stacked expert tensors stay
 * contiguous), through pinned staging, converting matmul tensors (in_dim !=
 * 0) to the device layout; the rest are copied as is. Matmul tensors are
 * registered under their
 * host range, like rsllm_hip_register_weights, so the host-pointer entry
 * points use the resident copy. An upload whose fingerprint
 * (GgufFile::fingerprint, file.rs:175-177: names, types and shapes only),
 * tensor table and payload match a live model on the same device returns
 * that model, adds a reference and registers the new host ranges, without
 * copying. The payload comparison is a 64-bit hash of every byte (taken by
 * the copy threads during an upload; for a candidate that also matches a
 * 16-window sampled digest, over the new bytes by a host read pass), so
 * files that differ anywhere get separate models. Errors, all before any
 * device work: INVALID_ARGUMENT for
 * NULL arguments or duplicate names, SHAPE_MISMATCH for a matmul tensor
 * whose length is not whole rows of a block-aligned in_dim. Uploads are
 * serialised with each other and with the lookups below.
 * rsllm_hip_model_tensor returns a tensor's device address and length (the
 * device-layout bytes the _dev entry points take). rsllm_hip_model_release
 * drops one reference; the last one removes the registrations, and the
 * allocation is freed once no host-pointer call in flight still uses one of
 * its tensors. `_dev` work on addresses from rsllm_hip_model_tensor must end
 * before the last release. rsllm_hip_release_weights does not touch
 * models. */
typedef struct rsllm_hip_tensor_desc {
    const char *name;
    const uint8_t *data;
    size_t len;
    uint32_t dtype;
    size_t in_dim;
} rsllm_hip_tensor_desc;

typedef struct rsllm_hip_model_info {
    uint64_t device_bytes;   /* size of the model's device allocation */
    uint64_t uploaded_bytes; /* payload bytes copied when it was uploaded */
    double upload_seconds;   /* wall time of that upload */
    uint32_t refs, n_tensors;
} rsllm_hip_model_info;

int rsllm_hip_model_upload(const uint8_t *fingerprint /* 32 bytes */,
                           const rsllm_hip_tensor_desc *tensors, size_t n_tensors,
                           uint64_t *model);
int rsllm_hip_model_tensor(uint64_t model, const char *name, const uint8_t **dev, size_t *len);
int rsllm_hip_model_info_get(uint64_t model, rsllm_hip_model_info *out);
int rsllm_hip_model_release(uint64_t model);

/* GGUF rows -> device layout: `len` bytes holding whole rows of `in_dim`
 * elements (n = len / block_bytes blocks in matrix order, row-major over
 * (row, block)). Q4_K: unchanged (`dst` may equal `src`). Q6_K, Q8_0, Q4_0,
 * Q2_K, IQ2_XXS: the blocks are regrouped into super-tiles of 8 consecutive
 * blocks (the last tile holds the n % 8 remaining blocks, r of them), each
 * tile split into field runs so that every field of every block is aligned:
 *   Q6_K    [ql r*128 | qh r*64 | scales r*16 | d r*2]   (8 blocks: 1680 B)
 *   Q8_0    [qs r*32 | d r*2]                           (8 blocks: 272 B)
 *   Q4_0    [qs r*16 | d r*2]                           (8 blocks: 144 B)
 *   Q2_K    [qs r*64 | scales r*16 | (d, dmin) r*4]     (8 blocks: 672 B)
 *   IQ2_XXS [qs r*64 | d r*2]                           (8 blocks: 528 B)
 * with r = 8 except in the last tile; tile S starts at byte
 * S * 8 * block_bytes. `dst` must not overlap `src`. Enqueued on `stream`. */
int rsllm_hip_prepare_weights_dev(uint8_t *dst, const uint8_t *src, size_t len, uint32_t dtype,
                                  size_t in_dim, rsllm_hip_stream_t stream);

/* ---- prefill GEMM (bf16 activations) ---------------------------------------
 * The prefill form of matmul_quant_f32 (backend-cpu/src/ops/quant_matmul.rs:
 * 45-119, called from models/src/engine_impl.rs:277 prefill with n_tok = T):
 * out[t * out_dim + o] = sum_i deq(W)[o, i] * f32(x[t * in_dim + i]) for a
 * GGUF Q4_K weight (device copy of the GGUF bytes) and bf16 activations
 * (x_len = n_tok * in_dim 16-bit patterns). Runs on the matrix cores
 * (f16 MFMA, fp32 accumulation); within 1e-3 (max|d|/max|y|) of the
 * reference on f32(x). Validation as matmul_quant_f32 (dtype -> in_dim %
 * 256 -> weights -> x -> out); dtypes other than Q4_K return
 * RSLLM_HIP_ERR_UNIMPLEMENTED. Uses a per-thread device workspace of about
 * 2 * n_tok * in_dim bytes; enqueued on `stream`. */
int rsllm_hip_matmul_q4k_bf16_dev(float *out, size_t out_len, const uint8_t *weights,
                                  size_t weights_len, const uint16_t *x_bf16, size_t x_len,
                                  size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                  rsllm_hip_stream_t stream);

/* ---- routed experts (MoE) ---------------------------------------------------
 * accumulate_moe_outputs (models/src/dsv4/moe.rs:648-707) with
 * apply_expert_swiglu (:479-502) and apply_swiglu_clamp (:515-531): for
 * every token t and slot i with weights[t*k+i] != 0 and e = ids[t*k+i]:
 *   out[t] += weights[t*k+i] * down[e] (silu(min(gate[e] x_t, c)) *
 *                                       clamp(up[e] x_t, -c, c))
 * with the clamp applied only when c > 1e-6 (NaN passes through), slots
 * accumulated in i order. `out` [n_tok x n_embd] is ACCUMULATED into (the
 * caller pre-clears or pre-fills it, as the reference's caller does).
 * gate, up: n_expert stacked [n_ff x n_embd] matrices of dtype_gate_up
 * (gate_up_len bytes each blob); down: n_expert stacked [n_embd x n_ff]
 * matrices of dtype_down (StackedExperts::expert, moe.rs:69-108). Q4_K
 * blobs are the GGUF bytes; other dtypes are in the device layout
 * (rsllm_hip_prepare_weights_dev over the whole blob), which needs each
 * expert's block count to be a multiple of 8. ids, weights: n_tok * k.
 * Validation: dtypes, then n_embd % block(gate/up) and n_ff % block(down)
 * (NotBlockAligned), blob lengths, x, out, ids lengths (ShapeMismatch);
 * n_expert <= 16384. Any number of tokens (the reference's prefill passes
 * every token of the forward pass, moe.rs:281,346): calls of more than 8192
 * (token, slot) pairs run in token chunks, each routed and computed on its
 * own, which gives the same result. The reference panics on an expert id
 * out of range: the host entry point returns RSLLM_HIP_ERR_INVALID_ARGUMENT,
 * the device entry point (which cannot inspect ids) skips such slots. Uses
 * the stream's device workspace. */
int rsllm_hip_moe_routed_dev(float *out, size_t out_len, const float *x, size_t x_len,
                             const uint8_t *gate, const uint8_t *up, size_t gate_up_len,
                             const uint8_t *down, size_t down_len, const int32_t *ids,
                             const float *weights, size_t ids_len, size_t n_tok, size_t n_embd,
                             size_t n_ff, size_t n_expert, size_t k, uint32_t dtype_gate_up,
                             uint32_t dtype_down, float clamp, rsllm_hip_stream_t stream);
/* Host-pointer form (synchronous). Expert blobs registered with
 * rsllm_hip_register_weights (in_dim n_embd for gate/up, n_ff for down) are
 * used from the device; otherwise they are uploaded for the call. */
int rsllm_hip_moe_routed(float *out, size_t out_len, const float *x, size_t x_len,
                         const uint8_t *gate, const uint8_t *up, size_t gate_up_len,
                         const uint8_t *down, size_t down_len, const int32_t *ids,
                         const float *weights, size_t ids_len, size_t n_tok, size_t n_embd,
                         size_t n_ff, size_t n_expert, size_t k, uint32_t dtype_gate_up,
                         uint32_t dtype_down, float clamp);

/* ---- caller chain: matmul_weight_f32, matmul_grouped_lora_down ------------
 * rsllm_hip_matmul_weight_f32 replaces matmul_weight_f32
 * (rsllm-models/src/dsv4/weight.rs:113-169): out[t, o] = sum_i W[o, i] x[t, i]
 * for a WeightBlob. dtype 0 (GGML F32) is the F32 arm: `weights` holds
 * out_dim * in_dim f32 values, weights_len counts bytes (out_dim * in_dim *
 * 4). Any other dtype is the Quant arm, matmul_quant_f32 on the blob.
 * Validation in the reference's order:
 *   out_len != n_tok * out_dim            SHAPE_MISMATCH (matmul_weight_f32.out)
 *   x_len != n_tok * in_dim               SHAPE_MISMATCH (matmul_weight_f32.x)
 *   F32: weights_len != out_dim*in_dim*4  SHAPE_MISMATCH (.weight_f32)
 *   Quant: every error of matmul_quant_f32 (dtype, block alignment,
 *          lengths) becomes SHAPE_MISMATCH (.quant), as the reference maps
 *          it; out_dim == 0 (a panic there) is INVALID_ARGUMENT.
 *
 * rsllm_hip_matmul_grouped_lora_down replaces matmul_grouped_lora_down
 * (weight.rs:209-266): x is [n_tok x n_groups * group_dim], out
 * [n_tok x n_groups * rank], weights n_groups stacked [rank x group_dim]
 * row-major matrices (the [n_groups * rank x group_dim] matrix), F32 or a
 * quant dtype as above; out[t, g * rank + o] = sum_i W_g[o, i]
 * x[t, g * group_dim + i]. Validation: x length (.x), out length (.out),
 * then for the groups grouped_weight_slice (weight.rs:271-323: group_dim *
 * rank a multiple of the block (.alignment), each group's slice inside the
 * blob (.f32 / .quant)) and the group's matmul_weight_f32 checks, all
 * SHAPE_MISMATCH; n_groups == 0 is OK. The reference computes group by group
 * and can fail on a later group's slice after writing earlier groups; here
 * every check runs before anything is written.
 *
 * Device forms: weights in this backend's device layout (Quant arm:
 * rsllm_hip_prepare_weights_dev of the [n_groups * rank x group_dim]
 * matrix; F32: as is), x and out on the device, enqueued on `stream`. Each
 * chunk of up to 8 tokens is one launch for all groups (each workgroup holds
 * one group's x in LDS). A group_dim too long for that (over about 60k
 * elements for the 256-element formats) runs each group as its own launch
 * on gathered x, which needs the group to be a whole number of 8-block
 * super-tiles of the device layout (non-Q4_K dtypes: rank * group_dim /
 * block elements a multiple of 8). For such groups that are not, the host
 * form converts each group to the device layout on its own, and the device
 * form returns RSLLM_HIP_ERR_UNIMPLEMENTED (writing nothing). The host form
 * uses a registered copy of the blob only when the groups use all of it and
 * it is not converted group by group. */
int rsllm_hip_matmul_weight_f32(float *out, size_t out_len, const uint8_t *weights,
                                size_t weights_len, const float *x, size_t x_len, size_t n_tok,
                                size_t in_dim, size_t out_dim, uint32_t dtype);
int rsllm_hip_matmul_weight_f32_dev(float *out, size_t out_len, const uint8_t *weights,
                                    size_t weights_len, const float *x, size_t x_len,
                                    size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                    rsllm_hip_stream_t stream);
int rsllm_hip_matmul_grouped_lora_down(float *out, size_t out_len, const uint8_t *weights,
                                       size_t weights_len, const float *x, size_t x_len,
                                       size_t n_tok, size_t n_groups, size_t group_dim,
                                       size_t rank, uint32_t dtype);
int rsllm_hip_matmul_grouped_lora_down_dev(float *out, size_t out_len, const uint8_t *weights,
                                           size_t weights_len, const float *x, size_t x_len,
                                           size_t n_tok, size_t n_groups, size_t group_dim,
                                           size_t rank, uint32_t dtype,
                                           rsllm_hip_stream_t stream);

/* ---- shared expert: apply_shared_expert / apply_expert_swiglu ---------------
 * rsllm_hip_apply_shared_expert replaces apply_shared_expert
 * (rsllm-models/src/dsv4/moe.rs:422-455): every token t of x [n_tok x
 * n_embd] through apply_expert_swiglu (:479-502),
 *   out[t] = down @ (silu(min(gate @ x[t], c)) * clamp(up @ x[t], -c, c)),
 * out [n_tok x n_embd] overwritten. apply_expert_swiglu on one token is the
 * n_tok = 1 call. gate and up are [n_ff x n_embd] and down [n_embd x n_ff]
 * WeightBlobs, each F32 (dtype 0, length in bytes) or a quant dtype of its
 * own; the clamp is skipped when clamp <= 1e-6 (apply_swiglu_clamp
 * :515-531, so 0 stands for the reference's None). Validation:
 * check_moe_shapes (:557-573) x_len then out_len (SHAPE_MISMATCH "moe.x" /
 * "moe.out"), then, if n_tok > 0, matmul_weight_f32's checks of the gate,
 * up and down calls in that order (as for rsllm_hip_matmul_weight_f32).
 * Gate and up of one quant format run as one GEMV launch per chunk of up to
 * 8 tokens (the two matrices as two row groups on the same x), then an
 * elementwise SwiGLU and the down GEMV; other combinations (F32 blobs,
 * mixed formats) run gate and up as separate GEMVs. Host blobs registered with
 * rsllm_hip_register_weights are used from the device.
 *
 * Device form: blobs in the device layout (rsllm_hip_prepare_weights_dev
 * for quant formats; F32 as is), enqueued on `stream`. */
int rsllm_hip_apply_shared_expert(float *out, size_t out_len, const float *x, size_t x_len,
                                  const uint8_t *gate, size_t gate_len, uint32_t dtype_gate,
                                  const uint8_t *up, size_t up_len, uint32_t dtype_up,
                                  const uint8_t *down, size_t down_len, uint32_t dtype_down,
                                  size_t n_tok, size_t n_embd, size_t n_ff, float clamp);
int rsllm_hip_apply_shared_expert_dev(float *out, size_t out_len, const float *x, size_t x_len,
                                      const uint8_t *gate, size_t gate_len, uint32_t dtype_gate,
                                      const uint8_t *up, size_t up_len, uint32_t dtype_up,
                                      const uint8_t *down, size_t down_len, uint32_t dtype_down,
                                      size_t n_tok, size_t n_embd, size_t n_ff, float clamp,
                                      rsllm_hip_stream_t stream);

/* ---- Q8_0 int8-activation path ---------------------------------------------
 * quantize_q8_0_batch (backend-cpu/src/ops/q8_0.rs:95-129, per token
 * quantize_q8_0_activation :42-88): x [n_tok x in_dim] -> xq [n_tok x blocks
 * x 32] int8 and scale [n_tok x blocks], blocks = ceil(in_dim / 32); per
 * block d = amax / 127, q = clamp(round_half_even(x / d), -128, 127) (x * (1
 * / d) exactly as the reference), a partial last block zero-padded.
 * Bit-exact with the reference. Validation order :101-118: x_len, xq_len,
 * scale_len (ShapeMismatch); in_dim == 0 is INVALID_ARGUMENT (the
 * reference's par_chunks_mut(0) panics). A non-finite input returns
 * RSLLM_HIP_ERR_NON_FINITE_INPUT (:67-69); xq and scale are then
 * unspecified. */
int rsllm_hip_quantize_q8_0_batch(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                                  float *scale, size_t scale_len, size_t n_tok, size_t in_dim);
/* Device-pointer form, enqueued on `stream`. Non-finite inputs cannot be
 * reported synchronously: when `status` (a device int32) is non-NULL it is
 * set to 0, or to 1 if any input was non-finite, once the work completes. */
int rsllm_hip_quantize_q8_0_batch_dev(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                                      float *scale, size_t scale_len, size_t n_tok,
                                      size_t in_dim, int32_t *status, rsllm_hip_stream_t stream);

/* matmul_q8_0_batch (backend-cpu/src/ops/q8_0.rs:217-263): out[t*out_dim + o]
 * = sum over blocks b, in order, of (wscale[o,b] * xscale[t,b]) * dot_i32(
 * wq[o,b], xq[t,b]) (dot_q8_0_row_scalar :163-193; a non-finite weight scale
 * counts as 0, :143-146; only the first in_dim - 32 b lanes of a partial
 * last block take part). `weights` are raw GGUF Q8_0 rows (out_dim * blocks
 * * 34 bytes, in_dim need not be a multiple of 32). Bit-exact with the
 * reference's scalar tier. Validation order :229-252: weights_len, xq_len,
 * xscale_len, out_len (ShapeMismatch); out_dim == 0 is INVALID_ARGUMENT
 * (parallel.rs:44). `tier` is accepted and ignored (the scalar result is
 * what every call returns). Weights are uploaded (and regrouped into the
 * device layout) for the call unless the same (pointer, length) was
 * registered as Q8_0 with this in_dim. */
int rsllm_hip_matmul_q8_0_batch(float *out, size_t out_len, const uint8_t *weights,
                                size_t weights_len, const int8_t *xq, size_t xq_len,
                                const float *xscale, size_t xscale_len, size_t n_tok,
                                size_t in_dim, size_t out_dim, uint32_t tier);
/* Device-pointer form, enqueued on `stream`: `weights` in the device layout
 * (rsllm_hip_prepare_weights_dev of the GGUF rows with in_dim rounded up to
 * a multiple of 32 — the same bytes matmul_quant_f32_dev takes for Q8_0),
 * weights and xq 16-byte aligned. */
int rsllm_hip_matmul_q8_0_batch_dev(float *out, size_t out_len, const uint8_t *weights,
                                    size_t weights_len, const int8_t *xq, size_t xq_len,
                                    const float *xscale, size_t xscale_len, size_t n_tok,
                                    size_t in_dim, size_t out_dim, rsllm_hip_stream_t stream);

/* ---- dequantisation ------------------------------------------------------ */

/* dequant_to_f32 (rsllm-gguf/src/dequant/mod.rs:69-85): decode `src` (GGUF
 * bytes) into dst[dst_len]. Bit-exact with the reference on every arm of its
 * dispatch: F32, F16, BF16, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, Q8_0, Q2_K, Q8_K,
 * IQ2_XXS; any other dtype is UNSUPPORTED_DEQUANT. Size rule of
 * q4_k.rs:36-49 (and siblings). */
int rsllm_hip_dequant_to_f32(uint32_t dtype, const uint8_t *src, size_t src_len, float *dst,
                             size_t dst_len);
int rsllm_hip_dequant_to_f32_dev(uint32_t dtype, const uint8_t *src, size_t src_len, float *dst,
                                 size_t dst_len, rsllm_hip_stream_t stream);

/* The measurement aids bench.py uses (a streaming read, the matrix-core
 * issue rate) are exported by the same library and declared in
 * rsllm_hip_probe.h: they are not part of the drop-in boundary. */

#ifdef __cplusplus
}
#endif
#endif /* RSLLM_HIP_H */
