// Routed-expert MoE layer on the GPU:
//   out[t] += sum_i w[t, i] * down[e] ( silu(min(gate[e] x_t, c)) * clamp(up[e] x_t, -c, c) ),
//   e = ids[t, i], for every token t and selected slot i with w[t, i] != 0.
//
// Restates accumulate_moe_outputs (rsllm-models/src/dsv4/moe.rs:648-707) with
// apply_expert_swiglu (:479-502) and apply_swiglu_clamp (:515-531). The
// reference runs three matmul_quant_f32 GEMVs per (token, expert) pair,
// re-reading each selected expert's weights once per token. Here the
// (token, slot) pairs are grouped by expert on the device, and each expert's
// gate/up and down matrices are streamed once per batch of up to 4 of its
// tokens (grouped GEMV, gemv.hip):
//   1. k_moe_route: slots sorted by expert (ties in (t, i) order), per-expert
//      offsets, slot -> token, (t, i) -> slot, the list of active experts;
//      slots with w == 0 are skipped (moe.rs:681-683).
//   2. activation limbs of x for the gate/up format;
//   3. grouped GEMV, gate and up in one launch -> hg, hu [slot x n_ff];
//   4+5. clamp (only when c > 1e-6; NaN passes), silu(g) * u and the
//      activation limbs for the down format in one pass;
//   6. grouped GEMV, down -> yd [slot x n_embd];
//   7. k_moe_accumulate: out[t, j] += w[t, i] * yd[slot(t, i), j] in i order,
//      as the reference's `out_t[j] += we * expert_out[j]` (no contraction).
#include "kernels.h"

namespace rsllm_hip {

// One workgroup. ids and weights are cached in LDS; a slot's rank inside its
// expert is the number of earlier valid slots with the same expert
// (deterministic order). Also lists the experts with at least one slot, in
// ascending order (act, count in *n_act), for the grouped GEMV grids.
__global__ __launch_bounds__(256) void k_moe_route(const int *__restrict__ ids,
                                                   const float *__restrict__ wts, int n_pairs,
                                                   int k, int n_expert, int *__restrict__ off,
                                                   int *__restrict__ slot_tok,
                                                   int *__restrict__ slot_of,
                                                   int *__restrict__ act, int *__restrict__ n_act) {
    extern __shared__ int lds[];
    int *cnt = lds;                     // n_expert + 1
    int *eid = lds + n_expert + 1;      // n_pairs: expert id, or -1 for a skipped slot
    const int tid = threadIdx.x;
    for (int e = tid; e <= n_expert; e += 256) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < n_pairs; p += 256) {
        const int e = ids[p];
        const bool valid = wts[p] != 0.0f && e >= 0 && e < n_expert;
        eid[p] = valid ? e : -1;
        if (valid) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, na = 0;
        for (int e = 0; e < n_expert; e++) {
            const int c = cnt[e];
            cnt[e] = run;
            off[e] = run;
            if (c) act[na++] = e;
            run += c;
        }
        off[n_expert] = run;
        *n_act = na;
    }
    __syncthreads();
    for (int p = tid; p < n_pairs; p += 256) {
        const int e = eid[p];
        int slot = -1;
        if (e >= 0) {
            int rank = 0;
            for (int q = 0; q < p; q++) rank += eid[q] == e ? 1 : 0;
            slot = cnt[e] + rank;
            slot_tok[slot] = p / k;
        }
        slot_of[p] = slot;
    }
}

__global__ __launch_bounds__(256) void k_moe_accumulate(float *__restrict__ out,
                                                        const float *__restrict__ yd,
                                                        const float *__restrict__ wts,
                                                        const int *__restrict__ slot_of,
                                                        int n_tok, int k, int n_embd) {
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n_tok * n_embd) return;
    const int t = (int)(i / n_embd), j = (int)(i % n_embd);
    float v = out[i];
    for (int p = 0; p < k; p++) {
        const int s = slot_of[t * k + p];
        if (s >= 0) {
            const float prod = wts[t * k + p] * yd[(size_t)s * n_embd + j];
            v = v + prod;
        }
    }
    out[i] = v;
}

size_t moe_scratch_bytes(uint32_t dt_gu, uint32_t dt_d, int n_tok, int k, int n_expert,
                         int n_embd, int n_ff) {
    const size_t P = (size_t)n_tok * k;
    size_t b = 0;
    auto add = [&](size_t n) { b += (n + 255) / 256 * 256; };
    add((size_t)(n_expert + 1) * 4);                      // off
    add((size_t)(n_expert + 1) * 4);                      // act, n_act
    add(P * 4);                                           // slot_tok
    add(P * 4);                                           // slot_of
    add(gemv_scratch_bytes(dt_gu, n_tok, n_embd));        // x limbs
    add(P * n_ff * 4);                                    // hg
    add(P * n_ff * 4);                                    // hu
    add(gemv_scratch_bytes(dt_d, (int)P, n_ff));          // SwiGLU limbs
    add(P * n_embd * 4);                                  // yd
    return b;
}

hipError_t launch_moe(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                      const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                      const int *ids, const float *wts, float *out, uint8_t *scratch, int n_tok,
                      int k, int n_expert, int n_embd, int n_ff, float clamp, hipStream_t s) {
    if (n_tok <= 0 || k <= 0) return hipSuccess;
    const size_t P = (size_t)n_tok * k;
    uint8_t *p = scratch;
    auto take = [&](size_t n) {
        uint8_t *r = p;
        p += (n + 255) / 256 * 256;
        return r;
    };
    int *off = reinterpret_cast<int *>(take((size_t)(n_expert + 1) * 4));
    int *act = reinterpret_cast<int *>(take((size_t)(n_expert + 1) * 4));
    int *n_act = act + n_expert;
    int *slot_tok = reinterpret_cast<int *>(take(P * 4));
    int *slot_of = reinterpret_cast<int *>(take(P * 4));
    const size_t xq1_bytes = gemv_scratch_bytes(dt_gu, n_tok, n_embd);
    uint8_t *xq1 = take(xq1_bytes);
    float *hg = reinterpret_cast<float *>(take(P * n_ff * 4));
    float *hu = reinterpret_cast<float *>(take(P * n_ff * 4));
    const size_t xq2_bytes = gemv_scratch_bytes(dt_d, (int)P, n_ff);
    uint8_t *xq2 = take(xq2_bytes);
    float *yd = reinterpret_cast<float *>(take(P * n_embd * 4));
    // at most min(n_expert, n_tok * k) experts are active
    const int grid_experts = (int)(P < (size_t)n_expert ? P : (size_t)n_expert);

    k_moe_route<<<1, 256, (size_t)(n_expert + 1 + P) * 4, s>>>(ids, wts, (int)P, k, n_expert, off,
                                                               slot_tok, slot_of, act, n_act);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((e = launch_quantize_x(dt_gu, x, xq1, n_tok, n_embd, s)) != hipSuccess) return e;
    if ((e = launch_gemv_grouped(dt_gu, gate, up, gu_stride, xq1, xq1_bytes, off, slot_tok, act,
                                 n_act, grid_experts, hg, hu, n_embd, n_ff, s)) != hipSuccess)
        return e;
    if ((e = launch_quantize_swiglu(dt_d, hg, hu, clamp, xq2, (int)P, n_ff, off, n_expert, s)) !=
        hipSuccess)
        return e;
    if ((e = launch_gemv_grouped(dt_d, down, nullptr, d_stride, xq2, xq2_bytes, off, nullptr, act,
                                 n_act, grid_experts, yd, nullptr, n_ff, n_embd, s)) != hipSuccess)
        return e;
    k_moe_accumulate<<<(unsigned)(((size_t)n_tok * n_embd + 255) / 256), 256, 0, s>>>(
        out, yd, wts, slot_of, n_tok, k, n_embd);
    return hipGetLastError();
}

}  // namespace rsllm_hip
