// Q8_0 int8-activation path, bit-exact with the reference's scalar tier:
//   quantize_q8_0_batch  (rsllm-backend-cpu/src/ops/q8_0.rs:42-129)
//   matmul_q8_0_batch    (q8_0.rs:217-263, dot_q8_0_row_scalar :163-193)
//
// Quantizer: per 32-element block, amax over the block (a non-finite input
// sets the caller's status word: the reference returns NonFiniteInput),
// d = amax / 127 and id = 1 / d (correctly rounded f32 divisions, HIP's
// default), q = clamp(rint(x * id), -128, 127) (round half to even, as
// round_ties_even; NaN -> 0 and +-inf saturate, as `as i32`), the tail of a
// partial last block zero-padded. One lane per element slot, the block's
// amax by cross-lane max over its 32 lanes.
//
// Matmul: weights in the device layout (8-block super-tiles [qs 8*32 | d
// 8*2], written by launch_prepare from the GGUF rows). For every (token,
// row, block) a lane forms the exact int32 dot of the 32 int8 pairs with
// v_dot4_i32_i8 and the product (wscale * xscale) * dot in f32, wscale = the
// f16 block scale with non-finite values taken as 0 (block_scale_finite
// :143-146). The products go to LDS; one thread per (token, row) then adds
// them in block order starting from 0.0 — the reference's sequential
// accumulation — so the result is bit-identical.
#include "kernels.h"

namespace rsllm_hip {

__global__ __launch_bounds__(256) void k_q8_quantize(const float *__restrict__ x,
                                                     int8_t *__restrict__ xq,
                                                     float *__restrict__ scale, int n_slots,
                                                     int in_dim, int blocks,
                                                     int *__restrict__ status) {
#pragma clang fp contract(off)
    const int gid = blockIdx.x * 256 + threadIdx.x;  // element slot: (t, b, i)
    const bool in_range = gid < n_slots;
    const int row_slots = blocks * 32;
    const int t = gid / row_slots;
    const int e = gid - t * row_slots;  // b * 32 + i
    const bool valid = in_range && e < in_dim;
    const float v = valid ? x[(size_t)t * in_dim + e] : 0.0f;
    const bool bad = valid && !__builtin_isfinite(v);
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    if (status && __ballot(bad) && (threadIdx.x & 63) == 0) atomicOr(status, 1);
    if (!in_range) return;
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    // x * id is NaN for x == 0 when 1/d overflowed (subnormal d): `as i32` -> 0
    const float r = rintf(v * id);
    const int q = r != r ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
    xq[gid] = (int8_t)q;
    if ((e & 31) == 0) scale[gid >> 5] = d;
}

// Workgroup: ROWS weight rows x BT tokens, blocks in chunks of 128. Thread
// (r, j), r = tid / LPR, j = tid % LPR (LPR = 256 / ROWS lanes per row),
// computes the products of row r for blocks j + LPR * k of the chunk into
// LDS; then thread (t, r) continues its sequential sum over the chunk.
constexpr int kQ8Chunk = 128;
constexpr int kQ8Pad = kQ8Chunk + 1;  // LDS row stride (floats)
constexpr int kQ8Tile = 272;          // 8 blocks: qs 8*32 | d 8*2

template <int ROWS, int BT>
__global__ __launch_bounds__(256) void k_q8_int8_gemv(const uint8_t *__restrict__ w,
                                                      uint32_t w_bytes,
                                                      const int8_t *__restrict__ xq,
                                                      const float *__restrict__ xscale,
                                                      float *__restrict__ out, int n_tok,
                                                      int in_dim, int out_dim, int blocks) {
#pragma clang fp contract(off)
    constexpr int LPR = 256 / ROWS, KPT = kQ8Chunk / LPR;
    __shared__ float prod[BT * ROWS * kQ8Pad];
    const int tid = threadIdx.x;
    const int r = tid / LPR, j = tid % LPR;
    const int row = min((int)blockIdx.x * ROWS + r, out_dim - 1);
    const int t0 = blockIdx.y * BT;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const uint32_t nblk = (uint32_t)out_dim * (uint32_t)blocks;
    const uint32_t full_tiles = nblk >> 3, last_r = nblk & 7u;
    const int last_bn = in_dim - (blocks - 1) * 32;  // valid elements of the last block
    float acc = 0.0f;                                // thread (t, r) = (tid / ROWS, tid % ROWS)
    for (int c0 = 0; c0 < blocks; c0 += kQ8Chunk) {
        uint4 qa[KPT], qb[KPT];
        float ws[KPT];
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const int b = min(c0 + j + LPR * k, blocks - 1);
            const uint32_t g = (uint32_t)row * (uint32_t)blocks + (uint32_t)b;
            const uint32_t S = g >> 3, sl = g & 7u;
            const uint32_t rS = S < full_tiles ? 8u : last_r;
            const uint32_t base = S * (uint32_t)kQ8Tile;
            qa[k] = bload16(rw, base + sl * 32u, 0);
            qb[k] = bload16(rw, base + sl * 32u + 16u, 0);
            const float s = f16_to_f32(bload2(rw, base + rS * 32u + sl * 2u, 0));
            ws[k] = __builtin_isfinite(s) ? s : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const int tok = min(t0 + t, n_tok - 1);
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int b = c0 + j + LPR * k;
                float p = 0.0f;
                if (b < blocks) {
                    const uint4 *xp =
                        reinterpret_cast<const uint4 *>(xq + ((size_t)tok * blocks + b) * 32);
                    uint4 u0 = xp[0], u1 = xp[1];
                    if (b == blocks - 1 && last_bn < 32) {
                        // only the block's first last_bn lanes take part (:184-187)
                        uint32_t m[8];
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const int keep = min(max(last_bn - 4 * i, 0), 4);
                            m[i] = keep == 4 ? 0xFFFFFFFFu : ((1u << (8 * keep)) - 1u);
                        }
                        u0.x &= m[0]; u0.y &= m[1]; u0.z &= m[2]; u0.w &= m[3];
                        u1.x &= m[4]; u1.y &= m[5]; u1.z &= m[6]; u1.w &= m[7];
                    }
                    int dot = 0;
                    dot = __builtin_amdgcn_sdot4((int)qa[k].x, (int)u0.x, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[k].y, (int)u0.y, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[k].z, (int)u0.z, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[k].w, (int)u0.w, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[k].x, (int)u1.x, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[k].y, (int)u1.y, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[k].z, (int)u1.z, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[k].w, (int)u1.w, dot, false);
                    const float xs = xscale[(size_t)tok * blocks + b];
                    p = (ws[k] * xs) * (float)dot;
                }
                prod[(t * ROWS + r) * kQ8Pad + j + LPR * k] = p;
            }
        }
        __syncthreads();
        if (tid < BT * ROWS) {
            const float *pr = prod + tid * kQ8Pad;
            const int n = min(kQ8Chunk, blocks - c0);
            for (int i = 0; i < n; i++) acc = acc + pr[i];
        }
        __syncthreads();
    }
    if (tid < BT * ROWS) {
        const int t = t0 + tid / ROWS, o = (int)blockIdx.x * ROWS + tid % ROWS;
        if (t < n_tok && o < out_dim) out[(size_t)t * out_dim + o] = acc;
    }
}

// Row-tiled form for 2 or more tokens. Thread (h, j), j = tid % CB, h = tid
// / CB, holds weight block c0 + j of each of the workgroup's ROWS rows in
// registers and multiplies it with tokens h, h + 256/CB, ... of the tile, so
// an activation block is read once per workgroup rather than once per row.
// The products go to LDS and thread (t, r) adds them in block order as in
// k_q8_int8_gemv. Workgroup order: ids go round robin over the 8 XCDs, and
// the token tiles of one row tile take ids L, L + 8, ..., so they run on one
// XCD and share its L2 copy of the rows.
template <int ROWS, int BT, int CB>
__global__ __launch_bounds__(256) void k_q8_int8_rows(const uint8_t *__restrict__ w,
                                                      uint32_t w_bytes,
                                                      const int8_t *__restrict__ xq,
                                                      const float *__restrict__ xscale,
                                                      float *__restrict__ out, int n_tok,
                                                      int in_dim, int out_dim, int blocks,
                                                      int n_rt, int n_tt) {
#pragma clang fp contract(off)
    constexpr int TG = 256 / CB, Pad = CB + 1;
    static_assert(BT * ROWS <= 256, "tile");
    __shared__ float prod[BT * ROWS * Pad];
    const int L = blockIdx.x;
    const int rt = (L / (8 * n_tt)) * 8 + L % 8, tt = (L / 8) % n_tt;
    if (rt >= n_rt) return;  // the whole workgroup, before any barrier
    const int tid = threadIdx.x, j = tid % CB, h = tid / CB;
    const int row0 = rt * ROWS, t0 = tt * BT;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const uint32_t nblk = (uint32_t)out_dim * (uint32_t)blocks;
    const uint32_t full_tiles = nblk >> 3, last_r = nblk & 7u;
    const int last_bn = in_dim - (blocks - 1) * 32;
    float acc = 0.0f;  // thread (t, r) = (tid / ROWS, tid % ROWS)
    for (int c0 = 0; c0 < blocks; c0 += CB) {
        const int b = c0 + j;
        const bool live = b < blocks;
        const int bb = min(b, blocks - 1);
        uint4 qa[ROWS], qb[ROWS];
        float ws[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int row = min(row0 + r, out_dim - 1);
            const uint32_t g = (uint32_t)row * (uint32_t)blocks + (uint32_t)bb;
            const uint32_t S = g >> 3, sl = g & 7u;
            const uint32_t rS = S < full_tiles ? 8u : last_r;
            const uint32_t base = S * (uint32_t)kQ8Tile;
            qa[r] = bload16(rw, base + sl * 32u, 0);
            qb[r] = bload16(rw, base + sl * 32u + 16u, 0);
            const float sc = f16_to_f32(bload2(rw, base + rS * 32u + sl * 2u, 0));
            ws[r] = __builtin_isfinite(sc) ? sc : 0.0f;
        }
        // only the first last_bn lanes of a partial last block take part (:184-187)
        const bool part = last_bn < 32 && b == blocks - 1;
        uint32_t m[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int keep = part ? min(max(last_bn - 4 * i, 0), 4) : 4;
            m[i] = keep == 4 ? 0xFFFFFFFFu : ((1u << (8 * keep)) - 1u);
        }
#pragma unroll
        for (int t = h; t < BT; t += TG) {
            const int tok = min(t0 + t, n_tok - 1);
            float p[ROWS];
#pragma unroll
            for (int r = 0; r < ROWS; r++) p[r] = 0.0f;
            // tokens past n_tok (a partial last tile) give 0: their sums are not stored
            if (live && t0 + t < n_tok) {
                const uint4 *xp =
                    reinterpret_cast<const uint4 *>(xq + ((size_t)tok * blocks + b) * 32);
                uint4 u0 = xp[0], u1 = xp[1];
                if (part) {
                    u0.x &= m[0]; u0.y &= m[1]; u0.z &= m[2]; u0.w &= m[3];
                    u1.x &= m[4]; u1.y &= m[5]; u1.z &= m[6]; u1.w &= m[7];
                }
                const float xs = xscale[(size_t)tok * blocks + b];
#pragma unroll
                for (int r = 0; r < ROWS; r++) {
                    int dot = 0;
                    dot = __builtin_amdgcn_sdot4((int)qa[r].x, (int)u0.x, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[r].y, (int)u0.y, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[r].z, (int)u0.z, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qa[r].w, (int)u0.w, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[r].x, (int)u1.x, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[r].y, (int)u1.y, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[r].z, (int)u1.z, dot, false);
                    dot = __builtin_amdgcn_sdot4((int)qb[r].w, (int)u1.w, dot, false);
                    p[r] = (ws[r] * xs) * (float)dot;
                }
            }
#pragma unroll
            for (int r = 0; r < ROWS; r++) prod[(t * ROWS + r) * Pad + j] = p[r];
        }
        __syncthreads();
        if (tid < BT * ROWS) {
            const float *pr = prod + tid * Pad;
            const int n = min(CB, blocks - c0);
            for (int i = 0; i < n; i++) acc = acc + pr[i];
        }
        __syncthreads();
    }
    if (tid < BT * ROWS) {
        const int t = t0 + tid / ROWS, o = row0 + tid % ROWS;
        if (t < n_tok && o < out_dim) out[(size_t)t * out_dim + o] = acc;
    }
}

template <int ROWS, int BT, int CB>
static hipError_t q8_rows_go(const uint8_t *w, size_t w_bytes, const int8_t *xq,
                             const float *xscale, float *out, int n_tok, int in_dim, int out_dim,
                             hipStream_t s) {
    const int blocks = (in_dim + 31) / 32;
    const int n_rt = (out_dim + ROWS - 1) / ROWS, n_tt = (n_tok + BT - 1) / BT;
    const long long n_wg = (long long)((n_rt + 7) / 8) * 8 * n_tt;
    k_q8_int8_rows<ROWS, BT, CB><<<(unsigned)n_wg, 256, 0, s>>>(
        w, (uint32_t)w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, blocks, n_rt, n_tt);
    return hipGetLastError();
}

template <int ROWS, int BT>
static hipError_t q8_rows_cb(const uint8_t *w, size_t w_bytes, const int8_t *xq,
                             const float *xscale, float *out, int n_tok, int in_dim, int out_dim,
                             hipStream_t s) {
    const int blocks = (in_dim + 31) / 32;
    if (blocks >= 128) return q8_rows_go<ROWS, BT, 128>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    if (blocks >= 64) return q8_rows_go<ROWS, BT, 64>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    return q8_rows_go<ROWS, BT, 32>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
}

hipError_t launch_q8_quantize(const float *x, int8_t *xq, float *scale, int n_tok, int in_dim,
                              int *status, hipStream_t s) {
    const int blocks = (in_dim + 31) / 32;
    const long long n = (long long)n_tok * blocks * 32;
    if (n <= 0) return hipSuccess;
    k_q8_quantize<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, xq, scale, (int)n, in_dim, blocks,
                                                             status);
    return hipGetLastError();
}

template <int ROWS, int BT>
static hipError_t q8_gemv_go(const uint8_t *w, size_t w_bytes, const int8_t *xq,
                             const float *xscale, float *out, int n_tok, int in_dim, int out_dim,
                             hipStream_t s) {
    const int blocks = (in_dim + 31) / 32;
    const dim3 grid((unsigned)((out_dim + ROWS - 1) / ROWS), (unsigned)((n_tok + BT - 1) / BT));
    k_q8_int8_gemv<ROWS, BT><<<grid, 256, 0, s>>>(w, (uint32_t)w_bytes, xq, xscale, out, n_tok,
                                                  in_dim, out_dim, blocks);
    return hipGetLastError();
}

hipError_t launch_q8_int8_matmul(const uint8_t *w, size_t w_bytes, const int8_t *xq,
                                 const float *xscale, float *out, int n_tok, int in_dim,
                                 int out_dim, hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0 || in_dim <= 0) return hipSuccess;
    // one token: the row-tiled kernel's 2-token tile (4096 x 4096: 6.7 ->
    // 6.3 us, 4096 x 14336: 18.8 -> 14.8 us) except on tall, narrow
    // matrices (14336 x 4096: 13.4 against 14.0 us) and below 4096 rows,
    // where k_q8_int8_gemv is kept, with fewer rows per workgroup for short
    // matrices so the grid still fills the 256 CUs
    if (n_tok == 1) {
        if (out_dim >= 4096 && (out_dim < 8192 || in_dim >= 8192))
            return q8_rows_cb<8, 2>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
        if (out_dim >= 4096)
            return q8_gemv_go<8, 1>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
        return q8_gemv_go<4, 1>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    }
    // more: the row-tiled kernel, 8 rows (4 below 4096 rows, for a fuller
    // grid) x 2, 4 or 8 tokens up to 8 tokens, 4 x 16 above
    if (out_dim < 4096 && n_tok <= 8) {
        if (n_tok == 2) return q8_rows_cb<4, 2>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
        if (n_tok <= 4) return q8_rows_cb<4, 4>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
        return q8_rows_cb<4, 8>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    }
    if (n_tok == 2) return q8_rows_cb<8, 2>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    if (n_tok <= 4) return q8_rows_cb<8, 4>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    if (n_tok <= 8) return q8_rows_cb<8, 8>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
    return q8_rows_cb<4, 16>(w, w_bytes, xq, xscale, out, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
