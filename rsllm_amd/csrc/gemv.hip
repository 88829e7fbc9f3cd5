// Quantized GEMV, batch 1..n: y[t, o] = sum_i deq(W)[o, i] * x[t, i].
//
// Restates matmul_quant_f32 (rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119)
// without materialising dequantised rows: each lane decodes its 16-byte
// slice of a block in registers and folds the block scales out of the inner
// sum, e.g. for Q4_K sub-block j
//     sum_l (d*sc_j*q_l - dmin*m_j) x_l = (d*sc_j) sum_l q_l x_l - (dmin*m_j) sum_l x_l.
// Products and sums are fp32; only the summation order differs from the
// reference's sequential dot.
//
// Work split: a workgroup is 4 wavefronts; a wavefront owns R consecutive
// rows and BT consecutive tokens. Within a wavefront, 8 lanes share one
// block (one 16-byte load each, fully coalesced: 64 lanes read 8 whole
// blocks = 1152 contiguous bytes for Q4_K) and the 8 lane groups stride over
// the row's blocks. The per-lane partials are combined with a wavefront
// butterfly at the end.
#include "kernels.h"

namespace rsllm_hip {

__device__ __forceinline__ void load16f(const float *__restrict__ p, float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 f = *reinterpret_cast<const float4 *>(p + 4 * i);
        v[4 * i + 0] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
}

__device__ __forceinline__ float sum16(const float (&v)[16]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += v[i];
    return s;
}

// Dot of 16 bytes (4 dwords, each byte an unsigned value) with 16 floats.
__device__ __forceinline__ float dot16_u8(const uint32_t (&q)[4], const float (&xv)[16]) {
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int b = 0; b < 4; b++) s += ubyte_f(q[u], b) * xv[4 * u + b];
    return s;
}

// ---- Q4_K (GGUF layout) --------------------------------------------------
// Lane (grp, k): block b = grp + 8*i of the row, qs bytes 16k..16k+15, i.e.
// sub-block pair p = k/2, elements l = 16*(k&1) + 0..15 of sub-blocks 2p (low
// nibbles) and 2p+1 (high nibbles).
template <int R, int BT>
__global__ __launch_bounds__(256) void k_gemv_q4k(const uint8_t *__restrict__ w,
                                                  const float *__restrict__ x,
                                                  float *__restrict__ y, int n_tok, int in_dim,
                                                  int out_dim) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= out_dim) return;
    const int t0 = blockIdx.y * BT;
    const int nb = in_dim >> 8;
    const size_t row_bytes = (size_t)nb * kQ4kBytes;
    const int grp = lane >> 3, k = lane & 7;
    const int p = k >> 1;
    const int jlo = 2 * p, jhi = 2 * p + 1;
    const uint8_t *wrow[R];
#pragma unroll
    for (int r = 0; r < R; r++) wrow[r] = w + (size_t)min(row0 + r, out_dim - 1) * row_bytes;
    const float *xt[BT];
#pragma unroll
    for (int t = 0; t < BT; t++) xt[t] = x + (size_t)min(t0 + t, n_tok - 1) * in_dim;

    float acc[R][BT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = 0.f;

    for (int b = grp; b < nb; b += 8) {
        uint4 hdr[R], qv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *blk = wrow[r] + (size_t)b * kQ4kBytes;
            hdr[r] = *reinterpret_cast<const uint4 *>(blk);
            qv[r] = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * k);
        }
        float dlo[R], mlo[R], dhi[R], mhi[R];
        uint32_t qlo[R][4], qhi[R][4];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = f16_to_f32(hdr[r].x & 0xFFFFu);
            const float dmin = f16_to_f32(hdr[r].x >> 16);
            uint32_t sc, m;
            q4k_scale_min(jlo, hdr[r].y, hdr[r].z, hdr[r].w, sc, m);
            dlo[r] = d * (float)sc;
            mlo[r] = dmin * (float)m;
            q4k_scale_min(jhi, hdr[r].y, hdr[r].z, hdr[r].w, sc, m);
            dhi[r] = d * (float)sc;
            mhi[r] = dmin * (float)m;
            const uint32_t q4[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                qlo[r][u] = q4[u] & 0x0F0F0F0Fu;
                qhi[r][u] = (q4[u] >> 4) & 0x0F0F0F0Fu;
            }
        }
        const int xo = b * 256 + 64 * p + 16 * (k & 1);
#pragma unroll
        for (int t = 0; t < BT; t++) {
            float xl[16], xh[16];
            load16f(xt[t] + xo, xl);
            load16f(xt[t] + xo + 32, xh);
            const float sl = sum16(xl), sh = sum16(xh);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float pl = dot16_u8(qlo[r], xl);
                const float ph = dot16_u8(qhi[r], xh);
                acc[r][t] += dlo[r] * pl - mlo[r] * sl + dhi[r] * ph - mhi[r] * sh;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const float v = wave_sum(acc[r][t]);
            if (lane == 0 && row0 + r < out_dim && t0 + t < n_tok)
                y[(size_t)(t0 + t) * out_dim + row0 + r] = v;
        }
}

// ---- Q6_K (device layout: matrix planes [ql | qh | scales | d]) ------------
// Lane (grp, k): ql bytes 16k..16k+15 of block b: half h = k/4; those bytes
// hold stride kq = (k&3)/2 (low nibbles) and kq+2 (high nibbles), elements
// l = 16*(k&1) + 0..15, with their high bits in qh[32h + l] >> 2*kq (and
// >> 2*kq+4). Element index e = 128h + 32*kq + l; scale index e/16.
template <int R, int BT>
__global__ __launch_bounds__(256) void k_gemv_q6k(const uint8_t *__restrict__ w,
                                                  const float *__restrict__ x,
                                                  float *__restrict__ y, int n_tok, int in_dim,
                                                  int out_dim) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= out_dim) return;
    const int t0 = blockIdx.y * BT;
    const int nb = in_dim >> 8;
    const size_t nblk = (size_t)out_dim * nb;  // blocks in the matrix = plane length
    const uint8_t *qh_plane = w + nblk * 128;
    const uint8_t *sc_plane = w + nblk * 192;
    const uint8_t *d_plane = w + nblk * 208;
    const int grp = lane >> 3, k = lane & 7;
    const int h = k >> 2, kq = (k & 3) >> 1, l0 = 16 * (k & 1);
    const int sc_lo = 8 * h + 2 * kq + (k & 1);  // scale index for e_lo; e_hi uses +4
    const int e_lo = 128 * h + 32 * kq + l0;
    size_t rblk[R];  // index of the row's first block
#pragma unroll
    for (int r = 0; r < R; r++) rblk[r] = (size_t)min(row0 + r, out_dim - 1) * nb;
    const float *xt[BT];
#pragma unroll
    for (int t = 0; t < BT; t++) xt[t] = x + (size_t)min(t0 + t, n_tok - 1) * in_dim;

    float acc[R][BT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = 0.f;

    for (int b = grp; b < nb; b += 8) {
        float slo[R], shi[R];
        uint32_t qlo[R][4], qhi[R][4];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const size_t bi = rblk[r] + b;
            const uint4 qlv = *reinterpret_cast<const uint4 *>(w + bi * 128 + 16 * k);
            const uint4 qhv = *reinterpret_cast<const uint4 *>(qh_plane + bi * 64 + 32 * h + l0);
            const uint4 scv = *reinterpret_cast<const uint4 *>(sc_plane + bi * 16);
            const uint32_t dbits = *reinterpret_cast<const uint16_t *>(d_plane + bi * 2);
            const float d = f16_to_f32(dbits);
            const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
            const int8_t s_lo = (int8_t)(scw[sc_lo >> 2] >> (8 * (sc_lo & 3)));
            const int8_t s_hi = (int8_t)(scw[(sc_lo + 4) >> 2] >> (8 * ((sc_lo + 4) & 3)));
            slo[r] = d * (float)s_lo;
            shi[r] = d * (float)s_hi;
            const uint32_t ql4[4] = {qlv.x, qlv.y, qlv.z, qlv.w};
            const uint32_t qh4[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                qlo[r][u] = (ql4[u] & 0x0F0F0F0Fu) | (((qh4[u] >> (2 * kq)) & 0x03030303u) << 4);
                qhi[r][u] = ((ql4[u] >> 4) & 0x0F0F0F0Fu) |
                            (((qh4[u] >> (2 * kq + 4)) & 0x03030303u) << 4);
            }
        }
        const int xo = b * 256 + e_lo;
#pragma unroll
        for (int t = 0; t < BT; t++) {
            float xl[16], xh[16];
            load16f(xt[t] + xo, xl);
            load16f(xt[t] + xo + 64, xh);
            const float sl = sum16(xl), sh = sum16(xh);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float pl = dot16_u8(qlo[r], xl) - 32.f * sl;
                const float ph = dot16_u8(qhi[r], xh) - 32.f * sh;
                acc[r][t] += slo[r] * pl + shi[r] * ph;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const float v = wave_sum(acc[r][t]);
            if (lane == 0 && row0 + r < out_dim && t0 + t < n_tok)
                y[(size_t)(t0 + t) * out_dim + row0 + r] = v;
        }
}

// ---- Q8_0 / Q4_0 (device layout: matrix planes [qs | d]) -------------------
// Lane owns 16-byte qs chunks c = lane + 64*i. Q8_0: chunk c is half c&1 of
// block c/2 (16 signed weights). Q4_0: chunk c is block c (16 bytes, low
// nibbles = elements 0..15, high nibbles = 16..31, each minus 8).
template <int R, int BT, bool Q4>
__global__ __launch_bounds__(256) void k_gemv_q8(const uint8_t *__restrict__ w,
                                                 const float *__restrict__ x,
                                                 float *__restrict__ y, int n_tok, int in_dim,
                                                 int out_dim) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= out_dim) return;
    const int t0 = blockIdx.y * BT;
    const int nb = in_dim >> 5;
    const int qbytes = Q4 ? 16 : 32;
    const uint8_t *d_plane = w + (size_t)out_dim * nb * qbytes;
    const int nchunks = Q4 ? nb : 2 * nb;
    size_t rblk[R];  // index of the row's first block
#pragma unroll
    for (int r = 0; r < R; r++) rblk[r] = (size_t)min(row0 + r, out_dim - 1) * nb;
    const float *xt[BT];
#pragma unroll
    for (int t = 0; t < BT; t++) xt[t] = x + (size_t)min(t0 + t, n_tok - 1) * in_dim;

    float acc[R][BT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = 0.f;

    for (int c = lane; c < nchunks; c += 64) {
        const int b = Q4 ? c : (c >> 1);
        float dd[R];
        uint32_t q[R][4], q2[R][4];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 v =
                *reinterpret_cast<const uint4 *>(w + rblk[r] * qbytes + (size_t)c * 16);
            dd[r] = f16_to_f32(*reinterpret_cast<const uint16_t *>(d_plane + (rblk[r] + b) * 2));
            const uint32_t v4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (Q4) {
                    q[r][u] = v4[u] & 0x0F0F0F0Fu;
                    q2[r][u] = (v4[u] >> 4) & 0x0F0F0F0Fu;
                } else {
                    q[r][u] = v4[u] ^ 0x80808080u;  // signed byte s -> s + 128 as unsigned
                }
            }
        }
        const int xo = Q4 ? 32 * b : 16 * c;
#pragma unroll
        for (int t = 0; t < BT; t++) {
            float xa[16];
            load16f(xt[t] + xo, xa);
            const float sa = sum16(xa);
            if (Q4) {
                float xb[16];
                load16f(xt[t] + xo + 16, xb);
                const float sb = sum16(xb);
#pragma unroll
                for (int r = 0; r < R; r++)
                    acc[r][t] += dd[r] * ((dot16_u8(q[r], xa) - 8.f * sa) +
                                          (dot16_u8(q2[r], xb) - 8.f * sb));
            } else {
#pragma unroll
                for (int r = 0; r < R; r++) acc[r][t] += dd[r] * (dot16_u8(q[r], xa) - 128.f * sa);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const float v = wave_sum(acc[r][t]);
            if (lane == 0 && row0 + r < out_dim && t0 + t < n_tok)
                y[(size_t)(t0 + t) * out_dim + row0 + r] = v;
        }
}

__global__ void k_fill_zero(float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = 0.f;
}

hipError_t launch_fill_zero(float *y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    k_fill_zero<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(y, n);
    return hipGetLastError();
}

template <int R, int BT>
static hipError_t gemv_rb(uint32_t dtype, const uint8_t *w, const float *x, float *y, int n_tok,
                          int in_dim, int out_dim, hipStream_t s) {
    const dim3 grid((unsigned)((out_dim + 4 * R - 1) / (4 * R)), (unsigned)((n_tok + BT - 1) / BT));
    switch (dtype) {
    case T_Q4_K: k_gemv_q4k<R, BT><<<grid, 256, 0, s>>>(w, x, y, n_tok, in_dim, out_dim); break;
    case T_Q6_K: k_gemv_q6k<R, BT><<<grid, 256, 0, s>>>(w, x, y, n_tok, in_dim, out_dim); break;
    case T_Q8_0: k_gemv_q8<R, BT, false><<<grid, 256, 0, s>>>(w, x, y, n_tok, in_dim, out_dim); break;
    case T_Q4_0: k_gemv_q8<R, BT, true><<<grid, 256, 0, s>>>(w, x, y, n_tok, in_dim, out_dim); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(uint32_t dtype, const uint8_t *w, const float *x, float *y, int n_tok,
                       int in_dim, int out_dim, hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    if (n_tok == 1) return gemv_rb<2, 1>(dtype, w, x, y, n_tok, in_dim, out_dim, s);
    if (n_tok == 2) return gemv_rb<2, 2>(dtype, w, x, y, n_tok, in_dim, out_dim, s);
    if (n_tok <= 4) return gemv_rb<1, 4>(dtype, w, x, y, n_tok, in_dim, out_dim, s);
    return gemv_rb<1, 8>(dtype, w, x, y, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
