// GGUF block decode to f32 (bit-exact with the reference dequantizers) and
// the one-time re-layout of weights into the device layout the GEMV kernels
// read.
//
// Bit-exactness: every product in the reference formulas is exact in f32
// (Q4_K: d*sc <= 17 significant bits, times q <= 4 bits; Q6_K:
// d*sc*(q-32) <= 23 bits; Q8_0/Q4_0: <= 18 bits; Q2_K: d*sc <= 15 bits,
// times q <= 2; IQ2_XXS: d*(0.5+e)*0.25 <= 16 bits, times the grid byte
// <= 6; Q5_K: d*sc <= 17 bits, times q <= 5 bits; Q4_1: d times q <= 4
// bits), so the only roundings are the final subtractions / additions of
// Q4_K, Q5_K, Q2_K and Q4_1 and Q8_K's product d*q (an f32 scale). Contraction
// is switched off anyway so each line is evaluated exactly as written.
#include "iq2xxs_grid.h"
#include "kernels.h"

namespace rsllm_hip {

#pragma clang fp contract(off)

// One thread per (block, 32-element sub-block j): q4_k.rs:51-89.
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t *__restrict__ src,
                                                     float *__restrict__ dst, size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 8) return;
    const size_t b = gid >> 3;
    const int j = (int)(gid & 7);
    const uint8_t *blk = src + b * kQ4kBytes;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = f16_to_f32(blk[2] | (blk[3] << 8));
    uint32_t s[3];
    for (int i = 0; i < 3; i++)
        s[i] = blk[4 + 4 * i] | (blk[5 + 4 * i] << 8) | (blk[6 + 4 * i] << 16) |
               ((uint32_t)blk[7 + 4 * i] << 24);
    uint32_t sc, m;
    q4k_scale_min(j, s[0], s[1], s[2], sc, m);
    const float d1 = d * (float)sc;
    const float m1f = dmin * (float)m;
    const uint8_t *q = blk + 16 + 32 * (j >> 1);
    const int shift = (j & 1) ? 4 : 0;
    float *o = dst + b * 256 + 32 * j;
    for (int l = 0; l < 32; l += 4) {
        float4 v;
        v.x = d1 * (float)((q[l + 0] >> shift) & 15) - m1f;
        v.y = d1 * (float)((q[l + 1] >> shift) & 15) - m1f;
        v.z = d1 * (float)((q[l + 2] >> shift) & 15) - m1f;
        v.w = d1 * (float)((q[l + 3] >> shift) & 15) - m1f;
        *reinterpret_cast<float4 *>(o + l) = v;
    }
}

// One thread per (block, 32-element group g): q6_k.rs:50-99. Group g covers
// elements 32g..32g+31 = half h = g/4, stride k = g%4.
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t *__restrict__ src,
                                                     float *__restrict__ dst, size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 8) return;
    const size_t b = gid >> 3;
    const int g = (int)(gid & 7);
    const int h = g >> 2, k = g & 3;
    const uint8_t *blk = src + b * kQ6kBytes;
    const float d = f16_to_f32(blk[208] | (blk[209] << 8));
    const uint8_t *ql = blk + 64 * h + 32 * (k & 1);
    const uint8_t *qh = blk + 128 + 32 * h;
    const int8_t *scl = reinterpret_cast<const int8_t *>(blk + 192 + 8 * h + 2 * k);
    const int nshift = (k >= 2) ? 4 : 0;
    float *o = dst + b * 256 + 32 * g;
    for (int l = 0; l < 32; l += 4) {
        float r[4];
        for (int u = 0; u < 4; u++) {
            const int ll = l + u;
            const int q = (((ql[ll] >> nshift) & 15) | (((qh[ll] >> (2 * k)) & 3) << 4)) - 32;
            r[u] = d * (float)scl[ll >> 4] * (float)q;
        }
        *reinterpret_cast<float4 *>(o + l) = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// One thread per Q8_0 block: q8_0.rs:44-60.
__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t *__restrict__ src,
                                                      float *__restrict__ dst, size_t n_blocks) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t *blk = src + b * kQ8Bytes;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    float *o = dst + b * 32;
    for (int j = 0; j < 32; j += 4) {
        float4 v;
        v.x = (float)(int8_t)blk[2 + j] * d;
        v.y = (float)(int8_t)blk[3 + j] * d;
        v.z = (float)(int8_t)blk[4 + j] * d;
        v.w = (float)(int8_t)blk[5 + j] * d;
        *reinterpret_cast<float4 *>(o + j) = v;
    }
}

// One thread per Q4_0 block: q4_0.rs:47-61.
__global__ __launch_bounds__(256) void k_dequant_q4_0(const uint8_t *__restrict__ src,
                                                      float *__restrict__ dst, size_t n_blocks) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t *blk = src + b * 18;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    float *o = dst + b * 32;
    for (int j = 0; j < 16; j++) {
        const int x0 = (blk[2 + j] & 15) - 8;
        const int x1 = (blk[2 + j] >> 4) - 8;
        o[j] = (float)x0 * d;
        o[j + 16] = (float)x1 * d;
    }
}

// One thread per Q4_1 block (20 bytes: d, m as f16, 16 code bytes):
// q4_0.rs:66-87, code * d + m (the product exact: a 4-bit code times an f16
// scale), one rounding in the addition.
__global__ __launch_bounds__(256) void k_dequant_q4_1(const uint8_t *__restrict__ src,
                                                      float *__restrict__ dst, size_t n_blocks) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t *blk = src + b * 20;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    const float m = f16_to_f32(blk[2] | (blk[3] << 8));
    float *o = dst + b * 32;
    for (int j = 0; j < 16; j++) {
        o[j] = (float)(blk[4 + j] & 15) * d + m;
        o[j + 16] = (float)(blk[4 + j] >> 4) * d + m;
    }
}

// One thread per (Q5_K block, 32-element sub-block j): q5_k.rs:53-91. Block
// of 176 bytes: d, dmin (f16), the Q4_K scale packing (12 bytes), qh[32],
// qs[128]. Element l of sub-block j: low 4 bits from qs[32 (j / 2) + l]
// (low nibble for even j, high for odd), bit 4 from bit j of qh[l];
// (d * sc_j) * q - dmin * m_j with both products exact (6-bit scale times
// f16; 17-bit scale times a 5-bit code), one rounding in the subtraction.
__global__ __launch_bounds__(256) void k_dequant_q5k(const uint8_t *__restrict__ src,
                                                     float *__restrict__ dst, size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 8) return;
    const size_t b = gid >> 3;
    const int j = (int)(gid & 7);
    const uint8_t *blk = src + b * 176;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = f16_to_f32(blk[2] | (blk[3] << 8));
    uint32_t s[3];
    for (int i = 0; i < 3; i++)
        s[i] = blk[4 + 4 * i] | (blk[5 + 4 * i] << 8) | (blk[6 + 4 * i] << 16) |
               ((uint32_t)blk[7 + 4 * i] << 24);
    uint32_t sc, m;
    q4k_scale_min(j, s[0], s[1], s[2], sc, m);
    const float d1 = d * (float)sc;
    const float m1f = dmin * (float)m;
    const uint8_t *qh = blk + 16;
    const uint8_t *qs = blk + 48 + 32 * (j >> 1);
    const int shift = (j & 1) ? 4 : 0;
    float *o = dst + b * 256 + 32 * j;
    for (int l = 0; l < 32; l += 4) {
        float r[4];
        for (int u = 0; u < 4; u++) {
            const uint32_t q = ((qs[l + u] >> shift) & 15) | (((qh[l + u] >> j) & 1) << 4);
            r[u] = d1 * (float)q - m1f;
        }
        *reinterpret_cast<float4 *>(o + l) = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// One thread per (Q8_K block, 32-element group g): q8_k.rs:50-66. Block of
// 292 bytes: d (f32), qs[256] (int8), bsums (not used by the decode);
// d * q, one rounding.
__global__ __launch_bounds__(256) void k_dequant_q8k(const uint8_t *__restrict__ src,
                                                     float *__restrict__ dst, size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 8) return;
    const size_t b = gid >> 3;
    const int g = (int)(gid & 7);
    const uint8_t *blk = src + b * 292;
    const float d = __builtin_bit_cast(
        float, (uint32_t)(blk[0] | (blk[1] << 8) | (blk[2] << 16) | ((uint32_t)blk[3] << 24)));
    const uint8_t *q = blk + 4 + 32 * g;
    float *o = dst + b * 256 + 32 * g;
    for (int l = 0; l < 32; l += 4)
        *reinterpret_cast<float4 *>(o + l) =
            make_float4(d * (float)(int8_t)q[l], d * (float)(int8_t)q[l + 1],
                        d * (float)(int8_t)q[l + 2], d * (float)(int8_t)q[l + 3]);
}

// F32 / F16 / BF16 arms (float.rs): element-wise widening.
__global__ __launch_bounds__(256) void k_dequant_float(const uint8_t *__restrict__ src,
                                                       float *__restrict__ dst, size_t n,
                                                       uint32_t dtype) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (dtype == T_F32) {
        const uint8_t *p = src + 4 * i;
        const uint32_t u = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
        dst[i] = __builtin_bit_cast(float, u);
    } else if (dtype == T_F16) {
        dst[i] = f16_to_f32(src[2 * i] | (src[2 * i + 1] << 8));
    } else {
        const uint32_t u = ((uint32_t)(src[2 * i] | (src[2 * i + 1] << 8))) << 16;
        dst[i] = __builtin_bit_cast(float, u);
    }
}

#pragma clang fp contract(on)

// ---- device layout ---------------------------------------------------------
// Q4_K: GGUF bytes unchanged (144-byte blocks and rows are 16-byte aligned).
// Q6_K, Q8_0, Q4_0, Q2_K, IQ2_XXS: blocks are taken 8 at a time in matrix order (row-major
// over (row, block)) and each group of r <= 8 blocks becomes one contiguous
// super-tile with the fields split out:
//   Q6_K [ql r*128 | qh r*64 | scales r*16 | d r*2]   (8 blocks = 1680 B)
//   Q8_0 [qs r*32 | d r*2]                             (8 blocks =  272 B)
//   Q4_0 [qs r*16 | d r*2]                             (8 blocks =  144 B)
//   Q2_K [qs r*64 | scales r*16 | (d, dmin) r*4]       (8 blocks =  672 B)
//   IQ2_XXS [qs r*64 | d r*2]                          (8 blocks =  528 B)
// r = 8 except in the last super-tile of the matrix. The total size equals
// the GGUF size, every field offset is a multiple of 16 (2 for d), and a
// wavefront reading 8 consecutive blocks reads one contiguous region.
// One thread per block; GGUF blocks are 2-byte aligned, read as u16.
__global__ __launch_bounds__(256) void k_prepare_q6k(const uint8_t *__restrict__ src,
                                                     uint8_t *__restrict__ dst, size_t n_blocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const size_t S = i >> 3, j = i & 7;
    const size_t r = (S < (n_blocks >> 3)) ? 8 : (n_blocks & 7);
    uint8_t *st = dst + S * 1680;
    const uint16_t *s = reinterpret_cast<const uint16_t *>(src + i * kQ6kBytes);
    uint16_t *ql = reinterpret_cast<uint16_t *>(st + j * 128);
    uint16_t *qh = reinterpret_cast<uint16_t *>(st + r * 128 + j * 64);
    uint16_t *sc = reinterpret_cast<uint16_t *>(st + r * 192 + j * 16);
    uint16_t *dd = reinterpret_cast<uint16_t *>(st + r * 208 + j * 2);
    for (int k = 0; k < 64; k++) ql[k] = s[k];
    for (int k = 0; k < 32; k++) qh[k] = s[64 + k];
    for (int k = 0; k < 8; k++) sc[k] = s[96 + k];
    dd[0] = s[104];
}

// Q8_0 (block_bytes 34) and Q4_0 (18): [d | qs] -> super-tile [qs... | d...].
__global__ __launch_bounds__(256) void k_prepare_q8_0(const uint8_t *__restrict__ src,
                                                      uint8_t *__restrict__ dst, size_t n_blocks,
                                                      int block_bytes) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const int qbytes = block_bytes - 2;
    const size_t S = i >> 3, j = i & 7;
    const size_t r = (S < (n_blocks >> 3)) ? 8 : (n_blocks & 7);
    uint8_t *st = dst + S * 8 * block_bytes;
    const uint16_t *s = reinterpret_cast<const uint16_t *>(src + i * block_bytes);
    uint16_t *qs = reinterpret_cast<uint16_t *>(st + j * qbytes);
    uint16_t *dd = reinterpret_cast<uint16_t *>(st + r * qbytes + j * 2);
    for (int k = 0; k < qbytes / 2; k++) qs[k] = s[1 + k];
    dd[0] = s[0];
}

// One thread per (block, 16-element sub-block s): q2_k.rs:62-94. Element
// 16s + l (l < 16) of the block: code at shift 2 ((16s % 128) / 32) of qs
// byte 32 (s / 8) + 16 (s & 1) + l; dl = d * sc, ml = dmin * m.
__global__ __launch_bounds__(256) void k_dequant_q2k(const uint8_t *__restrict__ src,
                                                     float *__restrict__ dst, size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 16) return;
    const size_t b = gid >> 4;
    const int sb = (int)(gid & 15);
    const uint8_t *blk = src + b * 84;
    const float d = f16_to_f32(blk[80] | (blk[81] << 8));
    const float dmin = f16_to_f32(blk[82] | (blk[83] << 8));
    const uint32_t sc = blk[sb];
    const float dl = d * (float)(sc & 15u);
    const float ml = dmin * (float)(sc >> 4);
    const uint8_t *q = blk + 16 + 32 * (sb >> 3) + 16 * (sb & 1);
    const int shift = 2 * ((sb & 7) >> 1);
    float *o = dst + b * 256 + 16 * sb;
    for (int l = 0; l < 16; l += 4) {
        float4 v;
        v.x = dl * (float)((q[l + 0] >> shift) & 3) - ml;
        v.y = dl * (float)((q[l + 1] >> shift) & 3) - ml;
        v.z = dl * (float)((q[l + 2] >> shift) & 3) - ml;
        v.w = dl * (float)((q[l + 3] >> shift) & 3) - ml;
        *reinterpret_cast<float4 *>(o + l) = v;
    }
}

// One thread per (block, sub-group g, slot l): iq2_xxs.rs:66-111. Eight
// elements db * grid_byte * sign, db = d * (0.5 + extra) * 0.25.
__global__ __launch_bounds__(256) void k_dequant_iq2xxs(const uint8_t *__restrict__ src,
                                                        float *__restrict__ dst,
                                                        size_t n_blocks) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_blocks * 32) return;
    const size_t b = gid >> 5;
    const int g = (int)((gid >> 2) & 7), l = (int)(gid & 3);
    const uint8_t *blk = src + b * 66;
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    const uint8_t *q = blk + 2 + 8 * g;
    const uint32_t aux1 = q[4] | (q[5] << 8) | (q[6] << 16) | ((uint32_t)q[7] << 24);
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
    const uint64_t grid = kIq2Grid.v[q[l]];
    const uint32_t signs = iq2_signs((aux1 >> (7 * l)) & 0x7Fu);
    float r[8];
    for (int j = 0; j < 8; j++) {
        const float gv = (float)(int)(int8_t)(grid >> (8 * j));
        const float sg = ((signs >> j) & 1u) ? -1.0f : 1.0f;
        r[j] = db * gv * sg;
    }
    float *o = dst + b * 256 + 32 * g + 8 * l;
    *reinterpret_cast<float4 *>(o) = make_float4(r[0], r[1], r[2], r[3]);
    *reinterpret_cast<float4 *>(o + 4) = make_float4(r[4], r[5], r[6], r[7]);
}

// Q2_K (84-byte blocks, 4-byte aligned) -> super-tile [qs r*64 | scales r*16 |
// (d, dmin) r*4].
__global__ __launch_bounds__(256) void k_prepare_q2k(const uint8_t *__restrict__ src,
                                                     uint8_t *__restrict__ dst, size_t n_blocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const size_t S = i >> 3, j = i & 7;
    const size_t r = (S < (n_blocks >> 3)) ? 8 : (n_blocks & 7);
    uint8_t *st = dst + S * 8 * 84;
    const uint32_t *s = reinterpret_cast<const uint32_t *>(src + i * 84);
    uint32_t *qs = reinterpret_cast<uint32_t *>(st + j * 64);
    uint32_t *sc = reinterpret_cast<uint32_t *>(st + r * 64 + j * 16);
    uint32_t *dd = reinterpret_cast<uint32_t *>(st + r * 80 + j * 4);
    for (int k = 0; k < 16; k++) qs[k] = s[4 + k];
    for (int k = 0; k < 4; k++) sc[k] = s[k];
    dd[0] = s[20];
}

// IQ2_XXS (66-byte blocks, 2-byte aligned) -> super-tile [qs r*64 | d r*2].
__global__ __launch_bounds__(256) void k_prepare_iq2xxs(const uint8_t *__restrict__ src,
                                                        uint8_t *__restrict__ dst,
                                                        size_t n_blocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const size_t S = i >> 3, j = i & 7;
    const size_t r = (S < (n_blocks >> 3)) ? 8 : (n_blocks & 7);
    uint8_t *st = dst + S * 8 * 66;
    const uint16_t *s = reinterpret_cast<const uint16_t *>(src + i * 66);
    uint16_t *qs = reinterpret_cast<uint16_t *>(st + j * 64);
    uint16_t *dd = reinterpret_cast<uint16_t *>(st + r * 64 + j * 2);
    for (int k = 0; k < 32; k++) qs[k] = s[1 + k];
    dd[0] = s[0];
}

static inline unsigned grid_for(size_t n, unsigned bs) { return (unsigned)((n + bs - 1) / bs); }

hipError_t launch_dequant(uint32_t dtype, const uint8_t *src, float *dst, size_t n_elems,
                          hipStream_t s) {
    if (n_elems == 0) return hipSuccess;
    switch (dtype) {
    case T_Q4_K:
        k_dequant_q4k<<<grid_for(n_elems / 256 * 8, 256), 256, 0, s>>>(src, dst, n_elems / 256);
        break;
    case T_Q6_K:
        k_dequant_q6k<<<grid_for(n_elems / 256 * 8, 256), 256, 0, s>>>(src, dst, n_elems / 256);
        break;
    case T_Q8_0:
        k_dequant_q8_0<<<grid_for(n_elems / 32, 256), 256, 0, s>>>(src, dst, n_elems / 32);
        break;
    case T_Q4_0:
        k_dequant_q4_0<<<grid_for(n_elems / 32, 256), 256, 0, s>>>(src, dst, n_elems / 32);
        break;
    case T_Q4_1:
        k_dequant_q4_1<<<grid_for(n_elems / 32, 256), 256, 0, s>>>(src, dst, n_elems / 32);
        break;
    case T_Q5_K:
        k_dequant_q5k<<<grid_for(n_elems / 256 * 8, 256), 256, 0, s>>>(src, dst, n_elems / 256);
        break;
    case T_Q8_K:
        k_dequant_q8k<<<grid_for(n_elems / 256 * 8, 256), 256, 0, s>>>(src, dst, n_elems / 256);
        break;
    case T_Q2_K:
        k_dequant_q2k<<<grid_for(n_elems / 256 * 16, 256), 256, 0, s>>>(src, dst, n_elems / 256);
        break;
    case T_IQ2_XXS:
        k_dequant_iq2xxs<<<grid_for(n_elems / 256 * 32, 256), 256, 0, s>>>(src, dst,
                                                                         n_elems / 256);
        break;
    case T_F32:
    case T_F16:
    case T_BF16:
        k_dequant_float<<<grid_for(n_elems, 256), 256, 0, s>>>(src, dst, n_elems, dtype);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_prepare_blocks(uint32_t dtype, const uint8_t *src, uint8_t *dst,
                                 size_t n_blocks, hipStream_t s) {
    const size_t bytes = n_blocks * block_bytes_of(dtype);
    if (bytes == 0) return hipSuccess;
    switch (dtype) {
    case T_Q4_K:
        if (src != dst) return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
        return hipSuccess;
    case T_Q6_K:
        k_prepare_q6k<<<grid_for(n_blocks, 256), 256, 0, s>>>(src, dst, n_blocks);
        break;
    case T_Q8_0:
        k_prepare_q8_0<<<grid_for(n_blocks, 256), 256, 0, s>>>(src, dst, n_blocks, 34);
        break;
    case T_Q4_0:
        k_prepare_q8_0<<<grid_for(n_blocks, 256), 256, 0, s>>>(src, dst, n_blocks, 18);
        break;
    case T_Q2_K:
        k_prepare_q2k<<<grid_for(n_blocks, 256), 256, 0, s>>>(src, dst, n_blocks);
        break;
    case T_IQ2_XXS:
        k_prepare_iq2xxs<<<grid_for(n_blocks, 256), 256, 0, s>>>(src, dst, n_blocks);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_prepare(uint32_t dtype, const uint8_t *src, uint8_t *dst, size_t rows,
                          size_t in_dim, hipStream_t s) {
    const size_t be = block_elems_of(dtype);
    if (be == 0) return hipErrorInvalidValue;
    return launch_prepare_blocks(dtype, src, dst, rows * (in_dim / be), s);
}

}  // namespace rsllm_hip
