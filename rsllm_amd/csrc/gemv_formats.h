// Weight formats and activation limbs shared by the GEMV kernels (gemv.hip)
// and the fused routed-expert kernels (moe.hip).
//
// Restates matmul_quant_f32 (rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119)
// without materialising dequantised rows.
//
// Arithmetic. x is first re-expressed per 16-element group g as
//     x~_i = s_g * (256 * h_i + l_i),  h in [-127, 127], l in [-128, 127] (int8),
//     s_g = amax_g / 32512,  |x_i - x~_i| <= s_g / 2 = amax_g / 65024,
// i.e. about 16 bits relative to the group's largest element. A lane decodes
// a 16-byte slice of quantised weights to small integers (Q4_K 0..15,
// Q6_K 0..63, Q4_0 0..15, Q8_0 -128..127) and dots them with both limbs using
// v_dot4_i32_i8 (4 exact int8 MACs per instruction, exact int32 sums). Each
// 16-element partial is then scaled once in fp32:
//     Q4_K  (d*sc_j) * s_g * (256 H + L) - (dmin*m_j) * sum_g x
//     Q6_K  (d*sc_e) * (s_g * (256 H + L) - 32 * sum_g x)
//     Q8_0  d * s_g * (256 H + L)
//     Q4_0  d * (s_g * (256 H + L) - 8 * sum_g x)
// (sum_g x is the fp32 sum of the original x over the group). Only the
// limb representation of x and the summation order differ from the
// reference; the output error is far inside the 1e-3 budget.
//
// Layout of the limbs (the "pre-pass layout"). Per token: ncols columns x kXF
// fields x 64 lanes x 16 bytes, lane-major so one 16-byte read per lane feeds
// v_dot4_i32_i8. Fields: 0 h_lo, 1 l_lo, 2 meta (s_lo, sum_lo, s_hi, sum_hi),
// 3 h_hi, 4 l_hi (kXF = 3 keeps fields 0..2).
//
// Each format gives: kEPU (elements per unit; a unit is 128 bytes of
// quantised payload read by 8 lanes with one 16-byte load each), kXF,
// units(in_dim), the element ranges of a lane's groups, valid(), load() of a
// weight slice, dot().
#pragma once
#include "iq2xxs_grid.h"
#include "kernels.h"

namespace rsllm_hip {

// 256 * sum(q . h) + sum(q . l) over one 16-element group, exact in int32
// (|q| <= 128, |h| <= 127, |l| <= 128: at most 16 * 128 * 32640 < 2^31).
__device__ __forceinline__ int dot16_limbs(const uint32_t (&q)[4], const uint4 &h, const uint4 &l) {
    int ah = 0, al = 0;
    ah = __builtin_amdgcn_sdot4((int)q[0], (int)h.x, ah, false);
    al = __builtin_amdgcn_sdot4((int)q[0], (int)l.x, al, false);
    ah = __builtin_amdgcn_sdot4((int)q[1], (int)h.y, ah, false);
    al = __builtin_amdgcn_sdot4((int)q[1], (int)l.y, al, false);
    ah = __builtin_amdgcn_sdot4((int)q[2], (int)h.z, ah, false);
    al = __builtin_amdgcn_sdot4((int)q[2], (int)l.z, al, false);
    ah = __builtin_amdgcn_sdot4((int)q[3], (int)h.w, ah, false);
    al = __builtin_amdgcn_sdot4((int)q[3], (int)l.w, al, false);
    return ah * 256 + al;
}

// Activation limbs of one lane: groups "lo" and "hi" (see each format for
// which elements they are). meta = (s_lo, sum_lo, s_hi, sum_hi).
struct XSlice {
    uint4 hlo, hhi, llo, lhi, meta;
};

// ---- formats ------------------------------------------------------------------
// Each format gives: kEPU (elements per unit), kXF (activation fields per
// lane: 5 = two groups, 3 = one group), units(in_dim), the element ranges of
// a lane's groups, valid(), load() of a weight slice, dot(). Formats with
// kUniform also give the split form of load() for matrices whose rows are
// whole groups of 8 units (units(in_dim) % 8 == 0): the slice of lane
// (ks, k) in column `col` of row `row` is at tile_base(row, col) (the same
// for the whole wavefront, a scalar offset) plus lane_offs(ks, k) (fixed per
// lane), so a tile costs no per-lane address arithmetic.

// Q4_K, GGUF layout. Lane (ks, k) of column c reads block u = 8c + ks: the
// header (d, dmin, 12 scale bytes) and qs bytes 16k..16k+15 = elements
// l = 16*(k&1) + 0..15 of sub-blocks 2p (low nibbles, group "lo") and 2p+1
// (high nibbles, group "hi"), p = k/2.
struct FQ4K {
    static constexpr int kEPU = 256, kXF = 5;
    static constexpr bool kUniform = true;
    static constexpr int kNO = 2;
    struct Slice {
        uint4 hdr, qs;
    };
    // unit 8 col + ks of the row: block offset (row nb + 8 col) 144 + ks 144
    __device__ static uint32_t tile_base(uint32_t row, uint32_t col, int in_dim) {
        return (row * (uint32_t)(in_dim >> 8) + 8u * col) * 144u;
    }
    __device__ static void lane_offs(uint32_t (&o)[kNO], int ks, int k) {
        o[0] = (uint32_t)ks * 144u;
        o[1] = (uint32_t)ks * 144u + 16u + 16u * (uint32_t)k;
    }
    __device__ static void load_u(Slice &s, __amdgpu_buffer_rsrc_t r, const uint32_t (&o)[kNO],
                                  uint32_t base) {
        s.hdr = bload16(r, o[0], base);
        s.qs = bload16(r, o[1], base);
    }
    __device__ static int units(int in_dim) { return in_dim >> 8; }
    __device__ static int elem_lo(int unit, int k) { return unit * 256 + 64 * (k >> 1) + 16 * (k & 1); }
    __device__ static int elem_hi(int unit, int k) { return elem_lo(unit, k) + 32; }
    __device__ static bool valid(int unit, int, int in_dim) { return unit < (in_dim >> 8); }
    __device__ static void load(Slice &s, __amdgpu_buffer_rsrc_t r, int row, int unit, int k,
                                int in_dim, int) {
        const uint32_t off = ((uint32_t)row * (uint32_t)(in_dim >> 8) + (uint32_t)unit) * 144u;
        s.hdr = bload16(r, off, 0);
        s.qs = bload16(r, off + 16u + 16u * k, 0);
    }
    __device__ static float dot(const Slice &s, int k, const XSlice &x) {
        const int p = k >> 1;
        const float d = f16_to_f32(s.hdr.x & 0xFFFFu);
        const float dmin = f16_to_f32(s.hdr.x >> 16);
        uint32_t sc, m;
        q4k_scale_min(2 * p, s.hdr.y, s.hdr.z, s.hdr.w, sc, m);
        const float dl = d * (float)sc, ml = dmin * (float)m;
        q4k_scale_min(2 * p + 1, s.hdr.y, s.hdr.z, s.hdr.w, sc, m);
        const float dh = d * (float)sc, mh = dmin * (float)m;
        const uint32_t lo[4] = {s.qs.x & 0x0F0F0F0Fu, s.qs.y & 0x0F0F0F0Fu, s.qs.z & 0x0F0F0F0Fu,
                                s.qs.w & 0x0F0F0F0Fu};
        const uint32_t hi[4] = {(s.qs.x >> 4) & 0x0F0F0F0Fu, (s.qs.y >> 4) & 0x0F0F0F0Fu,
                                (s.qs.z >> 4) & 0x0F0F0F0Fu, (s.qs.w >> 4) & 0x0F0F0F0Fu};
        const float slo = __uint_as_float(x.meta.x), sumlo = __uint_as_float(x.meta.y);
        const float shi = __uint_as_float(x.meta.z), sumhi = __uint_as_float(x.meta.w);
        const float plo = (float)dot16_limbs(lo, x.hlo, x.llo) * slo;
        const float phi = (float)dot16_limbs(hi, x.hhi, x.lhi) * shi;
        return dl * plo - ml * sumlo + dh * phi - mh * sumhi;
    }
};

// Q6_K, super-tile layout. Lane (ks, k) of column c reads block u = 8c + ks:
// ql bytes 16k..16k+15 (half h = k/4; stride kq = (k&3)/2 in the low nibbles =
// group "lo", kq+2 in the high nibbles = group "hi"; elements l = 16*(k&1) +
// 0..15), the 16 qh bytes holding their high bit pairs (bits 2kq and 2kq+4),
// the block's 16 scales and d. Element e = 128h + 32kq + l uses scale e/16.
struct FQ6K {
    static constexpr int kEPU = 256, kXF = 5;
    static constexpr bool kUniform = true;
    static constexpr int kNO = 4;
    struct Slice {
        uint4 ql, qh, sc;
        uint32_t d;
    };
    // with units % 8 == 0, block row nb + 8 col + ks is block ks of super-tile
    // row nb / 8 + col, and every super-tile holds 8 blocks
    __device__ static uint32_t tile_base(uint32_t row, uint32_t col, int in_dim) {
        return (row * (uint32_t)(in_dim >> 11) + col) * 1680u;
    }
    __device__ static void lane_offs(uint32_t (&o)[kNO], int ks, int k) {
        o[0] = (uint32_t)ks * 128u + 16u * (uint32_t)k;
        o[1] = 1024u + (uint32_t)ks * 64u + 32u * (uint32_t)(k >> 2) + 16u * (uint32_t)(k & 1);
        o[2] = 1536u + (uint32_t)ks * 16u;
        o[3] = 1664u + (uint32_t)ks * 2u;
    }
    __device__ static void load_u(Slice &s, __amdgpu_buffer_rsrc_t r, const uint32_t (&o)[kNO],
                                  uint32_t base) {
        s.ql = bload16(r, o[0], base);
        s.qh = bload16(r, o[1], base);
        s.sc = bload16(r, o[2], base);
        s.d = bload2(r, o[3], base);
    }
    __device__ static int units(int in_dim) { return in_dim >> 8; }
    __device__ static int elem_lo(int unit, int k) {
        return unit * 256 + 128 * (k >> 2) + 32 * ((k & 3) >> 1) + 16 * (k & 1);
    }
    __device__ static int elem_hi(int unit, int k) { return elem_lo(unit, k) + 64; }
    __device__ static bool valid(int unit, int, int in_dim) { return unit < (in_dim >> 8); }
    __device__ static void load(Slice &s, __amdgpu_buffer_rsrc_t r, int row, int unit, int k,
                                int in_dim, int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)unit;
        const uint32_t S = bi >> 3, j = bi & 7;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 1680u;
        s.ql = bload16(r, base + j * 128u + 16u * k, 0);
        s.qh = bload16(r, base + rS * 128u + j * 64u + 32u * (k >> 2) + 16u * (k & 1), 0);
        s.sc = bload16(r, base + rS * 192u + j * 16u, 0);
        s.d = bload2(r, base + rS * 208u + j * 2u, 0);
    }
    __device__ static float dot(const Slice &s, int k, const XSlice &x) {
        const int kq = (k & 3) >> 1;
        const int sci = 8 * (k >> 2) + 2 * kq + (k & 1);  // scale of group "lo"; "hi" uses +4
        const float d = f16_to_f32(s.d);
        const float dlo = d * (float)sbyte16(s.sc, sci);
        const float dhi = d * (float)sbyte16(s.sc, sci + 4);
        const uint32_t sl = 4 - 2 * kq, sh = 2 * kq;
        const uint32_t lo[4] = {
            (s.ql.x & 0x0F0F0F0Fu) | ((s.qh.x << sl) & 0x30303030u),
            (s.ql.y & 0x0F0F0F0Fu) | ((s.qh.y << sl) & 0x30303030u),
            (s.ql.z & 0x0F0F0F0Fu) | ((s.qh.z << sl) & 0x30303030u),
            (s.ql.w & 0x0F0F0F0Fu) | ((s.qh.w << sl) & 0x30303030u)};
        const uint32_t hi[4] = {
            ((s.ql.x >> 4) & 0x0F0F0F0Fu) | ((s.qh.x >> sh) & 0x30303030u),
            ((s.ql.y >> 4) & 0x0F0F0F0Fu) | ((s.qh.y >> sh) & 0x30303030u),
            ((s.ql.z >> 4) & 0x0F0F0F0Fu) | ((s.qh.z >> sh) & 0x30303030u),
            ((s.ql.w >> 4) & 0x0F0F0F0Fu) | ((s.qh.w >> sh) & 0x30303030u)};
        const float plo = (float)dot16_limbs(lo, x.hlo, x.llo) * __uint_as_float(x.meta.x) -
                          32.f * __uint_as_float(x.meta.y);
        const float phi = (float)dot16_limbs(hi, x.hhi, x.lhi) * __uint_as_float(x.meta.z) -
                          32.f * __uint_as_float(x.meta.w);
        return dlo * plo + dhi * phi;
    }
};

// Q8_0 (Q4 = false) and Q4_0 (Q4 = true), super-tile layout.
// Q8_0: unit = 4 blocks (128 elements); lane (ks, k) reads half k&1 of block
//       32c + 4ks + k/2: 16 signed weights = one group.
// Q4_0: unit = 8 blocks (256 elements); lane (ks, k) reads block 64c + 8ks + k:
//       low nibbles = elements 0..15 (group "lo"), high = 16..31 ("hi"), minus 8.
template <bool Q4>
struct FQ8 {
    static constexpr int kEPU = Q4 ? 256 : 128, kXF = Q4 ? 5 : 3;
    static constexpr bool kUniform = false;
    static constexpr int kNO = 1;
    static constexpr int kQB = Q4 ? 16 : 32, kSTB = Q4 ? 144 : 272;
    struct Slice {
        uint4 q;
        uint32_t d;
    };
    __device__ static int units(int in_dim) { return (in_dim + kEPU - 1) / kEPU; }
    __device__ static int block_of(int unit, int k) { return Q4 ? unit * 8 + k : unit * 4 + (k >> 1); }
    __device__ static int elem_lo(int unit, int k) { return Q4 ? 32 * block_of(unit, k) : unit * 128 + 16 * k; }
    __device__ static int elem_hi(int unit, int k) { return elem_lo(unit, k) + 16; }
    __device__ static bool valid(int unit, int k, int in_dim) { return block_of(unit, k) < (in_dim >> 5); }
    __device__ static void load(Slice &s, __amdgpu_buffer_rsrc_t r, int row, int unit, int k,
                                int in_dim, int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 5);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t b = (uint32_t)block_of(unit, k);
        const uint32_t bi = (uint32_t)row * nb + (b < nb ? b : nb - 1);
        const uint32_t S = bi >> 3, j = bi & 7;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * (uint32_t)kSTB;
        s.q = bload16(r, base + j * (uint32_t)kQB + (Q4 ? 0u : 16u * (k & 1)), 0);
        s.d = bload2(r, base + rS * (uint32_t)kQB + j * 2u, 0);
    }
    __device__ static float dot(const Slice &s, int, const XSlice &x) {
        const float d = f16_to_f32(s.d);
        if (Q4) {
            const uint32_t lo[4] = {s.q.x & 0x0F0F0F0Fu, s.q.y & 0x0F0F0F0Fu, s.q.z & 0x0F0F0F0Fu,
                                    s.q.w & 0x0F0F0F0Fu};
            const uint32_t hi[4] = {(s.q.x >> 4) & 0x0F0F0F0Fu, (s.q.y >> 4) & 0x0F0F0F0Fu,
                                    (s.q.z >> 4) & 0x0F0F0F0Fu, (s.q.w >> 4) & 0x0F0F0F0Fu};
            const float plo = (float)dot16_limbs(lo, x.hlo, x.llo) * __uint_as_float(x.meta.x) -
                              8.f * __uint_as_float(x.meta.y);
            const float phi = (float)dot16_limbs(hi, x.hhi, x.lhi) * __uint_as_float(x.meta.z) -
                              8.f * __uint_as_float(x.meta.w);
            return d * (plo + phi);
        }
        const uint32_t q[4] = {s.q.x, s.q.y, s.q.z, s.q.w};
        return d * ((float)dot16_limbs(q, x.hlo, x.llo) * __uint_as_float(x.meta.x));
    }
};

// Q2_K, super-tile layout [qs 8x64 | scales 8x16 | (d, dmin) 8x4]. Lane (ks, k)
// of column c reads block u = 8c + ks: qs bytes 16 (k / 2) .. + 15 (half h = k / 4,
// run r = (k / 2) & 1) and takes the 2-bit codes at shifts 4p and 4p + 2
// (p = k & 1): elements 128h + 64p + 16r + 0..15 (group "lo", sub-block
// 8h + 4p + r) and the same + 32 (group "hi", sub-block + 2), as
// dequant_q2_k's element order (q2_k.rs:62-94) gives.
struct FQ2K {
    static constexpr bool kUniform = false;
    static constexpr int kNO = 1;
    static constexpr int kEPU = 256, kXF = 5;
    struct Slice {
        uint4 qs;
        uint32_t sc, dd;  // sc: the scale dword holding both of the lane's scale bytes
    };
    __device__ static int units(int in_dim) { return in_dim >> 8; }
    __device__ static int elem_lo(int unit, int k) {
        return unit * 256 + 128 * (k >> 2) + 64 * (k & 1) + 16 * ((k >> 1) & 1);
    }
    __device__ static int elem_hi(int unit, int k) { return elem_lo(unit, k) + 32; }
    __device__ static bool valid(int unit, int, int in_dim) { return unit < (in_dim >> 8); }
    __device__ static void load(Slice &s, __amdgpu_buffer_rsrc_t r, int row, int unit, int k,
                                int in_dim, int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)unit;
        const uint32_t S = bi >> 3, j = bi & 7;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 672u;
        s.qs = bload16(r, base + j * 64u + 16u * (uint32_t)(k >> 1), 0);
        // scale bytes sub and sub + 2 (see dot) share dword sub / 4 = 2 (k / 4) + (k & 1)
        s.sc = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            r, (int)(base + rS * 64u + j * 16u + 8u * (uint32_t)(k >> 2) + 4u * (uint32_t)(k & 1)), 0, 0);
        s.dd = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)(base + rS * 80u + j * 4u), 0, 0);
    }
    __device__ static float dot(const Slice &s, int k, const XSlice &x) {
        const float d = f16_to_f32(s.dd & 0xFFFFu), dmin = f16_to_f32(s.dd >> 16);
        // scale bytes sub = 8 (k / 4) + 4 (k & 1) + ((k / 2) & 1) and sub + 2
        const uint32_t c = 8u * (uint32_t)((k >> 1) & 1);
        const uint32_t sl = (s.sc >> c) & 0xFFu;
        const uint32_t sh = (s.sc >> (c + 16u)) & 0xFFu;
        const float dl = d * (float)(sl & 15u), ml = dmin * (float)(sl >> 4);
        const float dh = d * (float)(sh & 15u), mh = dmin * (float)(sh >> 4);
        const uint32_t shl = 4u * (uint32_t)(k & 1), shh = shl + 2u;
        const uint32_t lo[4] = {(s.qs.x >> shl) & 0x03030303u, (s.qs.y >> shl) & 0x03030303u,
                                (s.qs.z >> shl) & 0x03030303u, (s.qs.w >> shl) & 0x03030303u};
        const uint32_t hi[4] = {(s.qs.x >> shh) & 0x03030303u, (s.qs.y >> shh) & 0x03030303u,
                                (s.qs.z >> shh) & 0x03030303u, (s.qs.w >> shh) & 0x03030303u};
        const float plo = (float)dot16_limbs(lo, x.hlo, x.llo) * __uint_as_float(x.meta.x);
        const float phi = (float)dot16_limbs(hi, x.hhi, x.lhi) * __uint_as_float(x.meta.z);
        return dl * plo - ml * __uint_as_float(x.meta.y) + dh * phi - mh * __uint_as_float(x.meta.w);
    }
};

// Four sign bits (bytes 0..3) applied to four positive int8 magnitudes: each
// flagged byte becomes its two's complement; no byte is 0, so the +1 never
// carries into the next byte.
__device__ __forceinline__ uint32_t iq2_apply_signs(uint32_t mag, uint32_t bits4) {
    const uint32_t one = (bits4 * 0x00204081u) & 0x01010101u;  // bit i -> byte i
    const uint32_t m = (one << 8) - one;                       // 0xFF per flagged byte
    return (mag ^ m) + one;
}

// The IQ2_XXS codebook's LDS copy (2 KB) in every kernel that decodes
// IQ2_XXS rows with FIQ2XXS::dot: staged by stage_format_tables<F>() at the
// kernel's start (a codebook read per 8 weights from LDS instead of
// constant memory).
static __shared__ uint64_t s_iq2_grid64[256];

// IQ2_XXS, super-tile layout [qs 8x64 | d 8x2]. Lane (ks, k) of column c reads
// sub-group k (8 bytes) of block u = 8c + ks: elements 32k + 0..15 (grid slots
// 0, 1: group "lo") and 32k + 16..31 (slots 2, 3: "hi"), each an exact int8
// +-{8, 25, 43} (iq2_xxs.rs:66-111); the sub-group scale
// db = d * (0.5 + extra) * 0.25 multiplies the whole slice.
struct FIQ2XXS {
    static constexpr bool kUniform = false;
    static constexpr int kNO = 1;
    static constexpr int kEPU = 256, kXF = 5;
    struct Slice {
        uint32_t a0, a1, d;
    };
    __device__ static int units(int in_dim) { return in_dim >> 8; }
    __device__ static int elem_lo(int unit, int k) { return unit * 256 + 32 * k; }
    __device__ static int elem_hi(int unit, int k) { return elem_lo(unit, k) + 16; }
    __device__ static bool valid(int unit, int, int in_dim) { return unit < (in_dim >> 8); }
    __device__ static void load(Slice &s, __amdgpu_buffer_rsrc_t r, int row, int unit, int k,
                                int in_dim, int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)unit;
        const uint32_t S = bi >> 3, j = bi & 7;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 528u;
        const uint32_t off = base + j * 64u + 8u * (uint32_t)k;
        s.a0 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
        s.a1 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)(off + 4u), 0, 0);
        s.d = bload2(r, base + rS * 64u + j * 2u, 0);
    }
    __device__ static float dot(const Slice &s, int, const XSlice &x) { return dot_from<true>(s, x); }
    // LDS: the codebook from the workgroup's LDS copy, else from constant
    // memory
    template <bool LDS> __device__ static float dot_from(const Slice &s, const XSlice &x) {
        const float db = f16_to_f32(s.d) * (0.5f + (float)(s.a1 >> 28)) * 0.25f;
        uint32_t w[8];
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t gi = (s.a0 >> (8 * l)) & 0xFFu;
            const uint64_t g = LDS ? s_iq2_grid64[gi] : kIq2Grid.v[gi];
            const uint32_t sg = iq2_signs((s.a1 >> (7 * l)) & 0x7Fu);
            w[2 * l] = iq2_apply_signs((uint32_t)g, sg & 15u);
            w[2 * l + 1] = iq2_apply_signs((uint32_t)(g >> 32), sg >> 4);
        }
        const uint32_t lo[4] = {w[0], w[1], w[2], w[3]};
        const uint32_t hi[4] = {w[4], w[5], w[6], w[7]};
        const float plo = (float)dot16_limbs(lo, x.hlo, x.llo) * __uint_as_float(x.meta.x);
        const float phi = (float)dot16_limbs(hi, x.hhi, x.lhi) * __uint_as_float(x.meta.z);
        return db * (plo + phi);
    }
};

// FIQ2XXS with the codebook read from constant memory: the batch-1 kernel's
// form (there the LDS copy measured slower, 5.5 vs 5.0 us at 2048 x 4096;
// the fused MoE pair gained 13-21% from it).
struct FIQ2XXSK : FIQ2XXS {
    __device__ static float dot(const Slice &s, int, const XSlice &x) { return dot_from<false>(s, x); }
};

// LDS bytes of those tables per format (kernels that size their dynamic LDS
// up to a hard maximum leave them room)
template <class F>
constexpr size_t kFormatTableLds = std::is_same<F, FIQ2XXS>::value ? sizeof(s_iq2_grid64) : 0;

// Tables a format's dot reads from LDS, staged by every thread of the
// workgroup before any of them decodes (call at the kernel's start, before
// any return). BARRIER false: the kernel passes a workgroup barrier of its
// own before its first dot.
template <class F, bool BARRIER = true> __device__ __forceinline__ void stage_format_tables() {
    if constexpr (std::is_same<F, FIQ2XXS>::value) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) s_iq2_grid64[i] = kIq2Grid.v[i];
        if constexpr (BARRIER) __syncthreads();
    }
}

// ---- activation pre-pass -------------------------------------------------------
// Per token: ncols columns x kXF fields x 64 lanes x 16 bytes. Fields:
// 0 h_lo, 1 l_lo, 2 meta (s_lo, sum_lo, s_hi, sum_hi), 3 h_hi, 4 l_hi
// (kXF = 3 keeps fields 0..2). Groups past in_dim are written as zeros.
// Two int8 limbs of 16 values: v ~= s * (256 h + l), s = amax / 32512;
// `sum` is the fp32 sum of the values. A group holding NaN gets s = NaN, so
// every output it feeds is NaN (as in the fp32 reference); +-Inf gives
// s = Inf and limbs 0, hence NaN as well.
__device__ __forceinline__ void quant_values(const float (&v)[16], uint4 &h, uint4 &l, float &s,
                                             float &sum) {
    float amax = 0.f;
    sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    s = sum == sum ? amax * (1.0f / 32512.0f) : sum;
    // t = v / s in [-32512, 32512] (beyond by a few ulp of the approximate
    // reciprocal at most; round(t) stays within +-32512). f = t + 128 +
    // 1.5 * 2^23 rounds t to the nearest integer (ties to even) in the one
    // rounding of the fma, and leaves u = round(t) + 128 in the low 16 bits
    // of f's encoding, as a 16-bit two's complement integer. Then
    //     h = u >> 8 in [-127, 127]                 (byte 1 of f),
    //     l = round(t) - 256 h = (u & 255) - 128    (byte 0 of f, xor 0x80),
    // so round(t) = 256 h + l exactly; v_perm_b32 gathers the bytes. Groups
    // with amax below 2^-100 quantise to zero limbs.
    const float inv = amax > 0x1p-100f ? 32512.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t u[4];
#pragma unroll
        for (int b = 0; b < 4; b++) u[b] = __float_as_uint(fmaf(v[4 * q + b], inv, 12583040.0f));
        const uint32_t l01 = __builtin_amdgcn_perm(u[1], u[0], 0x0C0C0400u);
        const uint32_t l23 = __builtin_amdgcn_perm(u[3], u[2], 0x04000C0Cu);
        const uint32_t h01 = __builtin_amdgcn_perm(u[1], u[0], 0x0C0C0501u);
        const uint32_t h23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010C0Cu);
        lw[q] = (l01 | l23) ^ 0x80808080u;
        hw[q] = h01 | h23;
    }
    h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    l = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

// The 16 values of the group starting at element e (e < 0 or past in_dim:
// zeros).
__device__ __forceinline__ void load_group(const float *__restrict__ x, int e, int in_dim,
                                           float (&v)[16]) {
    if (e >= 0 && e + 16 <= in_dim) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = *reinterpret_cast<const float4 *>(x + e + 4 * i);
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.f;
    }
}

// Group of x starting at element e (e < 0 or past in_dim: zeros).
__device__ __forceinline__ void quant_group(const float *__restrict__ x, int e, int in_dim,
                                            uint4 &h, uint4 &l, float &s, float &sum) {
    float v[16];
    load_group(x, e, in_dim, v);
    quant_values(v, h, l, s, sum);
}

// Routed-expert SwiGLU with the pre-activation clamp (apply_swiglu_clamp,
// rsllm-models/src/dsv4/moe.rs:515-531: only when c > 1e-6, gate from above,
// up both sides, NaN passes) and silu(g) * u with the stable logistic of
// scalar::sigmoid (rsllm-backend-cpu/src/ops/scalar.rs:57-71).
__device__ __forceinline__ float swiglu_clamped(float g, float u, float c) {
    if (c > 1e-6f) {
        if (g > c) g = c;
        if (u > c) u = c;
        else if (u < -c) u = -c;
    }
    float sg;
    if (g >= 0.0f) {
        sg = 1.0f / (1.0f + expf(-g));
    } else {
        const float e = expf(g);
        sg = e / (1.0f + e);
    }
    return g * sg * u;
}

// Sum over a wavefront: DPP row reductions (quad_perm, row_half_mirror,
// row_mirror) plus four lane reads; the order is fixed, so results are
// deterministic. Every lane gets the total.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (a + b) + (c + d);
}


// Compute units of the current device (cached per device ordinal).
inline int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

}  // namespace rsllm_hip
