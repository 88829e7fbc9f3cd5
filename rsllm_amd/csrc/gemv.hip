// Quantized GEMV, batch 1..n: y[t, o] = sum_i deq(W)[o, i] * x[t, i].
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
// Shape. The kernel streams: a wavefront owns RT rows x one K column of 8
// units (a unit is 128 bytes of quantised payload read by 8 lanes with one
// 16-byte load each: one super-block for Q4_K/Q6_K, 4 blocks for Q8_0, 8
// blocks for Q4_0), issues every load of the column at once, computes, and
// the wavefronts of a workgroup (one per column, up to 16) combine their
// per-row partials through LDS. Weight loads are raw buffer loads, and the
// activation limbs are stored lane-major by the pre-pass so a wavefront's
// activation loads are contiguous 1 KB reads as well.
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
// a lane's groups, valid(), load() of a weight slice, dot().

// Q4_K, GGUF layout. Lane (ks, k) of column c reads block u = 8c + ks: the
// header (d, dmin, 12 scale bytes) and qs bytes 16k..16k+15 = elements
// l = 16*(k&1) + 0..15 of sub-blocks 2p (low nibbles, group "lo") and 2p+1
// (high nibbles, group "hi"), p = k/2.
struct FQ4K {
    static constexpr int kEPU = 256, kXF = 5;
    struct Slice {
        uint4 hdr, qs;
    };
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
    struct Slice {
        uint4 ql, qh, sc;
        uint32_t d;
    };
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

// IQ2_XXS, super-tile layout [qs 8x64 | d 8x2]. Lane (ks, k) of column c reads
// sub-group k (8 bytes) of block u = 8c + ks: elements 32k + 0..15 (grid slots
// 0, 1: group "lo") and 32k + 16..31 (slots 2, 3: "hi"), each an exact int8
// +-{8, 25, 43} (iq2_xxs.rs:66-111); the sub-group scale
// db = d * (0.5 + extra) * 0.25 multiplies the whole slice.
struct FIQ2XXS {
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
    __device__ static float dot(const Slice &s, int, const XSlice &x) {
        const float db = f16_to_f32(s.d) * (0.5f + (float)(s.a1 >> 28)) * 0.25f;
        uint32_t w[8];
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint64_t g = kIq2Grid.v[(s.a0 >> (8 * l)) & 0xFFu];
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

// One thread per 16-element group: thread (lane, half) of column `col` writes
// its limbs to field 0/1 (half 0, "lo") or 3/4 (half 1, "hi") and its
// (s, sum) pair to the lower or upper 8 bytes of the meta field.
template <class F>
__global__ __launch_bounds__(256) void k_quant_x(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                 int in_dim, int ncols, int n_tok) {
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int per_tok = ncols * 64 * kHalves;
    if (gid >= per_tok * n_tok) return;
    const int t = gid / per_tok, rem = gid % per_tok;
    const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
    const int half = r2 / 64, lane = r2 % 64;
    const int k = lane & 7, unit = col * 8 + (lane >> 3);
    const bool ok = unit < F::units(in_dim) && F::valid(unit, k, in_dim);
    const int e = ok ? (half ? F::elem_hi(unit, k) : F::elem_lo(unit, k)) : -1;
    uint4 h, l;
    float s, sum;
    quant_group(x + (size_t)t * in_dim, e, in_dim, h, l, s, sum);
    uint8_t *base = xq + ((size_t)t * ncols + col) * F::kXF * 1024 + lane * 16;
    *reinterpret_cast<uint4 *>(base + (half ? 3 : 0) * 1024) = h;
    *reinterpret_cast<uint4 *>(base + (half ? 4 : 1) * 1024) = l;
    *reinterpret_cast<float2 *>(base + 2 * 1024 + 8 * half) = make_float2(s, sum);
}

// k_quant_x on the SwiGLU of two row-major [rows x n] inputs (gate, up
// pre-activations), for rows < off[n_expert] (the routed slots in use).
template <class F>
__global__ __launch_bounds__(256) void k_quant_swiglu(const float *__restrict__ hg,
                                                      const float *__restrict__ hu, float c,
                                                      uint8_t *__restrict__ xq, int n, int ncols,
                                                      int n_rows, const int *__restrict__ off,
                                                      int n_expert) {
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = ncols * 64 * kHalves;
    const int rows = min(n_rows, off[n_expert]);
    if (gid >= per_row * rows) return;
    const int t = gid / per_row, rem = gid % per_row;
    const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
    const int half = r2 / 64, lane = r2 % 64;
    const int k = lane & 7, unit = col * 8 + (lane >> 3);
    const bool ok = unit < F::units(n) && F::valid(unit, k, n);
    const int e = ok ? (half ? F::elem_hi(unit, k) : F::elem_lo(unit, k)) : -1;
    float v[16];
    if (e >= 0 && e + 16 <= n) {
        const float *g = hg + (size_t)t * n + e, *u = hu + (size_t)t * n + e;
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = swiglu_clamped(g[i], u[i], c);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.f;
    }
    uint4 h, l;
    float s, sum;
    quant_values(v, h, l, s, sum);
    uint8_t *base = xq + ((size_t)t * ncols + col) * F::kXF * 1024 + lane * 16;
    *reinterpret_cast<uint4 *>(base + (half ? 3 : 0) * 1024) = h;
    *reinterpret_cast<uint4 *>(base + (half ? 4 : 1) * 1024) = l;
    *reinterpret_cast<float2 *>(base + 2 * 1024 + 8 * half) = make_float2(s, sum);
}

// ---- GEMV --------------------------------------------------------------------
// blockDim = 64 * NW (NW = min(columns, kMaxWaves)); grid = (ceil(out_dim /
// RT), ceil(n_tok / BT)). Wavefront w handles columns w, w + NW, ...
constexpr int kMaxWaves = 8;
// LDS of the fused batch-1 GEMV (the quantised x of one token): up to 160 KB,
// in_dim <= 32768 for the 256-element formats.
constexpr size_t kGemv1MaxLds = 160 * 1024;

template <class F, int RT, int BT>
__global__ __launch_bounds__(64 * kMaxWaves) void k_gemv(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                               const uint8_t *__restrict__ xq, uint32_t xq_bytes,
                                               float *__restrict__ y, int n_tok, int in_dim,
                                               int out_dim) {
    __shared__ float red[kMaxWaves * RT * BT];
    const int nw = blockDim.x >> 6;
    // wavefront index, made explicitly uniform so per-column offsets stay scalar
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, k = lane & 7, ks = lane >> 3;
    const int row0 = blockIdx.x * RT;
    const int t0 = blockIdx.y * BT;
    const int nunits = F::units(in_dim);
    const int ncols = (nunits + 7) >> 3;
    const uint32_t col_bytes = (uint32_t)F::kXF * 1024u;
    const uint32_t tok_bytes = (uint32_t)ncols * col_bytes;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xq, xq_bytes);

    float acc[RT][BT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = 0.f;

    for (int col = wv; col < ncols; col += nw) {
        const int unit = col * 8 + ks;
        typename F::Slice sl[RT];
#pragma unroll
        for (int r = 0; r < RT; r++)
            F::load(sl[r], rw, min(row0 + r, out_dim - 1), min(unit, nunits - 1), k, in_dim, out_dim);
        XSlice xs[BT];
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const uint32_t so = (uint32_t)min(t0 + t, n_tok - 1) * tok_bytes + (uint32_t)col * col_bytes;
            const uint32_t vo = (uint32_t)lane * 16u;
            xs[t].hlo = bload16(rx, vo, so);
            xs[t].llo = bload16(rx, vo + 1024u, so);
            xs[t].meta = bload16(rx, vo + 2048u, so);
            if (F::kXF == 5) {
                xs[t].hhi = bload16(rx, vo + 3072u, so);
                xs[t].lhi = bload16(rx, vo + 4096u, so);
            }
        }
        if (unit < nunits && F::valid(unit, k, in_dim)) {
#pragma unroll
            for (int t = 0; t < BT; t++)
#pragma unroll
                for (int r = 0; r < RT; r++) acc[r][t] += F::dot(sl[r], k, xs[t]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = wave_sum(acc[r][t]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < BT; t++) red[(r * BT + t) * kMaxWaves + wv] = acc[r][t];
    }
    __syncthreads();
    if ((int)threadIdx.x < RT * BT) {
        const int r = threadIdx.x / BT, t = threadIdx.x % BT;
        float v = 0.f;
        for (int q = 0; q < nw; q++) v += red[threadIdx.x * kMaxWaves + q];
        if (row0 + r < out_dim && t0 + t < n_tok) y[(size_t)(t0 + t) * out_dim + row0 + r] = v;
    }
}

// ---- batch-1 GEMV with the activation pre-pass fused -------------------------
// One launch of n_wg workgroups (one or two per CU) of NW wavefronts.
//
// Rows. Workgroup b owns rows b + n_wg * l (l = 0, 1, ...); wavefront w of
// it takes that list's entries w, w + NW, ... and streams each row's K
// columns (a column = 8 units, one weight "tile") in order, PD tiles in
// flight, keeping the row's per-lane partials in registers: one wavefront
// reduction per row, lane 0 writes the total. Concurrent wavefronts
// therefore read neighbouring rows, and every CU gets the same number of
// rows to within one per wavefront.
//
// Prologue. The workgroup quantises x into LDS in the pre-pass layout
// (thread i takes groups i, i + 64 NW, ...; whole wavefronts without a group
// skip it). Its x loads are issued first and the first PD - 1 tiles right
// after, so the weight stream runs while x is quantised.
//
// Loads are branch-free: a tile past the wavefront's last one is read through
// a zero-length buffer resource (the hardware returns zeros without memory
// traffic), and compiler scheduling barriers keep each step's loads ahead of
// its arithmetic, so the waits before each tile's arithmetic leave the later
// tiles in flight.
//
// DPP row reductions (quad_perm, row_half_mirror, row_mirror) plus four lane
// reads sum a wavefront; the order is fixed, so results are deterministic.
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

template <class F, int NW, int PD, int GPT>
__global__ __launch_bounds__(64 * NW) void k_gemv1(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                  const float *__restrict__ x,
                                                  float *__restrict__ y, int in_dim, int out_dim,
                                                  int n_wg) {
    extern __shared__ uint4 xl[];
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    constexpr int kThreads = 64 * NW;
    const int lane = threadIdx.x & 63, k = lane & 7, ks = lane >> 3;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nunits = F::units(in_dim), ncols = (nunits + 7) >> 3;
    const int n_groups = ncols * 64 * kHalves;
    const int r0 = blockIdx.x;
    const int nrows = (out_dim - r0 + n_wg - 1) / n_wg;                 // this workgroup's rows
    const int my_rows = nrows > wv ? (nrows - wv + NW - 1) / NW : 0;   // this wavefront's rows
    const int T = my_rows * ncols;                                       // its tiles
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(w, 0);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)in_dim * 4u);

    auto group_elem = [&](int g) {
        const int col = g / (64 * kHalves), r2 = g % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        const int kk = ln & 7, unit = col * 8 + (ln >> 3);
        const bool ok = g < n_groups && unit < nunits && F::valid(unit, kk, in_dim);
        return ok ? (half ? F::elem_hi(unit, kk) : F::elem_lo(unit, kk)) : -1;
    };
    auto row_of = [&](int j) { return r0 + n_wg * (wv + NW * j); };
    typename F::Slice buf[PD];
    auto load_tile = [&](typename F::Slice &sl, int t) {
        const int j = t / ncols, col = t - j * ncols;
        const int unit = min(col * 8 + ks, nunits - 1);
        const __amdgpu_buffer_rsrc_t r = t < T ? rw : rnull;
        F::load(sl, r, min(row_of(j), out_dim - 1), unit, k, in_dim, out_dim);
    };

    // Prologue: x loads, the first tiles, then quantisation into LDS. Group
    // indices past n_groups store into one spare column.
    uint4 xv[GPT][4];
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        if (wv * 64 + i * kThreads >= n_groups) continue;
        const int e = group_elem(threadIdx.x + i * kThreads);
        const uint32_t off = e >= 0 ? (uint32_t)e * 4u : 0x80000000u;  // past the end: zeros
#pragma unroll
        for (int q = 0; q < 4; q++) xv[i][q] = bload16(rx, off + 16u * q, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PD - 1; j++) load_tile(buf[j], j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        if (wv * 64 + i * kThreads >= n_groups) continue;
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[4 * q] = __uint_as_float(xv[i][q].x);
            v[4 * q + 1] = __uint_as_float(xv[i][q].y);
            v[4 * q + 2] = __uint_as_float(xv[i][q].z);
            v[4 * q + 3] = __uint_as_float(xv[i][q].w);
        }
        uint4 h, l;
        float sc, sum;
        quant_values(v, h, l, sc, sum);
        const int g = threadIdx.x + i * kThreads;
        const int gg = g < n_groups ? g : n_groups;
        const int col = gg / (64 * kHalves), r2 = gg % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        uint4 *b = xl + col * F::kXF * 64 + ln;
        b[(half ? 3 : 0) * 64] = h;
        b[(half ? 4 : 1) * 64] = l;
        reinterpret_cast<float2 *>(b + 2 * 64)[half] = make_float2(sc, sum);
    }
    __syncthreads();

    float acc = 0.f;
    int col = 0, j = 0;
    for (int t0 = 0; t0 < T; t0 += PD) {
#pragma unroll
        for (int jj = 0; jj < PD; jj++) {
            const int t = t0 + jj;
            load_tile(buf[(jj + PD - 1) % PD], t + PD - 1);
            __builtin_amdgcn_sched_barrier(0);
            XSlice xs;
            const uint4 *bx = xl + col * F::kXF * 64 + lane;
            xs.hlo = bx[0];
            xs.llo = bx[64];
            xs.meta = bx[128];
            if (F::kXF == 5) {
                xs.hhi = bx[192];
                xs.lhi = bx[256];
            }
            const int unit = col * 8 + ks;
            const bool ok = t < T && unit < nunits && F::valid(unit, k, in_dim);
            const float d = F::dot(buf[jj], k, xs);
            acc += ok ? d : 0.f;
            if (col == ncols - 1) {
                const float tot = wave_sum_dpp(acc);
                if (lane == 0 && t < T) y[row_of(j)] = tot;
                acc = 0.f;
                col = 0;
                j++;
            } else {
                col++;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// LDS of k_gemv1: the quantised x (ncols columns) plus one spare column.
template <class F>
static size_t gemv1_lds_bytes(int in_dim) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    return (size_t)(ncols + 1) * F::kXF * 1024;
}

// Groups of x per thread the prologue needs (1, 2 or 4; 0 = too long).
template <class F>
static int gemv1_gpt(int in_dim, int nw) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    const int groups = ncols * 64 * (F::kXF == 5 ? 2 : 1);
    const int gpt = (groups + 64 * nw - 1) / (64 * nw);
    return gpt <= 1 ? 1 : gpt <= 2 ? 2 : gpt <= 4 ? 4 : 0;
}

// Compute units of the current device (cached per device ordinal).
static int device_cus() {
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

template <class F, int NW, int PD, int GPT>
static hipError_t gemv1_go(const uint8_t *w, size_t w_bytes, const float *x, float *y, int in_dim,
                           int out_dim, int n_wg, hipStream_t s) {
    static bool attr_set = false;  // per instantiation; idempotent if raced
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)k_gemv1<F, NW, PD, GPT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kGemv1MaxLds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    n_wg = min(n_wg, out_dim);
    k_gemv1<F, NW, PD, GPT><<<(unsigned)n_wg, 64 * NW, gemv1_lds_bytes<F>(in_dim), s>>>(
        w, (uint32_t)w_bytes, x, y, in_dim, out_dim, n_wg);
    return hipGetLastError();
}

template <class F, int NW, int PD>
static hipError_t gemv1_gpt_go(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                               int in_dim, int out_dim, int n_wg, hipStream_t s) {
    switch (gemv1_gpt<F>(in_dim, NW)) {
    case 1: return gemv1_go<F, NW, PD, 1>(w, w_bytes, x, y, in_dim, out_dim, n_wg, s);
    case 2: return gemv1_go<F, NW, PD, 2>(w, w_bytes, x, y, in_dim, out_dim, n_wg, s);
    case 4: return gemv1_go<F, NW, PD, 4>(w, w_bytes, x, y, in_dim, out_dim, n_wg, s);
    default: return hipErrorInvalidValue;
    }
}

// ---- grouped GEMV (routed experts) ------------------------------------------
// Slot lists sorted by expert: expert e owns slots [off[e], off[e + 1]).
// Workgroup (row tile, e, m) computes y_m[s, rows] = W_m[e] x~[row(s)] for
// every slot s of expert e, in token batches of 4, 2 or 1 (one weight pass
// per batch); row(s) = tok[s] (gate/up: the slot's token) or s (down: the
// slot's own activation). W_m[e] starts at w[m] + e * w_stride.
struct GroupedArgs {
    const uint8_t *w[2];
    uint32_t w_stride;
    const uint8_t *xq;
    uint32_t xq_bytes;
    const int *off;
    const int *tok;  // nullptr: row(s) = s
    const int *act;  // active experts (blockIdx.y indexes it), count in *n_act
    const int *n_act;
    float *y[2];
    int in_dim, out_dim;
};

template <class F, int RT, int BT>
__device__ __forceinline__ void grouped_batch(const GroupedArgs &a, __amdgpu_buffer_rsrc_t rw,
                                              __amdgpu_buffer_rsrc_t rx, float *y, int s_base,
                                              int row0, float *red) {
    const int nw = blockDim.x >> 6;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, k = lane & 7, ks = lane >> 3;
    const int nunits = F::units(a.in_dim);
    const int ncols = (nunits + 7) >> 3;
    const uint32_t col_bytes = (uint32_t)F::kXF * 1024u;
    const uint32_t tok_bytes = (uint32_t)ncols * col_bytes;
    uint32_t trow[BT];
#pragma unroll
    for (int t = 0; t < BT; t++)
        trow[t] = (uint32_t)(a.tok ? a.tok[s_base + t] : s_base + t);

    float acc[RT][BT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = 0.f;

    for (int col = wv; col < ncols; col += nw) {
        const int unit = col * 8 + ks;
        typename F::Slice sl[RT];
#pragma unroll
        for (int r = 0; r < RT; r++)
            F::load(sl[r], rw, min(row0 + r, a.out_dim - 1), min(unit, nunits - 1), k, a.in_dim,
                    a.out_dim);
        XSlice xs[BT];
#pragma unroll
        for (int t = 0; t < BT; t++) {
            const uint32_t so = trow[t] * tok_bytes + (uint32_t)col * col_bytes;
            const uint32_t vo = (uint32_t)lane * 16u;
            xs[t].hlo = bload16(rx, vo, so);
            xs[t].llo = bload16(rx, vo + 1024u, so);
            xs[t].meta = bload16(rx, vo + 2048u, so);
            if (F::kXF == 5) {
                xs[t].hhi = bload16(rx, vo + 3072u, so);
                xs[t].lhi = bload16(rx, vo + 4096u, so);
            }
        }
        if (unit < nunits && F::valid(unit, k, a.in_dim)) {
#pragma unroll
            for (int t = 0; t < BT; t++)
#pragma unroll
                for (int r = 0; r < RT; r++) acc[r][t] += F::dot(sl[r], k, xs[t]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[r][t] = wave_sum(acc[r][t]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < BT; t++) red[(r * BT + t) * kMaxWaves + wv] = acc[r][t];
    }
    __syncthreads();
    if ((int)threadIdx.x < RT * BT) {
        const int r = threadIdx.x / BT, t = threadIdx.x % BT;
        float v = 0.f;
        for (int q = 0; q < nw; q++) v += red[threadIdx.x * kMaxWaves + q];
        if (row0 + r < a.out_dim) y[(size_t)(s_base + t) * a.out_dim + row0 + r] = v;
    }
    __syncthreads();  // red is reused by the next batch
}

template <class F, int RT>
__global__ __launch_bounds__(64 * kMaxWaves) void k_gemv_grouped(GroupedArgs a) {
    __shared__ float red[kMaxWaves * RT * 4];
    if ((int)blockIdx.y >= *a.n_act) return;
    const int e = a.act[blockIdx.y], m = blockIdx.z;
    const int s0 = a.off[e], cnt = a.off[e + 1] - s0;
    if (cnt <= 0) return;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w[m] + (size_t)e * a.w_stride, a.w_stride);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.xq, a.xq_bytes);
    const int row0 = blockIdx.x * RT;
    int done = 0;
    while (cnt - done >= 4) {
        grouped_batch<F, RT, 4>(a, rw, rx, a.y[m], s0 + done, row0, red);
        done += 4;
    }
    if (cnt - done >= 2) {
        grouped_batch<F, RT, 2>(a, rw, rx, a.y[m], s0 + done, row0, red);
        done += 2;
    }
    if (cnt - done >= 1) grouped_batch<F, RT, 1>(a, rw, rx, a.y[m], s0 + done, row0, red);
}

template <class F>
static hipError_t grouped(const GroupedArgs &a, int grid_experts, int n_mat, hipStream_t s) {
    constexpr int RT = 2;
    const int ncols = ((a.in_dim + F::kEPU - 1) / F::kEPU + 7) / 8;
    const int nw = ncols < kMaxWaves ? ncols : kMaxWaves;
    const dim3 grid((unsigned)((a.out_dim + RT - 1) / RT), (unsigned)grid_experts, (unsigned)n_mat);
    k_gemv_grouped<F, RT><<<grid, 64 * nw, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_gemv_grouped(uint32_t dtype, const uint8_t *w0, const uint8_t *w1,
                               size_t w_stride, const uint8_t *xq, size_t xq_bytes,
                               const int *off, const int *tok, const int *act, const int *n_act,
                               int grid_experts, float *y0, float *y1, int in_dim, int out_dim,
                               hipStream_t s) {
    if (grid_experts <= 0 || out_dim <= 0 || in_dim <= 0) return hipSuccess;
    GroupedArgs a;
    a.w[0] = w0;
    a.w[1] = w1 ? w1 : w0;
    a.w_stride = (uint32_t)w_stride;
    a.xq = xq;
    a.xq_bytes = (uint32_t)xq_bytes;
    a.off = off;
    a.tok = tok;
    a.act = act;
    a.n_act = n_act;
    a.y[0] = y0;
    a.y[1] = y1 ? y1 : y0;
    a.in_dim = in_dim;
    a.out_dim = out_dim;
    const int n_mat = w1 ? 2 : 1;
    switch (dtype) {
    case T_Q4_K: return grouped<FQ4K>(a, grid_experts, n_mat, s);
    case T_Q6_K: return grouped<FQ6K>(a, grid_experts, n_mat, s);
    case T_Q8_0: return grouped<FQ8<false>>(a, grid_experts, n_mat, s);
    case T_Q4_0: return grouped<FQ8<true>>(a, grid_experts, n_mat, s);
    case T_Q2_K: return grouped<FQ2K>(a, grid_experts, n_mat, s);
    case T_IQ2_XXS: return grouped<FIQ2XXS>(a, grid_experts, n_mat, s);
    default: return hipErrorInvalidValue;
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

template <class F>
static size_t xq_bytes_for(int n_tok, int in_dim) {
    const int nunits = (in_dim + F::kEPU - 1) / F::kEPU;
    const int ncols = (nunits + 7) / 8;
    return (size_t)n_tok * ncols * F::kXF * 1024;
}

size_t gemv_scratch_bytes(uint32_t dtype, int n_tok, int in_dim) {
    switch (dtype) {
    case T_Q4_K: return xq_bytes_for<FQ4K>(n_tok, in_dim);
    case T_Q6_K: return xq_bytes_for<FQ6K>(n_tok, in_dim);
    case T_Q8_0: return xq_bytes_for<FQ8<false>>(n_tok, in_dim);
    case T_Q4_0: return xq_bytes_for<FQ8<true>>(n_tok, in_dim);
    case T_Q2_K: return xq_bytes_for<FQ2K>(n_tok, in_dim);
    case T_IQ2_XXS: return xq_bytes_for<FIQ2XXS>(n_tok, in_dim);
    default: return 0;
    }
}

size_t gemv_work_bytes(uint32_t dtype, int n_tok, int in_dim, int out_dim) {
    size_t b = gemv_scratch_bytes(dtype, n_tok, in_dim);
    if (gemv_mfma_supported(dtype, n_tok, in_dim, out_dim)) {
        const size_t m = gemv_mfma_scratch_bytes(n_tok, in_dim);
        if (m > b) b = m;
    }
    return b;
}

template <class F, int RT, int BT>
static hipError_t go(const uint8_t *w, size_t w_bytes, const uint8_t *xq, size_t xqb, float *y,
                     int n_tok, int in_dim, int out_dim, hipStream_t s) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) / 8;
    const int nw = ncols < kMaxWaves ? ncols : kMaxWaves;
    const dim3 grid((unsigned)((out_dim + RT - 1) / RT), (unsigned)((n_tok + BT - 1) / BT));
    k_gemv<F, RT, BT><<<grid, 64 * nw, 0, s>>>(w, (uint32_t)w_bytes, xq, (uint32_t)xqb, y, n_tok,
                                               in_dim, out_dim);
    return hipGetLastError();
}

template <class F>
static hipError_t quantize(const float *x, uint8_t *xq, int n_tok, int in_dim, hipStream_t s) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) / 8;
    const int threads = n_tok * ncols * 64 * (F::kXF == 5 ? 2 : 1);
    k_quant_x<F><<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(x, xq, in_dim, ncols, n_tok);
    return hipGetLastError();
}

template <class F>
static hipError_t gemv_pre(const uint8_t *w, size_t w_bytes, const uint8_t *xq, float *y, int n_tok,
                           int in_dim, int out_dim, hipStream_t s) {
    const size_t xqb = xq_bytes_for<F>(n_tok, in_dim);
    if (n_tok == 1) return go<F, 4, 1>(w, w_bytes, xq, xqb, y, n_tok, in_dim, out_dim, s);
    if (n_tok == 2) return go<F, 2, 2>(w, w_bytes, xq, xqb, y, n_tok, in_dim, out_dim, s);
    if (n_tok <= 4) return go<F, 2, 4>(w, w_bytes, xq, xqb, y, n_tok, in_dim, out_dim, s);
    return go<F, 1, 8>(w, w_bytes, xq, xqb, y, n_tok, in_dim, out_dim, s);
}

hipError_t launch_quantize_x(uint32_t dtype, const float *x, uint8_t *xq, int n_tok, int in_dim,
                             hipStream_t s) {
    if (n_tok <= 0 || in_dim <= 0) return hipSuccess;
    switch (dtype) {
    case T_Q4_K: return quantize<FQ4K>(x, xq, n_tok, in_dim, s);
    case T_Q6_K: return quantize<FQ6K>(x, xq, n_tok, in_dim, s);
    case T_Q8_0: return quantize<FQ8<false>>(x, xq, n_tok, in_dim, s);
    case T_Q4_0: return quantize<FQ8<true>>(x, xq, n_tok, in_dim, s);
    case T_Q2_K: return quantize<FQ2K>(x, xq, n_tok, in_dim, s);
    case T_IQ2_XXS: return quantize<FIQ2XXS>(x, xq, n_tok, in_dim, s);
    default: return hipErrorInvalidValue;
    }
}

template <class F>
static hipError_t quantize_swiglu(const float *hg, const float *hu, float c, uint8_t *xq, int n_rows,
                                  int n, const int *off, int n_expert, hipStream_t s) {
    const int ncols = ((n + F::kEPU - 1) / F::kEPU + 7) / 8;
    const int threads = n_rows * ncols * 64 * (F::kXF == 5 ? 2 : 1);
    k_quant_swiglu<F><<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(hg, hu, c, xq, n, ncols,
                                                                       n_rows, off, n_expert);
    return hipGetLastError();
}

hipError_t launch_quantize_swiglu(uint32_t dtype, const float *hg, const float *hu, float clamp,
                                  uint8_t *xq, int n_rows, int n, const int *off, int n_expert,
                                  hipStream_t s) {
    if (n_rows <= 0 || n <= 0) return hipSuccess;
    switch (dtype) {
    case T_Q4_K: return quantize_swiglu<FQ4K>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    case T_Q6_K: return quantize_swiglu<FQ6K>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    case T_Q8_0: return quantize_swiglu<FQ8<false>>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    case T_Q4_0: return quantize_swiglu<FQ8<true>>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    case T_Q2_K: return quantize_swiglu<FQ2K>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    case T_IQ2_XXS: return quantize_swiglu<FIQ2XXS>(hg, hu, clamp, xq, n_rows, n, off, n_expert, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_prequant(uint32_t dtype, const uint8_t *w, size_t w_bytes,
                                const uint8_t *xq, float *y, int n_tok, int in_dim, int out_dim,
                                hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    switch (dtype) {
    case T_Q4_K: return gemv_pre<FQ4K>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    case T_Q6_K: return gemv_pre<FQ6K>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    case T_Q8_0: return gemv_pre<FQ8<false>>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    case T_Q4_0: return gemv_pre<FQ8<true>>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    case T_Q2_K: return gemv_pre<FQ2K>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    case T_IQ2_XXS: return gemv_pre<FIQ2XXS>(w, w_bytes, xq, y, n_tok, in_dim, out_dim, s);
    default: return hipErrorInvalidValue;
    }
}

// Batch 1: the fused kernel. Matrices of 32 MB or more (the weight stream
// dominates) use 8-wavefront workgroups: two per CU with two tiles in flight
// for tall matrices (out_dim >= 2 in_dim), one per CU with three for the
// rest; smaller ones use one 16-wavefront workgroup per CU with two tiles in
// flight. Chosen from sweeps of the C0-C3 shapes on MI355X.
template <class F>
static hipError_t gemv1(const uint8_t *w, size_t w_bytes, const float *x, float *y, int in_dim,
                        int out_dim, hipStream_t s) {
    const int cus = device_cus();
    if (w_bytes >= ((size_t)32 << 20)) {
        if (out_dim >= 2 * in_dim) return gemv1_gpt_go<F, 8, 2>(w, w_bytes, x, y, in_dim, out_dim, 2 * cus, s);
        return gemv1_gpt_go<F, 8, 3>(w, w_bytes, x, y, in_dim, out_dim, cus, s);
    }
    return gemv1_gpt_go<F, 16, 2>(w, w_bytes, x, y, in_dim, out_dim, cus, s);
}

template <class F>
static bool gemv1_fits_f(int in_dim) {
    return gemv1_lds_bytes<F>(in_dim) <= kGemv1MaxLds && gemv1_gpt<F>(in_dim, 8) != 0;
}

static bool gemv1_fits(uint32_t dtype, int in_dim) {
    switch (dtype) {
    case T_Q4_K: return gemv1_fits_f<FQ4K>(in_dim);
    case T_Q6_K: return gemv1_fits_f<FQ6K>(in_dim);
    case T_Q8_0: return gemv1_fits_f<FQ8<false>>(in_dim);
    case T_Q4_0: return gemv1_fits_f<FQ8<true>>(in_dim);
    case T_Q2_K: return gemv1_fits_f<FQ2K>(in_dim);
    case T_IQ2_XXS: return gemv1_fits_f<FIQ2XXS>(in_dim);
    default: return false;
    }
}

hipError_t launch_gemv(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                       uint8_t *xq_scratch, float *y, int n_tok, int in_dim, int out_dim,
                       hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    if (gemv_mfma_supported(dtype, n_tok, in_dim, out_dim))
        return launch_gemv_mfma(dtype, w, w_bytes, x, xq_scratch, y, n_tok, in_dim, out_dim, s);
    if (n_tok == 1 && gemv1_fits(dtype, in_dim)) {
        switch (dtype) {
        case T_Q4_K: return gemv1<FQ4K>(w, w_bytes, x, y, in_dim, out_dim, s);
        case T_Q6_K: return gemv1<FQ6K>(w, w_bytes, x, y, in_dim, out_dim, s);
        case T_Q8_0: return gemv1<FQ8<false>>(w, w_bytes, x, y, in_dim, out_dim, s);
        case T_Q4_0: return gemv1<FQ8<true>>(w, w_bytes, x, y, in_dim, out_dim, s);
        case T_Q2_K: return gemv1<FQ2K>(w, w_bytes, x, y, in_dim, out_dim, s);
        case T_IQ2_XXS: return gemv1<FIQ2XXS>(w, w_bytes, x, y, in_dim, out_dim, s);
        default: return hipErrorInvalidValue;
        }
    }
    hipError_t e = launch_quantize_x(dtype, x, xq_scratch, n_tok, in_dim, s);
    if (e != hipSuccess) return e;
    return launch_gemv_prequant(dtype, w, w_bytes, xq_scratch, y, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
