// Batched GEMV (5..32 tokens; Q8_0 from 9, or from 3 / 5 on matrices of 8192
// or more columns / rows) on the matrix cores:
// y[t, o] = sum_i W[o, i] x[t, i].
//
// Restates matmul_quant_f32 (rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119)
// for the decode batches of C1/C2-style shapes, where the int8-limb GEMV
// (gemv.hip) spends VALU work per (weight, token) pair and stops being
// memory-bound above a few tokens. Here each weight is decoded once per pass
// into an exact f16 integer — Q4_K sc*q, Q6_K sc*(q - 32), Q8_0 q — the B
// operand of v_mfma_f32_16x16x32_f16, against 16 tokens of activations as
// the A operand (fp32 accumulation), so the decode cost is independent of
// the batch. The per-row scales the reference applies in f32 (d, and
// dmin*m for Q4_K through a second MFMA with B = m) multiply each step's
// MFMA result in fp32: the weights reach the products exactly.
//
// Activations: a pre-pass scales each token by 2^e (max |x| into
// [2^14, 2^15)) and splits it into two f16 planes in MFMA operand order,
//   hi[((s * 4 + j) * 4 + q) * ntp + t][0..7] = f16(v), lo[...] = f16(v - hi),
//   v = 2^e_t x[t, F::elem(s, j, q) + 0..7],
// s = K step of 128 elements, j = MFMA of the step, q = lane group, ntp =
// padded token count (8, 16 or 32, padding tokens zero); unscale[t] =
// 2^-e_t. v - hi is exact in fp32, so hi + lo holds x to about 2^-22
// relative; every weight operand meets both planes (one packed operand up
// to 8 tokens, two MFMAs above).
//
// Kernel: workgroup = NK wavefronts over the same 16*RT weight rows; wavefront
// w takes K steps [w * nsteps / NK, (w + 1) * nsteps / NK) with the next
// step's weights and activations in flight while the current one is
// computed. Lane (r, q) = (lane % 16, lane / 16) decodes 32 weights of
// row r per step (8 for each of the 4 MFMAs) and holds D for tokens 4q + 0..3
// of row r. The NK partial tiles are added through LDS in wavefront order
// (deterministic), scaled by 2^-e_t, stored.
#include <type_traits>

#include "gemv_formats.h"
#include "moe_route.h"

namespace rsllm_hip {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfStep = 128;  // K elements per step

// Max over a wavefront (every lane gets it): DPP row reductions plus lane reads.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0);
}

// The weights are the B operand of v_mfma_f32_16x16x32_f16 (K x 16 weight
// rows) and the activations the A operand (16 tokens x K), so lane
// (r16, q) = (lane % 16, lane / 16) supplies weights of row r16 and receives
// D[4q + i][r16], i = 0..3: four tokens of its own row. Every B value is an
// exact integer in f16 — Q4_K sc * q (at most 63 * 15), Q6_K sc * (q - 32)
// (an f16 part and a -1/0/1 remainder where |.| > 2048), Q8_0 q — and the
// per-row scales the reference multiplies in f32 (d, dmin * m) are applied
// to each step's MFMA result in fp32 by the lane that holds that row.
// Products of two f16 values are exact in fp32, so the weights are exact;
// the activations enter as hi + lo f16 planes (about 2^-22 relative).
//
// Each format gives: W (a lane's bytes for one step), elem / piece (the K
// order: element of MFMA j, lane group q, step s), load, and step<NT, PACK>:
// the MFMAs of one step for one 16-row tile against NT token tiles, folded
// into acc[NT] with the scales. With PACK (up to 8 tokens) the A operand x
// holds the hi plane of tokens 0..7 in its rows 0..7 and the lo plane in
// rows 8..15, and xl is not read: one MFMA per sub-step, and D rows t and
// t + 8 add up to token t.

__device__ __forceinline__ f32x4 mfma16x32(const uint4 &x, const f16x8 &w, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, x), w, c, 0, 0, 0);
}

// Q4_K (GGUF layout). Step s = half (s & 1) of super-block s >> 1. Lane group
// q reads qs bytes 32q + 16 (s & 1) .. + 15 (sub-block pair q): low nibbles are
// sub-block 2q, positions 16 (s & 1) + 0..15; high nibbles sub-block 2q + 1.
// MFMA j: low (j even) / high (j odd) nibbles of bytes 0..7 (j < 2) or 8..15.
// B = sc_j * q (exact); a second MFMA per j with B = m_j gives sum m_j x, and
// the step adds d * P - dmin * M (dequant_q4_k, q4_k.rs:66-88: w = d sc q -
// dmin m).
struct MQ4K {
    struct W {
        uint4 hdr, qs;
    };
    __device__ static int elem(int s, int j, int q) {
        return 256 * (s >> 1) + 64 * q + 32 * (j & 1) + 16 * (s & 1) + 8 * (j >> 1);
    }
    // inverse of elem for an 8-aligned element offset: (s, j, q)
    __device__ static void piece(int e, int &s, int &j, int &q) {
        const int r = e & 255;
        q = r >> 6;
        s = 2 * (e >> 8) + ((r >> 4) & 1);
        j = ((r >> 5) & 1) + 2 * ((r >> 3) & 1);
    }
    __device__ static void load(W &w, __amdgpu_buffer_rsrc_t r, int row, int s, int q, int in_dim,
                                int) {
        const uint32_t off = ((uint32_t)row * (uint32_t)(in_dim >> 8) + (uint32_t)(s >> 1)) * 144u;
        w.hdr = bload16(r, off, 0);
        w.qs = bload16(r, off + 16u + 32u * (uint32_t)q + 16u * (uint32_t)(s & 1), 0);
    }
    template <int NT, bool PACK = false>
    __device__ static void step(const W &w, int q, const uint4 (&x)[4][NT], const uint4 (&xl)[4][NT],
                                f32x4 (&acc)[NT]) {
        const float d = f16_to_f32(w.hdr.x & 0xFFFFu), dmin = f16_to_f32(w.hdr.x >> 16);
        // (sc, m) of sub-blocks 2q and 2q + 1 (q4_k_scale_min,
        // dequant/mod.rs:48-58), all four bytes of a word at once: sub-block
        // j < 4 has sc = s0[j] & 63, m = s1[j] & 63; j >= 4 has sc =
        // s2[j - 4] & 15 | (s0[j - 4] >> 6) << 4, m = s2[j - 4] >> 4 |
        // (s1[j - 4] >> 6) << 4. Lane group q takes bytes 2 (q & 1) and
        // 2 (q & 1) + 1 of the low (q < 2) or high words, each paired with
        // 0x64 by v_perm_b32 (the f16 1024 + v, exact) less 1024.
        // (masks and selectors as arithmetic: a conditional here became a
        // branch per tile)
        const uint32_t s0 = w.hdr.y, s1 = w.hdr.z, s2 = w.hdr.w;
        const uint32_t hm = 0u - (uint32_t)(q >> 1);  // all ones for q >= 2
        const uint32_t sc4 = (((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u)) & hm) |
                             (s0 & 0x3F3F3F3Fu & ~hm);
        const uint32_t m4 = ((((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u)) & hm) |
                            (s1 & 0x3F3F3F3Fu & ~hm);
        const uint32_t sel = 0x04010400u + (uint32_t)(q & 1) * 0x00020002u;
        const f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const f16x2 scp = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, sc4, sel)) - k1024;
        const f16x2 mp = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, m4, sel)) - k1024;
        const _Float16 sl = scp[0], sh = scp[1];
        const f16x2 zero = {(_Float16)0.0f, (_Float16)0.0f};
        const f16x2 ssl = {sl, sl}, ssh = {sh, sh};
        f16x8 b[4];
        b[0] = dequant_q4x8_f16(w.qs.x, w.qs.y, false, ssl, zero);
        b[1] = dequant_q4x8_f16(w.qs.x, w.qs.y, true, ssh, zero);
        b[2] = dequant_q4x8_f16(w.qs.z, w.qs.w, false, ssl, zero);
        b[3] = dequant_q4x8_f16(w.qs.z, w.qs.w, true, ssh, zero);
        const _Float16 ml = mp[0], mh = mp[1];
        const f16x8 bml = {ml, ml, ml, ml, ml, ml, ml, ml}, bmh = {mh, mh, mh, mh, mh, mh, mh, mh};
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f32x4 P = {0.f, 0.f, 0.f, 0.f}, M = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                P = mfma16x32(x[j][nt], b[j], P);
                if (!PACK) P = mfma16x32(xl[j][nt], b[j], P);
                M = mfma16x32(x[j][nt], (j & 1) ? bmh : bml, M);
                if (!PACK) M = mfma16x32(xl[j][nt], (j & 1) ? bmh : bml, M);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) acc[nt][i] = fmaf(-dmin, M[i], fmaf(d, P[i], acc[nt][i]));
        }
    }
};

// Four 6-bit codes (bytes 0..63 of q6) -> f16 q - 32 (exact): v_perm_b32
// pairs each byte with 0x64, the f16 pattern of 1024 + q, and subtracting
// 1056 leaves q - 32.
__device__ __forceinline__ void q6x4_f16(uint32_t q6, f16x2 &w01, f16x2 &w23) {
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, q6, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, q6, 0x04030402u);
    const f16x2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    w01 = __builtin_bit_cast(f16x2, p01) - bias;
    w23 = __builtin_bit_cast(f16x2, p23) - bias;
}

// Q6_K (super-tile device layout). Step s = half h = s & 1 of block s >> 1.
// Lane group q reads ql bytes 64h + 16q .. + 15 and qh bytes 32h + 16 (q & 1)
// .. + 15: low nibbles are elements 128h + 16q + b (high bits at 2 (q >> 1)),
// high nibbles elements 128h + 64 + 16q + b (high bits at 4 + 2 (q >> 1));
// their scales are sc[8h + q] and sc[8h + q + 4]. B = sc * (q - 32), and the
// step adds d * P (dequant_q6_k, q6_k.rs:86-92: w = d sc (q - 32)).
// |sc (q - 32)| <= 128 * 32 = 4096: exact in f16 up to 2048, and above that
// (|sc| > 64, which GGUF's int8 scales allow) f16 keeps the even integers
// only. So B = f16(sc (q - 32)) and B_lo = sc (q - 32) - B (one fused f16
// multiply-add, exact, in {-1, 0, 1}); a step whose wavefront has any
// |sc| > 64 adds x_hi * B_lo as a third MFMA per sub-step, which leaves out
// only x_lo * B_lo (below 2^-22 of the term). A step without such scales
// builds 2^-15 B instead, with one FMA per two weights on subnormal codes
// (the same products scaled by a power of two, so the same sums).
struct MQ6K {
    struct W {
        uint4 ql, qh;
        uint32_t sl, sh, d;
    };
    __device__ static int elem(int s, int j, int q) {
        return 256 * (s >> 1) + 128 * (s & 1) + 16 * q + 64 * (j & 1) + 8 * (j >> 1);
    }
    __device__ static void piece(int e, int &s, int &j, int &q) {
        const int r = e & 255;
        s = 2 * (e >> 8) + (r >> 7);
        j = ((r >> 6) & 1) + 2 * ((r >> 3) & 1);
        q = (r >> 4) & 3;
    }
    __device__ static void load(W &w, __amdgpu_buffer_rsrc_t r, int row, int s, int q, int in_dim,
                                int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)(s >> 1);
        const uint32_t S = bi >> 3, jb = bi & 7u;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 1680u, h = (uint32_t)(s & 1);
        w.ql = bload16(r, base + jb * 128u + 64u * h + 16u * (uint32_t)q, 0);
        w.qh = bload16(r, base + rS * 128u + jb * 64u + 32u * h + 16u * (uint32_t)(q & 1), 0);
        w.sl = bload4(r, base + rS * 192u + jb * 16u + 8u * h);
        w.sh = bload4(r, base + rS * 192u + jb * 16u + 8u * h + 4u);
        w.d = bload2(r, base + rS * 208u + jb * 2u, 0);
    }
    // lane holds a scale with |sc| > 64
    __device__ static bool wide_lane(const W &w, int q) {
        const int il = (int)(int8_t)(w.sl >> (8 * q)), ih = (int)(int8_t)(w.sh >> (8 * q));
        return il > 64 || il < -64 || ih > 64 || ih < -64;
    }
    template <int NT, bool PACK = false>
    __device__ static void step(const W &w, int q, const uint4 (&x)[4][NT], const uint4 (&xl)[4][NT],
                                f32x4 (&acc)[NT]) {
        step_m<NT, 2, PACK>(w, q, x, xl, acc);
    }
    // WIDE 0: no scale of the wavefront's step has |sc| > 64 (the caller
    // checked); 1: add the B_lo MFMAs; 2: decide here, per step
    template <int NT, int WIDE, bool PACK>
    __device__ static void step_m(const W &w, int q, const uint4 (&x)[4][NT],
                                  const uint4 (&xl)[4][NT], f32x4 (&acc)[NT]) {
        const float d = f16_to_f32(w.d);
        const int il = (int)(int8_t)(w.sl >> (8 * q)), ih = (int)(int8_t)(w.sh >> (8 * q));
        const bool wide = WIDE == 1 || (WIDE == 2 && __ballot(wide_lane(w, q)) != 0);
        // the high bit pairs sit at bits 2 (q >> 1) (low nibbles) and 4 + 2 (q >> 1)
        // (high nibbles) of each qh byte; one shift puts either pair at bits 4, 5
        const uint32_t shl = 2u * (uint32_t)(q >> 1), sup = 4u - shl;
        const uint32_t l[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
        const uint32_t hb[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        // four 6-bit codes of MFMA j, word u (bytes in K order)
        auto codes = [&](int j, int u) {
            const bool hi = j & 1;
            const int p = 2 * (j >> 1) + u;
            const uint32_t nib = hi ? (l[p] >> 4) & 0x0F0F0F0Fu : l[p] & 0x0F0F0F0Fu;
            const uint32_t top = (hi ? hb[p] >> shl : hb[p] << sup) & 0x30303030u;
            return nib | top;
        };
        f32x4 P[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) P[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto mma = [&](const f16x8 (&b)[4]) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    P[nt] = mfma16x32(x[j][nt], b[j], P[nt]);
                    if (!PACK) P[nt] = mfma16x32(xl[j][nt], b[j], P[nt]);
                }
        };
        float dd = d;
        if (!wide) {
            // |sc| <= 64: B = 2^-15 sc (q - 32), exact, in one FMA per pair:
            // v_perm_b32 zero-extends two codes to f16 bit patterns (the
            // subnormals code * 2^-24), times sc * 2^9, plus -sc * 2^-10; the
            // step's sum is scaled back by 2^15 with d
            const _Float16 ml = (_Float16)((float)il * 512.0f), mh = (_Float16)((float)ih * 512.0f);
            const _Float16 cl = (_Float16)((float)il * -0x1p-10f), ch = (_Float16)((float)ih * -0x1p-10f);
            f16x8 b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f16x2 m2 = (j & 1) ? f16x2{mh, mh} : f16x2{ml, ml};
                const f16x2 c2 = (j & 1) ? f16x2{ch, ch} : f16x2{cl, cl};
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint32_t c = codes(j, u);
                    const f16x2 t01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, c, 0x0c010c00u));
                    const f16x2 t23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, c, 0x0c030c02u));
                    const f16x2 w01 = __builtin_elementwise_fma(t01, m2, c2);
                    const f16x2 w23 = __builtin_elementwise_fma(t23, m2, c2);
                    b[j][4 * u] = w01[0];
                    b[j][4 * u + 1] = w01[1];
                    b[j][4 * u + 2] = w23[0];
                    b[j][4 * u + 3] = w23[1];
                }
            }
            mma(b);
            dd = d * 32768.0f;
        } else {
            const _Float16 scl = (_Float16)(float)il, sch = (_Float16)(float)ih;
            f16x8 a[4], b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                f16x2 v[4];
#pragma unroll
                for (int u = 0; u < 2; u++) q6x4_f16(codes(j, u), v[2 * u], v[2 * u + 1]);
                f16x8 r;
                r[0] = v[0][0]; r[1] = v[0][1]; r[2] = v[1][0]; r[3] = v[1][1];
                r[4] = v[2][0]; r[5] = v[2][1]; r[6] = v[3][0]; r[7] = v[3][1];
                const _Float16 sc = (j & 1) ? sch : scl;
                const f16x8 sv = {sc, sc, sc, sc, sc, sc, sc, sc};
                a[j] = r;
                b[j] = r * sv;
            }
            mma(b);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const _Float16 sc = (j & 1) ? sch : scl;
                const f16x8 sv = {sc, sc, sc, sc, sc, sc, sc, sc};
                const f16x8 bl = __builtin_elementwise_fma(a[j], sv, -b[j]);
#pragma unroll
                for (int nt = 0; nt < NT; nt++) P[nt] = mfma16x32(x[j][nt], bl, P[nt]);
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[nt][i] = fmaf(dd, P[nt][i], acc[nt][i]);
    }
};

// Q8_0 (super-tile device layout [qs 8x32 | d 8x2]). Step s = blocks 4s ..
// 4s + 3 of the row (in_dim is a multiple of 256, so they share one
// super-tile); MFMA j is block 4s + j, lane group q its elements 8q .. 8q + 7.
// A code q (int8) becomes f16 exactly as the pattern 0x64 with byte q ^ 0x80
// (1024 + q + 128) minus 1152; each block's MFMA result is multiplied by its
// scale d in fp32 (dequant_q8_0, q8_0.rs:25-63: w = d q).
struct MQ8 {
    struct W {
        uint2 q[4];
        uint2 d;  // the four blocks' f16 scales
    };
    __device__ static int elem(int s, int j, int q) { return 128 * s + 32 * j + 8 * q; }
    __device__ static void piece(int e, int &s, int &j, int &q) {
        s = e >> 7;
        j = (e >> 5) & 3;
        q = (e >> 3) & 3;
    }
    __device__ static void load(W &w, __amdgpu_buffer_rsrc_t r, int row, int s, int q, int in_dim,
                                int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 5);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + 4u * (uint32_t)s;  // jb is 0 or 4
        const uint32_t S = bi >> 3, jb = bi & 7u;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 272u;
#pragma unroll
        for (int j = 0; j < 4; j++)
            w.q[j] = bload8(r, base + (jb + (uint32_t)j) * 32u + 8u * (uint32_t)q, 0);
        w.d = bload8(r, base + rS * 32u + jb * 2u, 0);
    }
    template <int NT, bool PACK = false>
    __device__ static void step(const W &w, int, const uint4 (&x)[4][NT], const uint4 (&xl)[4][NT],
                                f32x4 (&acc)[NT]) {
        const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
        f16x8 b[4];
        float d[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            d[j] = f16_to_f32(((j & 2) ? w.d.y : w.d.x) >> (16 * (j & 1)));
            f16x8 r;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t bb = (u ? w.q[j].y : w.q[j].x) ^ 0x80808080u;
                const f16x2 w01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, bb, 0x04010400u)) - bias;
                const f16x2 w23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, bb, 0x04030402u)) - bias;
                r[4 * u] = w01[0];
                r[4 * u + 1] = w01[1];
                r[4 * u + 2] = w23[0];
                r[4 * u + 3] = w23[1];
            }
            b[j] = r;
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f32x4 P0 = mfma16x32(x[j][nt], b[j], f32x4{0.f, 0.f, 0.f, 0.f});
                const f32x4 P = PACK ? P0 : mfma16x32(xl[j][nt], b[j], P0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[nt][i] = fmaf(d[j], P[i], acc[nt][i]);
            }
    }
};

// Q2_K (super-tile device layout [qs 8x64 | scales 8x16 | (d, dmin) 8x4],
// 672 bytes per 8 blocks; the matrix's last super-tile holds the blocks
// left). Step s = half n = s & 1 of block s >> 1, its elements in order:
// element 128 n + 32 j + l (l < 32) is bits 2j, 2j + 1 of qs byte 32 n + l
// under scale byte 8 n + 2 j + l / 16 (low nibble sc, high nibble m)
// (dequant_q2_k, q2_k.rs:73-95: w = d sc q - dmin m). MFMA j takes the codes at
// shift 2j; lane group q reads qs bytes 32 n + 8 q .. + 7, all of sub-block
// 8 n + 2 j + q / 2. B = sc * q (exact, at most 45); a second MFMA per j
// with B = m gives sum m x; the step adds d * P - dmin * M.
struct MQ2K {
    struct W {
        uint2 qs, sc;  // the lane's 8 qs bytes; the half's 8 scale bytes
        uint32_t dd;   // f16 d, dmin
    };
    __device__ static int elem(int s, int j, int q) { return 128 * s + 32 * j + 8 * q; }
    __device__ static void piece(int e, int &s, int &j, int &q) {
        s = e >> 7;
        j = (e >> 5) & 3;
        q = (e >> 3) & 3;
    }
    __device__ static void load(W &w, __amdgpu_buffer_rsrc_t r, int row, int s, int q, int in_dim,
                                int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)(s >> 1);
        const uint32_t S = bi >> 3, jb = bi & 7u;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 672u, n = (uint32_t)(s & 1);
        w.qs = bload8(r, base + jb * 64u + 32u * n + 8u * (uint32_t)q, 0);
        w.sc = bload8(r, base + rS * 64u + jb * 16u + 8u * n, 0);
        w.dd = bload4(r, base + rS * 80u + jb * 4u);
    }
    template <int NT, bool PACK = false>
    __device__ static void step(const W &w, int q, const uint4 (&x)[4][NT], const uint4 (&xl)[4][NT],
                                f32x4 (&acc)[NT]) {
        const float d = f16_to_f32(w.dd & 0xFFFFu), dmin = f16_to_f32(w.dd >> 16);
        // the scale bytes 2 j + q / 2 (j = 0..3) of the half, then sc and m
        // as f16 integers (v_perm_b32 against 0x64: the f16 1024 + v, exact,
        // less 1024)
        const uint32_t b4 = __builtin_amdgcn_perm(w.sc.y, w.sc.x,
                                                  0x06040200u + (uint32_t)(q >> 1) * 0x01010101u);
        const uint32_t sc4 = b4 & 0x0F0F0F0Fu, m4 = (b4 >> 4) & 0x0F0F0F0Fu;
        const f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const f16x2 s01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, sc4, 0x04010400u)) - k1024;
        const f16x2 s23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, sc4, 0x04030402u)) - k1024;
        const f16x2 m01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, m4, 0x04010400u)) - k1024;
        const f16x2 m23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, m4, 0x04030402u)) - k1024;
        const _Float16 scj[4] = {s01[0], s01[1], s23[0], s23[1]};
        const _Float16 mj[4] = {m01[0], m01[1], m23[0], m23[1]};
        const f16x2 zero = {(_Float16)0.0f, (_Float16)0.0f};
        f16x8 b[4], bm[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t c0 = (w.qs.x >> (2 * j)) & 0x03030303u;
            const uint32_t c1 = (w.qs.y >> (2 * j)) & 0x03030303u;
            const f16x2 sc2 = {scj[j], scj[j]};
            b[j] = dequant_q4x8_f16(c0, c1, false, sc2, zero);
            const _Float16 m = mj[j];
            bm[j] = f16x8{m, m, m, m, m, m, m, m};
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f32x4 P = {0.f, 0.f, 0.f, 0.f}, M = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                P = mfma16x32(x[j][nt], b[j], P);
                if (!PACK) P = mfma16x32(xl[j][nt], b[j], P);
                M = mfma16x32(x[j][nt], bm[j], M);
                if (!PACK) M = mfma16x32(xl[j][nt], bm[j], M);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) acc[nt][i] = fmaf(-dmin, M[i], fmaf(d, P[i], acc[nt][i]));
        }
    }
};

// IQ2_XXS operands as f16: codebook entry i as 8 f16 magnitudes (8, 25, 43,
// exact), and for each 7-bit sign index the 8 f16 sign bits (its parity as
// the 8th), so a lane's 8 weights are one XOR of two 16-byte table reads.
struct Iq2F16Tables {
    uint32_t grid[256][4];
    uint32_t sign[128][4];
    constexpr Iq2F16Tables() : grid(), sign() {
        constexpr uint32_t f16v[3] = {0x4800u, 0x4E40u, 0x5160u};  // 8, 25, 43
        for (int i = 0; i < 256; i++) {
            uint32_t code = kIq2Codes[i];
            uint32_t h[8] = {};
            for (int j = 0; j < 8; j++) {
                h[j] = f16v[code % 3];
                code /= 3;
            }
            for (int k = 0; k < 4; k++) grid[i][k] = h[2 * k] | h[2 * k + 1] << 16;
        }
        for (uint32_t si = 0; si < 128; si++) {
            uint32_t par = 0;
            for (int b = 0; b < 7; b++) par ^= (si >> b) & 1u;
            const uint32_t s8 = si | par << 7;
            for (int k = 0; k < 4; k++)
                sign[si][k] = ((s8 >> (2 * k)) & 1u) << 15 | ((s8 >> (2 * k + 1)) & 1u) << 31;
        }
    }
};
static __constant__ Iq2F16Tables kIq2F16 = Iq2F16Tables();
// The workgroup's LDS copy (6 KB), staged by MIQ2::stage_tables before the
// first step of a kernel that runs MIQ2::step.
static __shared__ uint4 s_iq2_grid[256];
static __shared__ uint4 s_iq2_sign[128];

// IQ2_XXS (super-tile device layout [qs 8x64 | d 8x2], 528 bytes per 8
// blocks). Step s = sub-groups 4 (s & 1) .. + 3 of block s >> 1, its
// elements in order: MFMA j is sub-group 4 (s & 1) + j (32 elements: 8
// bytes aux0, aux1), lane group q its grid slot q, 8 values from the
// codebook entry aux0 byte q with the sign bits of aux1 bits 7q .. 7q + 6
// (and their parity), each +-{8, 25, 43} (iq2_xxs.rs:66-111), read as f16
// from the tables in LDS; the sub-group's scale db = d (0.5 + (aux1 >> 28)) / 4 is
// exact in fp32 (one FMA: ls d/4 + d/8). B = the value; the step adds
// db_j * P_j.
struct MIQ2 {
    struct W {
        uint4 a[2];  // the step's 4 sub-groups: (aux0, aux1) of 2 per uint4
        uint32_t d;  // f16 d in the low half
    };
    __device__ static int elem(int s, int j, int q) { return 128 * s + 32 * j + 8 * q; }
    __device__ static void piece(int e, int &s, int &j, int &q) {
        s = e >> 7;
        j = (e >> 5) & 3;
        q = (e >> 3) & 3;
    }
    // every thread of the workgroup, before its first step
    __device__ static void stage_tables() {
        for (int i = threadIdx.x; i < 384; i += blockDim.x) {
            if (i < 256)
                s_iq2_grid[i] = *reinterpret_cast<const uint4 *>(kIq2F16.grid[i]);
            else
                s_iq2_sign[i - 256] = *reinterpret_cast<const uint4 *>(kIq2F16.sign[i - 256]);
        }
        __syncthreads();
    }
    __device__ static void load(W &w, __amdgpu_buffer_rsrc_t r, int row, int s, int, int in_dim,
                                int out_dim) {
        const uint32_t nb = (uint32_t)(in_dim >> 8);
        const uint32_t nblk = (uint32_t)out_dim * nb;
        const uint32_t bi = (uint32_t)row * nb + (uint32_t)(s >> 1);
        const uint32_t S = bi >> 3, jb = bi & 7u;
        const uint32_t rS = (S < (nblk >> 3)) ? 8u : (nblk & 7u);
        const uint32_t base = S * 528u, off = base + jb * 64u + 32u * (uint32_t)(s & 1);
        w.a[0] = bload16(r, off, 0);
        w.a[1] = bload16(r, off + 16u, 0);
        w.d = bload2(r, base + rS * 64u + jb * 2u, 0);
    }
    template <int NT, bool PACK = false>
    __device__ static void step(const W &w, int q, const uint4 (&x)[4][NT], const uint4 (&xl)[4][NT],
                                f32x4 (&acc)[NT]) {
        const float d = f16_to_f32(w.d & 0xFFFFu), d4 = d * 0.25f, d8 = d * 0.125f;
        f16x8 b[4];
        float db[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 &a = w.a[j >> 1];
            const uint32_t aux0 = (j & 1) ? a.z : a.x, aux1 = (j & 1) ? a.w : a.y;
            db[j] = fmaf((float)(aux1 >> 28), d4, d8);
            const uint4 gv = s_iq2_grid[(aux0 >> (8 * q)) & 0xFFu];
            const uint4 sv = s_iq2_sign[(aux1 >> (7 * q)) & 0x7Fu];
            b[j] = __builtin_bit_cast(f16x8, make_uint4(gv.x ^ sv.x, gv.y ^ sv.y, gv.z ^ sv.z,
                                                        gv.w ^ sv.w));
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f32x4 P0 = mfma16x32(x[j][nt], b[j], f32x4{0.f, 0.f, 0.f, 0.f});
                const f32x4 P = PACK ? P0 : mfma16x32(xl[j][nt], b[j], P0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[nt][i] = fmaf(db[j], P[i], acc[nt][i]);
            }
    }
};

// Formats whose rows the staged kernels (k_gemv_mfs, k_gemv_mfgs) copy
// through LDS (MfsStage); Q6_K, Q2_K and IQ2_XXS only where in_dim is a
// multiple of 2048 (whole super-tiles per row).
template <class F>
constexpr bool kMfsStaged =
    std::is_same<F, MQ4K>::value || std::is_same<F, MQ6K>::value || std::is_same<F, MQ8>::value ||
    std::is_same<F, MQ2K>::value || std::is_same<F, MIQ2>::value;

// ---- activation pre-pass ---------------------------------------------------------
// Every activation image has two planes of the same layout: hi = f16(v) and
// lo = f16(v - hi) for v = 2^e x (v - hi is exact in fp32), so hi + lo holds
// v to about 2^-22 relative, and each weight operand meets both planes.
__device__ __forceinline__ void hilo8(const float4 &v0, const float4 &v1, float up, uint4 &hi,
                                      uint4 &lo) {
    const float v[8] = {v0.x * up, v0.y * up, v0.z * up, v0.w * up,
                        v1.x * up, v1.y * up, v1.z * up, v1.w * up};
    f16x8 h, l;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        h[i] = (_Float16)v[i];
        l[i] = (_Float16)(v[i] - (float)h[i]);
    }
    hi = __builtin_bit_cast(uint4, h);
    lo = __builtin_bit_cast(uint4, l);
}

// Scale exponent of a row whose largest magnitude is amax: amax * 2^e in
// [2^14, 2^15) (e clamped to [-126, 126]; 0 for a zero or non-finite amax).
// hilo8 with both roundings toward zero, two values per conversion
// instruction: hi keeps a prefix of v's bits, so v - hi is exact in fp32,
// and hi + lo is within 2^-21 |v| (the one-pass kernel converts its slice of
// the activations in every workgroup, where the conversion's VALU time
// shows).
typedef __fp16 h2rtz __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void hilo8_rtz(const float4 &v0, const float4 &v1, float up, uint4 &hi,
                                          uint4 &lo) {
    const float v[8] = {v0.x * up, v0.y * up, v0.z * up, v0.w * up,
                        v1.x * up, v1.y * up, v1.z * up, v1.w * up};
    uint32_t h[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const h2rtz p = __builtin_amdgcn_cvt_pkrtz(v[2 * k], v[2 * k + 1]);
        h[k] = __builtin_bit_cast(uint32_t, p);
        l[k] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(v[2 * k] - (float)p[0],
                                                                       v[2 * k + 1] - (float)p[1]));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}
__device__ __forceinline__ int mf_exponent(float amax) {
    int e = 0;
    if (amax > 0.f && amax <= 3.4e38f) {
        int ex;
        frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
        e = min(max(15 - ex, -126), 126);
    }
    return e;
}

__device__ __forceinline__ float max8(const float4 &a, const float4 &b) {
    return fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                 fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
}

// Max over a workgroup of TH threads (every thread gets it); `red`
// holds one float per wavefront.
constexpr int kMfxThreads = 1024;
template <int TH = 1024>
__device__ __forceinline__ float block_max(float m, float *red) {
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < TH / 64; i++) r = fmaxf(r, red[i]);
    return r;
}

// One workgroup of kMfxThreads per padded token. Each thread holds up to
// kMfxCache 8-element pieces of the row (piece i = thread + kMfxThreads r,
// read once), the workgroup takes the row's max |x|, and the pieces are
// scaled by 2^e, split into hi and lo and stored in operand order (the lo
// plane ntp * in_dim values after the hi plane; F::piece gives a piece's
// slot). Rows longer than kMfxThreads * kMfxCache pieces are read twice.
// Padding tokens write zeros.
constexpr int kMfxCache = 4;
template <class F>
__global__ __launch_bounds__(kMfxThreads) void k_mf_x(const float *__restrict__ x,
                                                      _Float16 *__restrict__ xh,
                                                      float *__restrict__ unscale, int n_tok,
                                                      int in_dim, int ntp) {
    __shared__ float red[kMfxThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    const bool real = t < n_tok;
    const int n8 = in_dim / 8;
    const float4 *xt = reinterpret_cast<const float4 *>(x + (size_t)(real ? t : 0) * in_dim);
    const size_t plane = (size_t)ntp * in_dim;
    auto store = [&](int i, const uint4 &hi, const uint4 &lo) {
        int s, j, q;
        F::piece(8 * i, s, j, q);
        const size_t slot = ((size_t)(s * 4 + j) * 4 + q) * ntp + t;
        *reinterpret_cast<uint4 *>(xh + slot * 8) = hi;
        *reinterpret_cast<uint4 *>(xh + plane + slot * 8) = lo;
    };
    if (!real) {
        if (tid == 0) unscale[t] = 0.f;
        const uint4 z = make_uint4(0, 0, 0, 0);
        for (int i = tid; i < n8; i += kMfxThreads) store(i, z, z);
        return;
    }
    const bool cached = n8 <= kMfxThreads * kMfxCache;
    float4 c[kMfxCache][2];
    float m = 0.f;
    if (cached) {
#pragma unroll
        for (int r = 0; r < kMfxCache; r++) {
            const int i = tid + r * kMfxThreads;
            if (i < n8) {
                c[r][0] = xt[2 * i];
                c[r][1] = xt[2 * i + 1];
                m = fmaxf(m, max8(c[r][0], c[r][1]));
            }
        }
    } else {
        for (int i = tid; i < n8; i += kMfxThreads) m = fmaxf(m, max8(xt[2 * i], xt[2 * i + 1]));
    }
    const int e = mf_exponent(block_max(m, red));
    const float up = ldexpf(1.0f, e);
    if (tid == 0) unscale[t] = ldexpf(1.0f, -e);
    if (cached) {
#pragma unroll
        for (int r = 0; r < kMfxCache; r++) {
            const int i = tid + r * kMfxThreads;
            if (i < n8) {
                uint4 hi, lo;
                hilo8(c[r][0], c[r][1], up, hi, lo);
                store(i, hi, lo);
            }
        }
    } else {
        for (int i = tid; i < n8; i += kMfxThreads) {
            uint4 hi, lo;
            hilo8(xt[2 * i], xt[2 * i + 1], up, hi, lo);
            store(i, hi, lo);
        }
    }
}

// ---- GEMV ----------------------------------------------------------------------------
// One workgroup's 16 * RT rows from row0 against the n_tok (<= 16 * NT)
// token columns of xh (two planes of plane_bytes each), y[t * y_stride + o];
// red: NK * RT * NT * 64 f32x4 of LDS. ROWX (NT = 1): a per-row image (a
// piece's hi and lo 16 bytes side by side), the lane's row at byte xcol,
// and lanes 0..15 hold their column's unscale in usc (unscale unused).
template <class F, int NT, int NK, int RT, bool ROWX = false>
__device__ __forceinline__ void mf_rows(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                        const _Float16 *__restrict__ xh, uint32_t plane_bytes,
                                        const float *__restrict__ unscale, float *__restrict__ y,
                                        int n_tok, int in_dim, int out_dim, int y_stride, int row0,
                                        f32x4 *red, int ntp, uint32_t xcol = 0, float usc = 0.f) {
    static_assert(!ROWX || NT == 1, "per-row images take one token tile");
    if constexpr (std::is_same<F, MIQ2>::value) MIQ2::stage_tables();
    const int lane = threadIdx.x & 63, r16 = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = in_dim / kMfStep;
    const int s0 = nsteps * wv / NK, s1 = nsteps * (wv + 1) / NK;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh, 2 * plane_bytes);

    f32x4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rt][nt] = {0.f, 0.f, 0.f, 0.f};

    typename F::W wa[RT], wb[RT];
    uint4 xa[4][NT], xb[4][NT], la[4][NT], lb[4][NT];
    auto load = [&](typename F::W (&wr)[RT], uint4 (&xr)[4][NT], uint4 (&lr)[4][NT], int s) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
            F::load(wr[rt], rw, min(row0 + 16 * rt + r16, out_dim - 1), s, q, in_dim, out_dim);
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                if (ROWX) {
                    const uint32_t o = xcol + (uint32_t)(((s * 4 + j) * 4 + q) * 32);
                    xr[j][nt] = bload16(rx, o, 0);
                    lr[j][nt] = bload16(rx, o + 16u, 0);
                    continue;
                }
                // image columns past ntp (ntp = 8): zeros, no access
                const int col = nt * 16 + r16;
                const uint32_t o = col < ntp
                    ? (uint32_t)((((s * 4 + j) * 4 + q) * ntp + col) * 16) : 0x7FFFFFF0u;
                xr[j][nt] = bload16(rx, o, 0);
                lr[j][nt] = bload16(rx, col < ntp ? o + plane_bytes : 0x7FFFFFF0u, 0);
            }
    };
    auto compute = [&](const typename F::W (&wr)[RT], const uint4 (&xr)[4][NT],
                       const uint4 (&lr)[4][NT]) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) F::template step<NT>(wr[rt], q, xr, lr, acc[rt]);
    };
    if (s0 < s1) {
        load(wa, xa, la, s0);
        for (int s = s0; s < s1; s += 2) {
            if (s + 1 < s1) load(wb, xb, lb, s + 1);
            compute(wa, xa, la);
            if (s + 1 < s1) {
                if (s + 2 < s1) load(wa, xa, la, s + 2);
                compute(wb, xb, lb);
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) red[((wv * RT + rt) * NT + nt) * 64 + lane] = acc[rt][nt];
    // ROWX: this lane's four tokens' unscales (lane % 64 is the same in
    // every pass of the loop below), read while every lane is active
    float uq[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (ROWX) {
#pragma unroll
        for (int i = 0; i < 4; i++) uq[i] = __shfl(usc, 4 * q + i, 64);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < RT * NT * 64; c += 64 * NK) {
        const int rt = c / (NT * 64), nt = (c / 64) % NT, ln = c % 64;
        f32x4 v = red[(rt * NT + nt) * 64 + ln];
        for (int k = 1; k < NK; k++) v += red[((k * RT + rt) * NT + nt) * 64 + ln];
        // D: tokens 4 (lane / 16) + 0..3 of weight row lane % 16
        const int o = row0 + 16 * rt + (ln & 15);
        const int t0 = nt * 16 + 4 * (ln >> 4);
        if (o < out_dim) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (t0 + i < n_tok)
                    y[(size_t)(t0 + i) * y_stride + o] = v[i] * (ROWX ? uq[i] : unscale[t0 + i]);
        }
    }
}

template <class F, int NT, int NK, int RT>
__global__ __launch_bounds__(64 * NK) void k_gemv_mf(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                     const _Float16 *__restrict__ xh,
                                                     uint32_t plane_bytes,
                                                     const float *__restrict__ unscale,
                                                     float *__restrict__ y, int n_tok, int in_dim,
                                                     int out_dim) {
    __shared__ f32x4 red[NK * RT * NT * 64];
    mf_rows<F, NT, NK, RT>(w, w_bytes, xh, plane_bytes, unscale, y, n_tok, in_dim, out_dim, out_dim,
                           blockIdx.x * 16 * RT, red, NT * 16);
}

// ---- GEMV with the weights staged through LDS -------------------------------------
// The operand loads of mf_rows give each lane of a 16-row tile its own row,
// so one load instruction touches 16 rows' cache lines for a few bytes each
// (L1 requests about 4x those of a contiguous stream). Here a workgroup of 4
// wavefronts (8 up to 8 tokens) owns kMfsRows = 32 rows and streams them in
// chunks of kMfsK = 1024 elements: each row's chunk is one contiguous byte
// range (4 Q4_K blocks; half a Q6_K super-tile's ql / qh / scale runs and
// its d run; 4 Q8_0 super-tiles), copied to LDS with 16-byte buffer-to-LDS
// pieces in row order (every line read whole, no registers held), two
// chunks in flight (double buffer, one barrier per chunk). The wavefronts
// split the chunk's 8 steps (2 each, or 1 with 8 wavefronts) for both row
// tiles, reading the operand fields from LDS (row strides pad to distinct
// LDS banks) against the activation image as mf_rows does. The wavefronts'
// tiles are summed in LDS in wavefront order.
//
// (A design with 512-element chunks in three buffers, two in flight, and
// the activations loaded a chunk ahead measured slower: 19.4 against
// 16.8 us at C1 14336 x 4096, 8 tokens; twice the barriers per byte.)
//
// Matrices with few rows split K: grid.y = sk workgroups per 32 rows, each
// over an equal run of chunks, writing its partial tile to part[split]; a
// second kernel adds the sk partials in split order (deterministic).
typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from a buffer resource into LDS (lane i writes bytes
// 16 i .. 16 i + 15 after the wavefront's base); a lane whose offset lies
// past the resource's size moves zeros without a memory access. (A
// non-template wrapper: the builtin called directly inside a kernel template
// keeps the host pass from emitting that kernel's stub.)
__device__ __forceinline__ void dma16b(__amdgpu_buffer_rsrc_t r, uint32_t voff, lds_void *l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, voff, 0, 0, 0);
}

constexpr int kMfsRows = 32;
constexpr int kMfsK = 1024;
constexpr int kMfsPackWaves = 8;  // wavefronts per workgroup of the packed kernel
// rows per workgroup of the grouped Q4_K kernel with 8-slot batches (64:
// the batch's activation image is read once per 64 rows, and two 80 KB
// workgroups still fit a CU; C3 T = 32: 468 -> 441 us per call)
constexpr int kMfgPackRowsQ4K = 64;
constexpr uint32_t kMfsNoPiece = 0xFFFFFFF0u;  // past every resource: zeros, no access

// Per format: PR 16-byte pieces per row chunk (one pad piece where needed for
// the bank spread); piece k of chunk c of row r is at byte
// off0(r, k) + c_off(c, k) of the weights; load() gives a step's operand
// fields (as F::load) from a row's slice in LDS.
template <class F> struct MfsStage;
template <> struct MfsStage<MQ4K> {
    static constexpr int PR = 37;  // 4 blocks x 144 B = 36 pieces + 1 pad
    __device__ static uint32_t row_bytes(int in_dim) { return (uint32_t)(in_dim >> 8) * 144u; }
    __device__ static uint32_t off0(uint32_t row, int k, int in_dim) {
        return k < 36 ? row * (uint32_t)(in_dim >> 8) * 144u + 16u * (uint32_t)k : kMfsNoPiece;
    }
    __device__ static uint32_t c_off(int c, int) { return (uint32_t)c * 576u; }
    __device__ static void load(MQ4K::W &v, const uint8_t *r, int st, int q, int) {
        const int jb = st >> 1, h = st & 1;
        v.hdr = *reinterpret_cast<const uint4 *>(r + 144 * jb);
        v.qs = *reinterpret_cast<const uint4 *>(r + 144 * jb + 16 + 32 * q + 16 * h);
    }
};
template <> struct MfsStage<MQ6K> {
    // half super-tile (in_dim % 2048 == 0, so a row's blocks fill whole
    // super-tiles): ql 512 B, qh 256 B, scales 64 B (32 + 16 + 4 pieces), and
    // the super-tile's 16 bytes of d
    static constexpr int PR = 53;
    __device__ static uint32_t row_bytes(int in_dim) { return (uint32_t)(in_dim >> 11) * 1680u; }
    __device__ static uint32_t off0(uint32_t row, int k, int in_dim) {
        const uint32_t base = row * (uint32_t)(in_dim >> 11) * 1680u;
        if (k < 32) return base + 16u * k;
        if (k < 48) return base + 1024u + 16u * (k - 32);
        if (k < 52) return base + 1536u + 16u * (k - 48);
        return base + 1664u;
    }
    __device__ static uint32_t c_off(int c, int k) {
        const uint32_t half = k < 32 ? 512u : (k < 48 ? 256u : (k < 52 ? 64u : 0u));
        return (uint32_t)(c >> 1) * 1680u + (uint32_t)(c & 1) * half;
    }
    __device__ static void load(MQ6K::W &v, const uint8_t *r, int st, int q, int c) {
        const int jb = st >> 1, h = st & 1;
        v.ql = *reinterpret_cast<const uint4 *>(r + 128 * jb + 64 * h + 16 * q);
        v.qh = *reinterpret_cast<const uint4 *>(r + 512 + 64 * jb + 32 * h + 16 * (q & 1));
        v.sl = *reinterpret_cast<const uint32_t *>(r + 768 + 16 * jb + 8 * h);
        v.sh = *reinterpret_cast<const uint32_t *>(r + 768 + 16 * jb + 8 * h + 4);
        v.d = *reinterpret_cast<const uint16_t *>(r + 832 + 2 * (4 * (c & 1) + jb));
    }
};
template <> struct MfsStage<MQ8> {
    static constexpr int PR = 69;  // 4 super-tiles x 272 B = 68 pieces + 1 pad
    __device__ static uint32_t row_bytes(int in_dim) { return (uint32_t)(in_dim >> 8) * 272u; }
    __device__ static uint32_t off0(uint32_t row, int k, int in_dim) {
        return k < 68 ? row * (uint32_t)(in_dim >> 8) * 272u + 16u * (uint32_t)k : kMfsNoPiece;
    }
    __device__ static uint32_t c_off(int c, int) { return (uint32_t)c * 1088u; }
    __device__ static void load(MQ8::W &v, const uint8_t *r, int st, int q, int) {
        const uint8_t *t = r + 272 * (st >> 1);
        const int jb = 4 * (st & 1);
#pragma unroll
        for (int j = 0; j < 4; j++) v.q[j] = *reinterpret_cast<const uint2 *>(t + (jb + j) * 32 + 8 * q);
        v.d = *reinterpret_cast<const uint2 *>(t + 256 + 2 * jb);
    }
};

template <> struct MfsStage<MQ2K> {
    // half super-tile (in_dim % 2048 == 0: a row's blocks fill whole
    // super-tiles): qs 256 B, scales 64 B, (d, dmin) 16 B (16 + 4 + 1
    // pieces), in that order in LDS
    static constexpr int PR = 22;
    __device__ static uint32_t row_bytes(int in_dim) { return (uint32_t)(in_dim >> 11) * 672u; }
    __device__ static uint32_t off0(uint32_t row, int k, int in_dim) {
        const uint32_t base = row * (uint32_t)(in_dim >> 11) * 672u;
        if (k < 16) return base + 16u * k;
        if (k < 20) return base + 512u + 16u * (k - 16);
        if (k == 20) return base + 640u;
        return kMfsNoPiece;
    }
    __device__ static uint32_t c_off(int c, int k) {
        const uint32_t half = k < 16 ? 256u : (k < 20 ? 64u : 16u);
        return (uint32_t)(c >> 1) * 672u + (uint32_t)(c & 1) * half;
    }
    __device__ static void load(MQ2K::W &v, const uint8_t *r, int st, int q, int) {
        const int jb = st >> 1, n = st & 1;
        v.qs = *reinterpret_cast<const uint2 *>(r + 64 * jb + 32 * n + 8 * q);
        v.sc = *reinterpret_cast<const uint2 *>(r + 256 + 16 * jb + 8 * n);
        v.dd = *reinterpret_cast<const uint32_t *>(r + 320 + 4 * jb);
    }
};
template <> struct MfsStage<MIQ2> {
    // half super-tile (in_dim % 2048 == 0): qs 256 B (16 pieces) and the
    // super-tile's 16-byte d run
    static constexpr int PR = 18;
    __device__ static uint32_t row_bytes(int in_dim) { return (uint32_t)(in_dim >> 11) * 528u; }
    __device__ static uint32_t off0(uint32_t row, int k, int in_dim) {
        const uint32_t base = row * (uint32_t)(in_dim >> 11) * 528u;
        if (k < 16) return base + 16u * k;
        if (k == 16) return base + 512u;
        return kMfsNoPiece;
    }
    __device__ static uint32_t c_off(int c, int k) {
        return (uint32_t)(c >> 1) * 528u + (k < 16 ? (uint32_t)(c & 1) * 256u : 0u);
    }
    __device__ static void load(MIQ2::W &v, const uint8_t *r, int st, int, int c) {
        const int jb = st >> 1;
        v.a[0] = *reinterpret_cast<const uint4 *>(r + 64 * jb + 32 * (st & 1));
        v.a[1] = *reinterpret_cast<const uint4 *>(r + 64 * jb + 32 * (st & 1) + 16);
        v.d = *reinterpret_cast<const uint16_t *>(r + 256 + 2 * (4 * (c & 1) + jb));
    }
};

template <class F, int NW = 4, int ROWS = kMfsRows> struct MfsGeo {
    static constexpr int THREADS = 64 * NW;
    static constexpr int PIECES = ROWS * MfsStage<F>::PR;
    static constexpr int P = (PIECES + THREADS - 1) / THREADS;  // DMA instructions per thread per chunk
    static constexpr int BUF = P * THREADS * 16;
    static constexpr int LDS = 2 * BUF;
};

// One workgroup's ROWS rows (32 or 64) from row0 of the matrix at w over
// chunks [c0, c0 + nch) against the activation image xh (ntp token columns:
// 8, 16 or 32); y[t * y_stride + o] = 2^-e_t * sum. PACK (ntp = 8, NT = 1):
// lanes of A rows 0..7 read the hi plane of tokens 0..7, lanes of rows 8..15
// the lo plane. NW wavefronts (64 NW threads) split each chunk's 8 steps,
// 8 / NW each, for every row tile. smem: MfsGeo<F, NW, ROWS>::LDS bytes.
// ROWX (NT = 1): a per-row image (a piece's hi and lo 16 bytes side by
// side), the row of the lane's column (r16 & 7 packed, else r16) at byte
// xcol, and lanes 0..15 hold their column's unscale in usc (unscale
// unused).
template <class F, int NT, bool PACK = false, int NW = 4, int ROWS = kMfsRows, bool ROWX = false>
__device__ __forceinline__ void mfs_rows(const uint8_t *__restrict__ w,
                                         const _Float16 *__restrict__ xh, uint32_t plane_bytes,
                                         const float *__restrict__ unscale, float *__restrict__ y,
                                         int y_stride, int n_tok, int in_dim, int out_dim,
                                         int row0, int c0, int nch, int ntp, uint8_t *smem,
                                         uint32_t xcol = 0, float usc = 0.f) {
    static_assert(!ROWX || NT == 1, "per-row images take one token tile");
    if constexpr (std::is_same<F, MIQ2>::value) MIQ2::stage_tables();
    using S = MfsStage<F>;
    using G = MfsGeo<F, NW, ROWS>;
    constexpr int RT = ROWS / 16;
    constexpr int SPW = (kMfsK / kMfStep) / NW;  // steps per wavefront per chunk
    constexpr int TH = G::THREADS;
    const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // this thread's DMA pieces: piece g = p * TH + tid is piece g % PR of
    // row g / PR (rows past out_dim repeat the last; slots past the tile
    // read nothing)
    uint32_t o0[G::P];
    int pk[G::P];
#pragma unroll
    for (int p = 0; p < G::P; p++) {
        const int g = p * TH + tid;
        const int row = min(row0 + g / S::PR, out_dim - 1);
        pk[p] = g % S::PR;
        o0[p] = g < G::PIECES ? S::off0((uint32_t)row, pk[p], in_dim) : kMfsNoPiece;
    }
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)out_dim * S::row_bytes(in_dim));
    auto dma = [&](int c) {
        uint8_t *buf = smem + (c & 1) * G::BUF;
#pragma unroll
        for (int p = 0; p < G::P; p++)
            dma16b(rw, o0[p] == kMfsNoPiece ? kMfsNoPiece : o0[p] + S::c_off(c0 + c, pk[p]),
                   (lds_void *)(buf + 16 * (p * TH + 64 * wv)));
    };
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh, 2 * plane_bytes);
    uint4 xr[SPW][4][NT], lr[SPW][4][NT];
    f32x4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rt][nt] = {0.f, 0.f, 0.f, 0.f};
    // One pass per chunk; every pass but the last issues the next chunk's
    // DMA. PACK: the last pass is a copy without it, so within each copy the
    // count of loads in flight is fixed and the compiler's waits for this
    // chunk's activations leave the next chunk's weights in flight (a
    // conditional DMA in one loop body makes it wait for everything). The
    // wider kernels keep the conditional: the copy costs them registers.
    auto pass = [&](int c, auto has_next) {
        // chunk c's pieces (every wavefront's) have landed, and chunk c - 1's
        // buffer is no longer read
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        // this chunk's activations first, then the next chunk's DMA
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const int st = (c0 + c) * (kMfsK / kMfStep) + SPW * wv + u;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if (ROWX) {
                        const uint32_t o = xcol + (uint32_t)(((st * 4 + j) * 4 + q) * 32);
                        if (PACK) {
                            xr[u][j][nt] = bload16(rx, o + (r16 >= 8 ? 16u : 0u), 0);
                        } else {
                            xr[u][j][nt] = bload16(rx, o, 0);
                            lr[u][j][nt] = bload16(rx, o + 16u, 0);
                        }
                        continue;
                    }
                    if (PACK) {
                        xr[u][j][nt] = bload16(
                            rx, (uint32_t)((((st * 4 + j) * 4 + q) * 8 + (r16 & 7)) * 16) +
                                    (r16 >= 8 ? plane_bytes : 0u), 0);
                        continue;
                    }
                    const int col = nt * 16 + r16;
                    const uint32_t o = col < ntp
                        ? (uint32_t)((((st * 4 + j) * 4 + q) * ntp + col) * 16) : 0x7FFFFFF0u;
                    xr[u][j][nt] = bload16(rx, o, 0);
                    lr[u][j][nt] = bload16(rx, col < ntp ? o + plane_bytes : 0x7FFFFFF0u, 0);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (std::is_same<decltype(has_next), bool>::value) {
            if (has_next) dma(c + 1);
        } else if constexpr (decltype(has_next)::value) {
            dma(c + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *buf = smem + (c & 1) * G::BUF;
        if constexpr (PACK && std::is_same<F, MQ6K>::value) {
            // one test of the scales per chunk keeps the steps in one block,
            // free to interleave
            MQ6K::W wr[SPW][RT];
            bool wl = false;
#pragma unroll
            for (int u = 0; u < SPW; u++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    S::load(wr[u][rt], buf + (16 * rt + r16) * (S::PR * 16), SPW * wv + u, q, c0 + c);
                    wl = wl || MQ6K::wide_lane(wr[u][rt], q);
                }
            if (__ballot(wl) != 0) {
#pragma unroll
                for (int u = 0; u < SPW; u++)
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
                        MQ6K::step_m<NT, 1, PACK>(wr[u][rt], q, xr[u], lr[u], acc[rt]);
            } else {
#pragma unroll
                for (int u = 0; u < SPW; u++)
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
                        MQ6K::step_m<NT, 0, PACK>(wr[u][rt], q, xr[u], lr[u], acc[rt]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < SPW; u++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    typename F::W wr;
                    S::load(wr, buf + (16 * rt + r16) * (S::PR * 16), SPW * wv + u, q, c0 + c);
                    F::template step<NT, PACK>(wr, q, xr[u], lr[u], acc[rt]);
                }
        }
    };
    dma(0);
    if constexpr (PACK) {
        for (int c = 0; c + 1 < nch; c++) pass(c, std::true_type{});
        pass(nch - 1, std::false_type{});
    } else {
        for (int c = 0; c < nch; c++) pass(c, c + 1 < nch);
    }
    __syncthreads();
    f32x4 *red = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) red[((wv * RT + rt) * NT + nt) * 64 + lane] = acc[rt][nt];
    // ROWX: this lane's four tokens' unscales (e % 64 below is the lane),
    // read while every lane is active
    float uq[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (ROWX) {
#pragma unroll
        for (int i = 0; i < 4; i++) uq[i] = __shfl(usc, 4 * q + i, 64);
    }
    __syncthreads();
    for (int e = tid; e < RT * NT * 64; e += TH) {
        const int rt = e / (NT * 64), nt = (e / 64) % NT, ln = e % 64;
        if (PACK && ln >= 32) continue;
        f32x4 v = red[(rt * NT + nt) * 64 + ln];
#pragma unroll
        for (int k = 1; k < NW; k++) v += red[((k * RT + rt) * NT + nt) * 64 + ln];
        if (PACK) {
            // D rows 8..15 (lanes 32..63): the lo plane of the same tokens
#pragma unroll
            for (int k = 0; k < NW; k++) v += red[((k * RT + rt) * NT + nt) * 64 + ln + 32];
        }
        // D: tokens 4 (lane / 16) + 0..3 of weight row lane % 16
        const int o = row0 + 16 * rt + (ln & 15);
        const int t0 = nt * 16 + 4 * (ln >> 4);
        if (o < out_dim) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (t0 + i < n_tok)
                    y[(size_t)(t0 + i) * y_stride + o] = v[i] * (ROWX ? uq[i] : unscale[t0 + i]);
        }
    }
}

// Grid (K splits, 32-row blocks): split x of sk = gridDim.x takes an
// equal run of chunks and writes y + split * n_tok * out_dim. The split
// index varies fastest, and workgroups are dealt to the 8 XCDs in turn, so
// with sk = 2, 4 or 8 each XCD runs one split's workgroups and its L2 holds
// only that split's slice of the activation image (C2 Q8_0 at 32 tokens:
// 12.2 -> 11.8 us for 1024 x 4096, 16.1 -> 15.7 us for 4096 x 4096).
template <class F, int NT, bool PACK = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) void k_gemv_mfs(const uint8_t *__restrict__ w,
                                                  const _Float16 *__restrict__ xh,
                                                  uint32_t plane_bytes,
                                                  const float *__restrict__ unscale,
                                                  float *__restrict__ y, int n_tok, int in_dim,
                                                  int out_dim, int ntp) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nall = in_dim / kMfsK, sk = (int)gridDim.x, z = (int)blockIdx.x;
    const int c0 = nall * z / sk;
    const int nch = nall * (z + 1) / sk - c0;
    mfs_rows<F, NT, PACK, NW>(w, xh, plane_bytes, unscale, y + (size_t)z * n_tok * out_dim,
                              out_dim, n_tok, in_dim, out_dim, (int)blockIdx.y * kMfsRows, c0,
                              nch, ntp, smem);
}

// y[i] = part[0][i] + part[1][i] + ... + part[sk - 1][i], in split order.
// (Adding the partials inside the GEMV, the last split of a row block
// reading the others' write-through partials after a system-scope counter,
// was slower: 12.2 -> 14.6 us at C2 1024 x 4096, 32 tokens: its three
// memory round trips cost more than this launch.)
// The partials are loaded 8 at a time before any is added (a loop of
// dependent load-add pairs waits a full memory round trip per split).
__global__ __launch_bounds__(256) void k_mfs_sum(const float *__restrict__ part,
                                                 float *__restrict__ y, int n, int sk) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = 0.f;
    for (int k0 = 0; k0 < sk; k0 += 8) {
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; k++) p[k] = k0 + k < sk ? part[(size_t)(k0 + k) * n + i] : 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (k0 + k < sk) v = k0 + k == 0 ? p[k] : v + p[k];
    }
    y[i] = v;
}

// ---- small matrices in one pass ----------------------------------------------------
// Matrices whose weights, spread over about one workgroup per CU, fit in
// LDS whole (C2-style 1024- and 4096-row Q8_0 / Q4_K matrices at 9..32
// tokens). Grid (sk K slices, row blocks of R = 16 RTW NW rows), slice z
// covering elements [z KS, (z + 1) KS). Each workgroup
//   1. reads its activations' slice (ntp tokens x KS values, fp32) and
//      issues the copy of its rows' weight slice (one contiguous byte run
//      per row: KS / 256 Q8_0 super-tiles or Q4_K blocks) into LDS with
//      16-byte buffer-to-LDS pieces, all in flight at once, in two phases
//      of half the slice where KS = 512;
//   2. scales each token's slice by 2^e (its max |x| into [2^14, 2^15),
//      over this slice only) and stores the hi and lo f16 planes to LDS in
//      the MFMA operand order of the activation image (k_mf_x);
//   3. after a barrier, wavefront w runs row tiles RTW w .. RTW w + RTW - 1
//      over the first phase's steps against every token tile (the
//      activation operands read from LDS once per step for all of them),
//      then, after a second barrier, over the second phase's, and
//   4. stores its tile scaled by 2^-e: to y when there is one slice, else to
//      the slice's partial, which k_mfs_sum adds in slice order.
// No activation pre-pass launch and no activation image in memory, and
// each workgroup reads only its slice of x (ntp * KS * 4 bytes, about its
// weight bytes at R = 128, KS = 512). The weights reach the products
// exactly, as in the other matrix-core kernels; the activations as hi + lo.
// LDS slot of piece row p (the ((s * 4 + j) * 4 + q) of the image layout),
// token column t: the column XOR-ed with p's low bits, so the prologue's
// stores (a wavefront's lanes: one token, consecutive p) and the operand
// reads (consecutive columns, four p) both spread over the LDS banks.
template <int NTP>
__device__ __forceinline__ int mfo_slot(int p, int t) {
    return p * NTP + (t ^ (p & (NTP - 1)));
}

// Max over each half of a wavefront (lanes 0..31 and 32..63), returned to
// every lane of that half: DPP within rows of 16, then the row maxima.
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (threadIdx.x & 32) ? fmaxf(c, d) : fmaxf(a, b);
}

template <class F> struct MfoRow;  // bytes per 256 elements of a row
template <> struct MfoRow<MQ8> { static constexpr int kB256 = 272; };
template <> struct MfoRow<MQ4K> { static constexpr int kB256 = 144; };

template <class F, int NT, int NW, int KS, int RTW>
struct MfoGeo {
    static constexpr int NTP = 16 * NT;                     // token columns
    static constexpr int TH = 64 * NW;
    static constexpr int R = 16 * RTW * NW;                 // rows per workgroup
    static constexpr int NPH = KS >= 512 ? 2 : 1;           // weight phases (256+ elements each)
    static constexpr int KP = KS / NPH;                     // elements per phase
    static constexpr int PR = KP / 256 * MfoRow<F>::kB256 / 16 + 1;  // pieces per row, + 1 pad
    static constexpr int WP = (R * PR + TH - 1) / TH;       // weight pieces per thread per phase
    static constexpr int NS = KS / kMfStep;                 // steps
    static constexpr int NSP = NS / NPH;                    // steps per phase
    static constexpr int PT = KS / 8;                       // 8-element pieces per token
    static constexpr int XP = NTP * PT / TH;                // activation pieces per thread
    static constexpr int W_BUF = WP * TH * 16;              // one phase's weights
    static constexpr int W_LDS = NPH * W_BUF;
    static constexpr int LDS = W_LDS + 2 * NTP * KS * 2;    // weights + two f16 planes
};

template <class F, int NT, int NW, int KS, int RTW>
__global__ __launch_bounds__(64 * NW) void k_gemv_mfo(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ dst, int n_tok,
                                                      int in_dim, int out_dim) {
    using G = MfoGeo<F, NT, NW, KS, RTW>;
    static_assert(G::PT == 32 || G::PT == 64, "a token's slice spans half or all of a wavefront");
    static_assert(G::XP * G::TH == G::NTP * G::PT, "activation pieces divide evenly");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float us[G::NTP];
    uint8_t *wbuf = smem;
    uint4 *xh = reinterpret_cast<uint4 *>(smem + G::W_LDS);  // hi plane, then lo
    uint4 *xlo = xh + G::NS * 16 * G::NTP;
    const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int z = blockIdx.x, k0 = z * KS, row0 = blockIdx.y * G::R;
    // 1. activation loads, then the weight copy
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)n_tok * (uint32_t)in_dim * 4u);
    uint4 xv[G::XP][2];
#pragma unroll
    for (int r = 0; r < G::XP; r++) {
        const int g = r * G::TH + tid, t = g / G::PT, i = g - t * G::PT;
        const uint32_t off =
            t < n_tok ? ((uint32_t)t * (uint32_t)in_dim + (uint32_t)(k0 + 8 * i)) * 4u : 0x80000000u;
        xv[r][0] = bload16(rx, off, 0);
        xv[r][1] = bload16(rx, off + 16u, 0);
    }
    // the weight copy waits for the activations: issued together, the
    // activation misses queue behind the whole slice's weight traffic
    // (MI355X, 4096 x 4096 Q8_0 at 32 tokens: activations after 3.5 us
    // instead of 0.8)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t row_bytes = (uint32_t)(in_dim / 256) * (uint32_t)MfoRow<F>::kB256;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)out_dim * row_bytes);
#pragma unroll
    for (int ph = 0; ph < G::NPH; ph++) {
        const uint32_t slice_off = (uint32_t)((k0 + ph * G::KP) / 256) * (uint32_t)MfoRow<F>::kB256;
#pragma unroll
        for (int p = 0; p < G::WP; p++) {
            const int g = p * G::TH + tid, row = g / G::PR, k = g - row * G::PR;
            const uint32_t off = g < G::R * G::PR && k < G::PR - 1 && row0 + row < out_dim
                ? (uint32_t)(row0 + row) * row_bytes + slice_off + 16u * (uint32_t)k
                : kMfsNoPiece;
            dma16b(rw, off, (lds_void *)(wbuf + ph * G::W_BUF + 16 * (p * G::TH + 64 * wv)));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. per-token exponent over the slice (a wavefront holds one token's
    // pieces, or two at PT = 32: its halves), then the two planes
#pragma unroll
    for (int r = 0; r < G::XP; r++) {
        const int g = r * G::TH + tid, t = g / G::PT, i = g - t * G::PT;
        const float4 a = __builtin_bit_cast(float4, xv[r][0]), b = __builtin_bit_cast(float4, xv[r][1]);
        const float m = G::PT == 64 ? wave_max(max8(a, b)) : half_wave_max(max8(a, b));
        const int e = mf_exponent(m);
        if (i == 0) us[t] = ldexpf(1.0f, -e);
        uint4 hi, lo;
        hilo8_rtz(a, b, ldexpf(1.0f, e), hi, lo);
        int s_, j_, q_;
        F::piece(8 * i, s_, j_, q_);
        const int slot = mfo_slot<G::NTP>((s_ * 4 + j_) * 4 + q_, t);
        xh[slot] = hi;
        xlo[slot] = lo;
    }
    // 3. row tiles wv * RTW .. + RTW - 1 over the slice (each step's
    // activation operands read from LDS once for all of them), phase by
    // phase: the first phase's steps run while the second's weights land
    f32x4 acc[RTW][NT];
#pragma unroll
    for (int rt = 0; rt < RTW; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rt][nt] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < G::NS; st++) {
        if (st % G::NSP == 0) {
            // this thread's pieces of phase st / NSP have landed (the later
            // phase's, issued after, may still be in flight), then everyone's
            if (st == 0 && G::NPH == 2)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(G::WP) : "memory");
            else
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __syncthreads();
        }
        const uint8_t *wph = wbuf + (st / G::NSP) * G::W_BUF;
        uint4 xr[4][NT], lr[4][NT];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int slot = mfo_slot<G::NTP>((st * 4 + j) * 4 + q, nt * 16 + r16);
                xr[j][nt] = xh[slot];
                lr[j][nt] = xlo[slot];
            }
#pragma unroll
        for (int rt = 0; rt < RTW; rt++) {
            typename F::W wr;
            MfsStage<F>::load(wr, wph + (16 * (wv * RTW + rt) + r16) * G::PR * 16, st % G::NSP, q, 0);
            F::template step<NT>(wr, q, xr, lr, acc[rt]);
        }
    }
    // 4. D: tokens 16 nt + 4 q + 0..3 of weight row r16
    float *out = dst + (gridDim.x > 1 ? (size_t)z * n_tok * out_dim : 0);
#pragma unroll
    for (int rt = 0; rt < RTW; rt++) {
        const int o = row0 + 16 * (wv * RTW + rt) + r16;
        if (o < out_dim) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = nt * 16 + 4 * q + i;
                    if (t < n_tok) out[(size_t)t * out_dim + o] = acc[rt][nt][i] * us[t];
                }
        }
    }
}

// ---- routed experts grouped by expert (many tokens) --------------------------------
// Slots sorted by expert (moe.hip routing): expert e owns sorted slots [off[e],
// off[e + 1]), cut into batches of up to bw = 8 or 16 (mfg_width; k_moe_scan
// lists them); a batch is the token set (the N dimension) of one pass over
// that expert's rows, so each expert's weights are streamed once per bw of
// its slots. The activation images hold one row per x row (gate/up) or per
// slot (down), not per batch column: row r's 8-element pieces in MFMA
// operand order, scaled by 2^e_r, piece p = ((s * 4 + j) * 4 + q) as its hi
// 16 bytes at byte 4 r in_dim + 32 p and its lo 16 bytes right after (a
// lane group's hi and lo pieces of one MFMA share a 128-byte line);
// unscale[r] = 2^-e_r. Column c of batch b reads row tok[first + c]
// (gate/up) or first + c (down). A row is written once however many
// batches read it, by one workgroup, in whole cache lines.

// One token column of an ntp-wide activation image (the k_mf_x conversion,
// one workgroup of TH threads, the row read once when it fits in
// registers): val4(i) gives elements i .. i + 3 of the column's row; the
// column's pieces go to both planes of the image at xb (the lo plane
// `plane` halves after the hi plane; 0: in_dim * ntp), 2^-e to *us.
template <class F, int TH = kMfxThreads, class V>
__device__ __forceinline__ void mf_x_column(V val4, int in_dim, int t, _Float16 *__restrict__ xb,
                                            float *__restrict__ us, int ntp, size_t plane = 0) {
    __shared__ float red[TH / 64];
    const int tid = threadIdx.x;
    const int n8 = in_dim / 8;
    if (plane == 0) plane = (size_t)in_dim * ntp;
    auto store = [&](int i, const uint4 &hi, const uint4 &lo) {
        int s, j, q;
        F::piece(8 * i, s, j, q);
        const size_t slot = ((size_t)(s * 4 + j) * 4 + q) * ntp + t;
        *reinterpret_cast<uint4 *>(xb + slot * 8) = hi;
        *reinterpret_cast<uint4 *>(xb + plane + slot * 8) = lo;
    };
    // pieces read once (kept in registers) when the row fits
    const bool cached = n8 <= TH * kMfxCache;
    float4 c[kMfxCache][2];
    float m = 0.f;
    if (cached) {
#pragma unroll
        for (int r = 0; r < kMfxCache; r++) {
            const int i = tid + r * TH;
            if (i < n8) {
                c[r][0] = val4(8 * i);
                c[r][1] = val4(8 * i + 4);
                m = fmaxf(m, max8(c[r][0], c[r][1]));
            }
        }
    } else {
        for (int i = tid; i < n8; i += TH) m = fmaxf(m, max8(val4(8 * i), val4(8 * i + 4)));
    }
    const int e = mf_exponent(block_max<TH>(m, red));
    const float up = ldexpf(1.0f, e);
    if (tid == 0) *us = ldexpf(1.0f, -e);
    if (cached) {
#pragma unroll
        for (int r = 0; r < kMfxCache; r++) {
            const int i = tid + r * TH;
            if (i < n8) {
                uint4 hi, lo;
                hilo8(c[r][0], c[r][1], up, hi, lo);
                store(i, hi, lo);
            }
        }
    } else {
        for (int i = tid; i < n8; i += TH) {
            uint4 hi, lo;
            hilo8(val4(8 * i), val4(8 * i + 4), up, hi, lo);
            store(i, hi, lo);
        }
    }
}

// Row blockIdx.x of a per-row image: x row r, or (SWIGLU) the clamped
// SwiGLU of rows r of hg (x) and hu. Rows at or past *n_rows (when given)
// exit: slots past the routed ones.
template <class F, bool SWIGLU, int TH>
__device__ __forceinline__ void mfg_row(const float *__restrict__ x, const float *__restrict__ hu,
                                        int r, float clamp, _Float16 *__restrict__ xh,
                                        float *__restrict__ unscale, int in_dim) {
    const float *xt = x + (size_t)r * in_dim;
    const float *ut = hu + (SWIGLU ? (size_t)r * in_dim : 0);
    auto val4 = [&](int i) {
        float4 v = *reinterpret_cast<const float4 *>(xt + i);
        if (SWIGLU) {
            const float4 u = *reinterpret_cast<const float4 *>(ut + i);
            v = make_float4(swiglu_clamped(v.x, u.x, clamp), swiglu_clamped(v.y, u.y, clamp),
                            swiglu_clamped(v.z, u.z, clamp), swiglu_clamped(v.w, u.w, clamp));
        }
        return v;
    };
    // hi of piece p at halves 16 p, lo 8 halves later: two "columns" per
    // piece with the lo plane 8 halves after the hi one
    mf_x_column<F, TH>(val4, in_dim, 0, xh + (size_t)r * 2 * in_dim, unscale + r, 2, 8);
}

// The SwiGLU image of the down projection: one workgroup per slot.
template <class F, int TH>
__global__ __launch_bounds__(TH) void k_mfg_xs(const float *__restrict__ hg,
                                               const float *__restrict__ hu,
                                               const int *__restrict__ n_rows, float clamp,
                                               _Float16 *__restrict__ xh,
                                               float *__restrict__ unscale, int in_dim) {
    const int r = blockIdx.x;
    if (r >= *n_rows) return;
    mfg_row<F, true, TH>(hg, hu, r, clamp, xh, unscale, in_dim);
}

// The first launch of the route: workgroup 0 runs the routing (when `route`;
// moe_route1, batches into bat / *n_bat), the others write the per-token
// image of x (x rows do not depend on the routing). Without `route` (calls
// the three-launch routing serves) every workgroup writes an image row.
template <class F>
__global__ __launch_bounds__(kScanThreads) void k_mfg_route_x(MoeRoute1Args ra, MfgBatch *bat,
                                                              int *n_bat, int bw, int route,
                                                              const float *__restrict__ x,
                                                              _Float16 *__restrict__ xh,
                                                              float *__restrict__ unscale,
                                                              int in_dim) {
    extern __shared__ int sh[];  // routing: 2 n_expert ints
    __shared__ int ep[kRoute1Pairs];
    __shared__ int part[kScanThreads];
    if (route && blockIdx.x == 0) {
        moe_route1(ra.ids, ra.wts, ra.n_pairs, ra.k, ra.n_expert, ra.off, ra.slot_tok, ra.slot_of,
                   ra.act, ra.n_act, bat, n_bat, bw, sh, ep, part);
        return;
    }
    mfg_row<F, false, kScanThreads>(x, nullptr, (int)blockIdx.x - (route ? 1 : 0), 0.f, xh, unscale,
                                    in_dim);
}

// ---- grouped LoRA-down on the matrix cores ----------------------------------------
// One stacked matrix of G * R rows (device layout as one matrix); row r dots
// group g = r / R's slice x[t * x_stride + g * D .. + D). Image (g, c) holds
// tokens 16 c .. 16 c + 15 of group g's slice (kMfgBatch = 16 columns).
template <class F>
__global__ __launch_bounds__(kMfxThreads) void k_mfl_x(const float *__restrict__ x, int x_stride, int n_tok,
                                               int D, int nchunks, _Float16 *__restrict__ xh,
                                               float *__restrict__ unscale) {
    const int b = blockIdx.y, g = b / nchunks, tc = (b - g * nchunks) * kMfgBatch + blockIdx.x;
    if (tc >= n_tok) return;
    const float *xt = x + (size_t)tc * x_stride + (size_t)g * D;
    auto val4 = [&](int i) { return *reinterpret_cast<const float4 *>(xt + i); };
    mf_x_column<F>(val4, D, blockIdx.x, xh + (size_t)b * 2 * D * kMfgBatch,
                   unscale + (size_t)b * kMfgBatch + blockIdx.x, kMfgBatch);
}

// Grid (G R / 64, chunks): workgroup (x, c) computes rows 64 x .. 64 x + 63
// (one group: R is a multiple of 64) for tokens 16 c .. into y[t * y_stride + row].
template <class F>
__global__ __launch_bounds__(256) void k_gemv_mfl(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                  const _Float16 *__restrict__ xh,
                                                  const float *__restrict__ unscale,
                                                  float *__restrict__ y, int y_stride, int n_tok,
                                                  int D, int R, int out_dim, int nchunks) {
    constexpr int NK = 4, RT = 4;
    __shared__ f32x4 red[NK * RT * (kMfgBatch / 16) * 64];
    const int row0 = blockIdx.x * 16 * RT, c = blockIdx.y;
    const int b = (row0 / R) * nchunks + c;
    const int t0 = c * kMfgBatch;
    const size_t img = (size_t)D * kMfgBatch;  // values per plane
    mf_rows<F, kMfgBatch / 16, NK, RT>(w, w_bytes, xh + b * 2 * img, (uint32_t)(img * 2),
                                       unscale + (size_t)b * kMfgBatch, y + (size_t)t0 * y_stride,
                                       min(kMfgBatch, n_tok - t0), D, out_dim, y_stride, row0,
                                       red, kMfgBatch);
}

// Batch column of lane r16 (c = r16 & 7 in the packed 8-column operand,
// else r16; columns past the batch's count read its first column, whose
// results are not stored) and its image row: the slot's token (tok given,
// gate/up) or the slot (down); its byte offset in a plane and its unscale.
__device__ __forceinline__ void mfg_column(const MfgBatch &bt, const int *__restrict__ tok,
                                           const float *__restrict__ unscale, int in_dim, int c,
                                           uint32_t &xcol, float &usc) {
    const int slot = bt.first + (c < bt.count ? c : 0);
    const int row = tok ? tok[slot] : slot;
    xcol = (uint32_t)row * (uint32_t)in_dim * 4u;
    usc = unscale[row];
}

// Grid (row blocks, batch slots, matrices): workgroup (x, b, m) computes
// rows 16 RT x of W_m[expert(b)] = w_m + expert * w_stride for batch b's
// slots into y_m, against the per-row image xh (planes of plane_bytes).
// Batch slots past *n_bat exit at once.
template <class F, int NK, int RT>
__global__ __launch_bounds__(64 * NK) void k_gemv_mfg(const uint8_t *__restrict__ w0,
                                                      const uint8_t *__restrict__ w1,
                                                      size_t w_stride,
                                                      const _Float16 *__restrict__ xh,
                                                      uint32_t plane_bytes,
                                                      const float *__restrict__ unscale,
                                                      const int *__restrict__ tok,
                                                      const MfgBatch *__restrict__ bat,
                                                      const int *__restrict__ n_bat,
                                                      float *__restrict__ y0, float *__restrict__ y1,
                                                      int in_dim, int out_dim) {
    __shared__ f32x4 red[NK * RT * 64];
    const int b = blockIdx.y;
    if (b >= *n_bat) return;
    const MfgBatch bt = bat[b];
    const bool m1 = blockIdx.z != 0;
    const uint8_t *w = (m1 ? w1 : w0) + (size_t)bt.expert * w_stride;
    float *y = (m1 ? y1 : y0) + (size_t)bt.first * out_dim;
    uint32_t xcol;
    float usc;
    mfg_column(bt, tok, unscale, in_dim, threadIdx.x & 15, xcol, usc);
    mf_rows<F, 1, NK, RT, true>(w, (uint32_t)w_stride, xh, plane_bytes, nullptr, y, bt.count,
                                in_dim, out_dim, out_dim, blockIdx.x * 16 * RT, red, 16, xcol, usc);
}

// The grouped GEMV with its weights staged through LDS (mfs_rows): grid
// (ROWS-row blocks, batch slots, matrices); workgroup (x, b, m) computes
// rows ROWS x of W_m[expert(b)] for batch b's slots into y_m, against the
// per-row image xh (planes of plane_bytes). Batch slots past *n_bat exit at
// once. PACK: 8-slot batches on the packed kernel (8 wavefronts); else
// 16-slot batches (4 wavefronts).
template <class F, bool PACK, int ROWS>
__global__ __launch_bounds__(PACK ? 64 * kMfsPackWaves : 256) void k_gemv_mfgs(const uint8_t *__restrict__ w0,
                                                   const uint8_t *__restrict__ w1,
                                                   size_t w_stride,
                                                   const _Float16 *__restrict__ xh,
                                                   uint32_t plane_bytes,
                                                   const float *__restrict__ unscale,
                                                   const int *__restrict__ tok,
                                                   const MfgBatch *__restrict__ bat,
                                                   const int *__restrict__ n_bat,
                                                   float *__restrict__ y0, float *__restrict__ y1,
                                                   int in_dim, int out_dim) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int b = blockIdx.y;
    if (b >= *n_bat) return;
    const MfgBatch bt = bat[b];
    const bool m1 = blockIdx.z != 0;
    const uint8_t *w = (m1 ? w1 : w0) + (size_t)bt.expert * w_stride;
    float *y = (m1 ? y1 : y0) + (size_t)bt.first * out_dim;
    constexpr int bw = PACK ? 8 : kMfgBatch;
    uint32_t xcol;
    float usc;
    mfg_column(bt, tok, unscale, in_dim, threadIdx.x & (bw - 1), xcol, usc);
    mfs_rows<F, 1, PACK, PACK ? kMfsPackWaves : 4, ROWS, true>(
        w, xh, plane_bytes, nullptr, y, out_dim, bt.count, in_dim, out_dim,
        (int)blockIdx.x * ROWS, 0, in_dim / kMfsK, bw, smem, xcol, usc);
}

// ---- fused batched GEMV: activations converted into LDS ------------------------------
// One launch of n_wg workgroups (one per CU) of NW wavefronts, for n_tok <=
// 16 tokens whose two f16 activation planes fit in LDS (n_tok * in_dim * 4
// bytes).
//
// Prologue: per-token max |x| (LDS atomic max on the float bits, all values
// being non-negative), then every 8-element piece of x scaled by 2^e_t into
// f16 (hi and lo planes) at LDS slot ((s * 4 + j) * 4 + q) * n_tok + t of
// each plane (MFMA operand order);
// unscale[t] = 2^-e_t. Lanes of tokens >= n_tok read a zero slot.
// Rows: blocks of 16 (the MFMA M); workgroup b owns blocks b + n_wg * l.
// Every wavefront streams its share of K steps [w ns / NW, (w + 1) ns / NW)
// of each of those blocks, PD steps in flight; after a block its partial D
// goes to LDS, and after the stream the workgroup adds the NW partials in
// wavefront order (deterministic), scales by 2^-e_t and stores.
template <class F, int NW, int PD, int XP>
__global__ __launch_bounds__(64 * NW) void k_gemv_mfb(const uint8_t *__restrict__ w,
                                                      uint32_t w_bytes,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, int n_tok,
                                                      int in_dim, int out_dim, int n_wg) {
    extern __shared__ uint4 lds[];
    __shared__ uint32_t amax_bits[16];
    __shared__ float unscale[16];
    constexpr int kThreads = 64 * NW;
    const int lane = threadIdx.x & 63, r16 = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ns = in_dim / kMfStep;
    const int n_rb = (out_dim + 15) >> 4;
    const int rb0 = blockIdx.x;
    const int nrb = (n_rb - rb0 + n_wg - 1) / n_wg;  // this workgroup's row blocks
    const int s_beg = ns * wv / NW, s_end = ns * (wv + 1) / NW, my_ns = s_end - s_beg;
    const int T = nrb * my_ns;  // this wavefront's tiles (block-major)
    const size_t n8s = (size_t)n_tok * in_dim / 8;
    uint4 *xs = lds;                                              // hi plane: n8s slots
    uint4 *xls = lds + n8s;                                       // lo plane: n8s slots
    uint4 *zero = lds + 2 * n8s;                                  // one zero slot
    f32x4 *part = reinterpret_cast<f32x4 *>(zero + 1);            // [nrb][NW][64]
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(w, 0);

    typename F::W buf[PD];
    auto load_tile = [&](typename F::W &wt, int t) {
        const int l = my_ns > 0 ? t / my_ns : 0;
        const int s = s_beg + (t - l * my_ns);
        const int row = min(16 * (rb0 + n_wg * l) + r16, out_dim - 1);
        F::load(wt, t < T ? rw : rnull, row, min(s, ns - 1), q, in_dim, out_dim);
    };

    // Prologue. x is read once: XP 8-element pieces per thread (piece i =
    // thread + k * 64 NW, token 8 i / in_dim), issued before the first
    // tiles' weight loads; per-token max |x| by LDS atomic max on the float
    // bits (non-negative values order like their bits); then the pieces are
    // scaled, converted and stored.
    const int n8 = n_tok * in_dim / 8;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)n8 * 32u);
    uint4 xv[XP][2];
#pragma unroll
    for (int r = 0; r < XP; r++) {
        const uint32_t i = threadIdx.x + r * kThreads;
        xv[r][0] = bload16(rx, i * 32u, 0);
        xv[r][1] = bload16(rx, i * 32u + 16u, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PD - 1; j++) load_tile(buf[j], j);
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < 16) amax_bits[threadIdx.x] = 0u;
    if (threadIdx.x == 0) *zero = make_uint4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < XP; r++) {
        const int i = threadIdx.x + r * kThreads;
        float m = 0.f;  // pieces past the end read zeros
#pragma unroll
        for (int h = 0; h < 2; h++) {
            m = fmaxf(m, fmaxf(fmaxf(fabsf(__uint_as_float(xv[r][h].x)), fabsf(__uint_as_float(xv[r][h].y))),
                               fmaxf(fabsf(__uint_as_float(xv[r][h].z)), fabsf(__uint_as_float(xv[r][h].w)))));
        }
        // a wavefront's 64 pieces span at most two tokens (in_dim >= 512):
        // reduce per token over the wavefront, then one atomic per token
        const int tl = min((8 * (i - lane)) / in_dim, n_tok - 1);
        const int tt = min((8 * i) / in_dim, n_tok - 1);
        const float m_lo = wave_max(tt == tl ? m : 0.f), m_hi = wave_max(tt != tl ? m : 0.f);
        if (lane == 0 && i - lane < n8) {
            atomicMax(&amax_bits[tl], __float_as_uint(m_lo));
            if (tl + 1 < n_tok) atomicMax(&amax_bits[tl + 1], __float_as_uint(m_hi));
        }
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const float amax = __uint_as_float(amax_bits[threadIdx.x]);
        int e = 0;
        if (amax > 0.f && amax <= 3.4e38f) {
            int ex;
            frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
            e = min(max(15 - ex, -126), 126);
        }
        amax_bits[threadIdx.x] = (uint32_t)e;
        unscale[threadIdx.x] = ldexpf(1.0f, -e);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < XP; r++) {
        const int i = threadIdx.x + r * kThreads;
        if (i < n8) {
            const int t = (8 * i) / in_dim, e0 = 8 * i - t * in_dim;
            const float up = ldexpf(1.0f, (int)amax_bits[t]);
            uint4 hi, lo;
            hilo8(__builtin_bit_cast(float4, xv[r][0]), __builtin_bit_cast(float4, xv[r][1]), up,
                  hi, lo);
            int s, j, qq;
            F::piece(e0, s, j, qq);
            xs[((s * 4 + j) * 4 + qq) * n_tok + t] = hi;
            xls[((s * 4 + j) * 4 + qq) * n_tok + t] = lo;
        }
    }
    __syncthreads();

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int l = 0, sc = 0;  // compute cursor: block l, step s_beg + sc
    const bool tok_ok = r16 < n_tok;
    for (int t0 = 0; t0 < T; t0 += PD) {
#pragma unroll
        for (int jj = 0; jj < PD; jj++) {
            const int t = t0 + jj;
            load_tile(buf[(jj + PD - 1) % PD], t + PD - 1);
            __builtin_amdgcn_sched_barrier(0);
            if (t < T) {
                const int s = s_beg + sc;
                uint4 xr[4][1], lr[4][1];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const size_t o = ((size_t)(s * 4 + j) * 4 + q) * n_tok + r16;
                    xr[j][0] = *(tok_ok ? xs + o : zero);
                    lr[j][0] = *(tok_ok ? xls + o : zero);
                }
                f32x4 a1[1] = {acc};
                F::template step<1>(buf[jj], q, xr, lr, a1);
                acc = a1[0];
                if (++sc == my_ns) {
                    part[((size_t)l * NW + wv) * 64 + lane] = acc;
                    acc = {0.f, 0.f, 0.f, 0.f};
                    sc = 0;
                    l++;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (my_ns == 0)  // more wavefronts than K steps: this one contributes zeros
        for (int b = 0; b < nrb; b++) part[((size_t)b * NW + wv) * 64 + lane] = acc;
    __syncthreads();
    // D lane layout: tokens 4 (lane / 16) + 0..3 of weight row lane % 16
    for (int c = threadIdx.x; c < nrb * 64; c += kThreads) {
        const int b = c >> 6, ln = c & 63;
        f32x4 v = part[((size_t)b * NW) * 64 + ln];
        for (int k = 1; k < NW; k++) v += part[((size_t)b * NW + k) * 64 + ln];
        const int o = 16 * (rb0 + n_wg * b) + (ln & 15);
        const int t0 = 4 * (ln >> 4);
        if (o < out_dim) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (t0 + i < n_tok) y[(size_t)(t0 + i) * out_dim + o] = v[i] * unscale[t0 + i];
        }
    }
}

template <class F>
static size_t mfb_lds_bytes(int n_tok, int in_dim, int out_dim, int n_wg, int nw) {
    const int n_rb = (out_dim + 15) >> 4;
    const int nrb = (n_rb + n_wg - 1) / n_wg;
    return (2 * (size_t)n_tok * in_dim / 8 + 1) * 16 + (size_t)nrb * nw * 64 * 16;
}
constexpr size_t kMfbMaxLds = 152 * 1024;

template <class F, int NW, int PD, int XP>
static hipError_t mfb_go(const uint8_t *w, size_t w_bytes, const float *x, float *y, int n_tok,
                         int in_dim, int out_dim, int n_wg, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)k_gemv_mfb<F, NW, PD, XP>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMfbMaxLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    n_wg = min(n_wg, (out_dim + 15) >> 4);
    k_gemv_mfb<F, NW, PD, XP><<<(unsigned)n_wg, 64 * NW, mfb_lds_bytes<F>(n_tok, in_dim, out_dim, n_wg, NW), s>>>(
        w, (uint32_t)w_bytes, x, y, n_tok, in_dim, out_dim, n_wg);
    return hipGetLastError();
}

// Pieces of x per thread (1, 2, 4 or 8; 0 = too many).
static int mfb_xp(int n_tok, int in_dim, int nw) {
    const int n8 = n_tok * in_dim / 8, thr = 64 * nw;
    const int xp = (n8 + thr - 1) / thr;
    return xp <= 1 ? 1 : xp <= 2 ? 2 : xp <= 4 ? 4 : xp <= 8 ? 8 : 0;
}

template <class F, int NW, int PD>
static hipError_t mfb_xp_go(const uint8_t *w, size_t w_bytes, const float *x, float *y, int n_tok,
                            int in_dim, int out_dim, int n_wg, hipStream_t s) {
    switch (mfb_xp(n_tok, in_dim, NW)) {
    case 1: return mfb_go<F, NW, PD, 1>(w, w_bytes, x, y, n_tok, in_dim, out_dim, n_wg, s);
    case 2: return mfb_go<F, NW, PD, 2>(w, w_bytes, x, y, n_tok, in_dim, out_dim, n_wg, s);
    case 4: return mfb_go<F, NW, PD, 4>(w, w_bytes, x, y, n_tok, in_dim, out_dim, n_wg, s);
    case 8: return mfb_go<F, NW, PD, 8>(w, w_bytes, x, y, n_tok, in_dim, out_dim, n_wg, s);
    default: return hipErrorInvalidValue;
    }
}

// ---- launchers -----------------------------------------------------------------------
// Taken from 5 tokens up: below that the int8-limb GEMV, whose VALU work
// grows with the batch, is still faster (C1: 26 vs 29 us at 4 tokens, 55 vs
// 29 us at 8). The weights are exact, so any number of rows qualifies.
bool gemv_mfma_supported(uint32_t dtype, int n_tok, int in_dim, int out_dim) {
    // Q8_0 below 8192 rows and 8192 columns from 9 tokens: up to 8 the
    // int8-limb kernel with x in LDS is as fast on 4096 x 4096 and faster on
    // 1024-row matrices. Taller ones gain from 5 (14336 x 4096: 28 -> 19 us
    // at 5 and 8 tokens), wider ones from 3 (4096 x 14336: 30 -> 23 us at 3
    // and 4 tokens, 76 -> 24 us at 8)
    const int min_tok =
        dtype != T_Q8_0 ? 5 : in_dim >= 8192 ? 3 : out_dim >= 8192 ? 5 : 9;
    return (dtype == T_Q4_K || dtype == T_Q6_K || dtype == T_Q8_0 || dtype == T_Q2_K ||
            dtype == T_IQ2_XXS) &&
           n_tok >= min_tok && n_tok <= 32 && in_dim % 256 == 0 && in_dim > 0 && out_dim > 0;
}

// K splits of the staged GEMV (k_gemv_mfs): the largest power of two up to
// 8 (and up to the number of chunks) that keeps 32-row workgroups x splits
// within 512, two per CU on 256 CUs (C1 4096 x 14336 Q6_K at 8 tokens: 4
// splits, 26.8 vs 36.2 us for the mf_rows kernel); 0 where the staged
// kernel does not apply (in_dim not a multiple of 1024, or of 2048 for Q6_K,
// whose super-tiles must not straddle rows).
template <class F> static int mfs_splits(int in_dim, int out_dim) {
    if (!kMfsStaged<F> || in_dim <= 0 || out_dim <= 0 || in_dim % kMfsK != 0) return 0;
    if ((std::is_same<F, MQ6K>::value || std::is_same<F, MQ2K>::value ||
         std::is_same<F, MIQ2>::value) &&
        in_dim % 2048 != 0)
        return 0;
    const int nch = in_dim / kMfsK;
    const long blocks = (out_dim + kMfsRows - 1) / kMfsRows;
    int sk = 1;
    while (sk < 8 && 2 * sk <= nch && blocks * 2 * sk <= 512) sk *= 2;
    return sk;
}
// The staged kernel's K splits for a dense call of n_tok tokens, or 0 where
// the call takes another kernel: IQ2_XXS takes it above 16 tokens only,
// Q2_K never (unstaged against staged: IQ2_XXS 2048 x 4096 at 8 tokens 10.5
// vs 12.0 us, at 32 13.2 vs 11.9 us, 14336 x 4096 at T = 512 in 32-token
// chunks 398 vs 342 us; Q2_K 7168 x 2048 at 8 tokens 9.9 vs 11.8 us,
// 4096 x 2048 at 32 9.4 vs 11.3 us, at T = 512 143 vs 176 us).
template <class F> static int mfs_dense_splits(int n_tok, int in_dim, int out_dim) {
    if (std::is_same<F, MQ2K>::value || (std::is_same<F, MIQ2>::value && n_tok <= 16)) return 0;
    return mfs_splits<F>(in_dim, out_dim);
}
// (the workspace sizing: every format the staged kernel takes must be here)
static int mfs_splits_for(uint32_t dtype, int n_tok, int in_dim, int out_dim) {
    switch (dtype) {
    case T_Q4_K: return mfs_dense_splits<MQ4K>(n_tok, in_dim, out_dim);
    case T_Q6_K: return mfs_dense_splits<MQ6K>(n_tok, in_dim, out_dim);
    case T_Q8_0: return mfs_dense_splits<MQ8>(n_tok, in_dim, out_dim);
    case T_Q2_K: return mfs_dense_splits<MQ2K>(n_tok, in_dim, out_dim);
    case T_IQ2_XXS: return mfs_dense_splits<MIQ2>(n_tok, in_dim, out_dim);
    default: return 0;
    }
}

// The one-pass kernel's rows per workgroup and slice length for this shape,
// or rows = 0: the first of (128, 512), (64, 512), (128, 256), (64, 256)
// that divides K and gives 192..512 workgroups (one or two rounds of one per
// CU). Q8_0 and Q4_K, whose rows' slices are contiguous byte runs; 9..32
// tokens.
template <class F>
static void mfo_choose(int n_tok, int in_dim, int out_dim, int &rows, int &ks) {
    rows = ks = 0;
    if constexpr (std::is_same<F, MQ8>::value || std::is_same<F, MQ4K>::value) {
        if (n_tok < 9 || n_tok > 32 || in_dim <= 0 || out_dim <= 0 || in_dim % 256 != 0) return;
        const size_t row_bytes = (size_t)(in_dim / 256) * MfoRow<F>::kB256;
        if ((size_t)out_dim * row_bytes > 0xFFFFFFF0u ||
            (size_t)n_tok * (size_t)in_dim * 4 > 0x7FFFFFFFu)
            return;
        const int cand[4][2] = {{128, 512}, {64, 512}, {128, 256}, {64, 256}};
        for (const auto &c : cand) {
            if (in_dim % c[1] != 0) continue;
            const long n_wg = (long)((out_dim + c[0] - 1) / c[0]) * (in_dim / c[1]);
            if (n_wg >= 192 && n_wg <= 512) {
                rows = c[0];
                ks = c[1];
                return;
            }
        }
    }
}
static void mfo_choose_dt(uint32_t dtype, int n_tok, int in_dim, int out_dim, int &rows, int &ks) {
    rows = ks = 0;
    if (dtype == T_Q8_0) mfo_choose<MQ8>(n_tok, in_dim, out_dim, rows, ks);
    if (dtype == T_Q4_K) mfo_choose<MQ4K>(n_tok, in_dim, out_dim, rows, ks);
}

template <class F, int NT, int NW, int KS, int RTW>
static hipError_t mfo_launch(const uint8_t *w, const float *x, float *part, float *y, int n_tok,
                             int in_dim, int out_dim, hipStream_t s) {
    using G = MfoGeo<F, NT, NW, KS, RTW>;
    static_assert(G::LDS + 16 * NT * 4 <= 160 * 1024, "one workgroup's LDS");
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_mfo<F, NT, NW, KS, RTW>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (attr != hipSuccess) return attr;
    const int sk = in_dim / KS;
    const dim3 grid((unsigned)sk, (unsigned)((out_dim + G::R - 1) / G::R));
    k_gemv_mfo<F, NT, NW, KS, RTW><<<grid, G::TH, G::LDS, s>>>(w, x, sk > 1 ? part : y, n_tok,
                                                               in_dim, out_dim);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || sk == 1) return e;
    const int n = n_tok * out_dim;
    k_mfs_sum<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(part, y, n, sk);
    return hipGetLastError();
}

// Wavefronts x row tiles per wavefront of the one-pass kernel for R rows.
constexpr int kMfoNW128 = 8, kMfoRTW128 = 1, kMfoNW64 = 4, kMfoRTW64 = 1;

template <class F>
static hipError_t mfo_go(const uint8_t *w, const float *x, uint8_t *scratch, float *y, int n_tok,
                         int in_dim, int out_dim, int rows, int ks, hipStream_t s) {
    if constexpr (std::is_same<F, MQ8>::value || std::is_same<F, MQ4K>::value) {
        float *part = reinterpret_cast<float *>(scratch);
        const int nt = n_tok > 16 ? 2 : 1;
#define MFO(NT, R, KS, NW, RTW)                                                                  \
    if (nt == NT && rows == R && ks == KS)                                                       \
        return mfo_launch<F, NT, NW, KS, RTW>(w, x, part, y, n_tok, in_dim, out_dim, s);
#define MFO_ALL(NT)                                                                              \
    MFO(NT, 128, 512, kMfoNW128, kMfoRTW128) MFO(NT, 64, 512, kMfoNW64, kMfoRTW64)              \
    MFO(NT, 128, 256, kMfoNW128, kMfoRTW128) MFO(NT, 64, 256, kMfoNW64, kMfoRTW64)
        MFO_ALL(1) MFO_ALL(2)
#undef MFO_ALL
#undef MFO
    }
    return hipErrorInvalidValue;
}

// Two f16 planes of ntp x in_dim, ntp unscale factors, and the staged
// kernel's partial outputs when it splits K; or the one-pass kernel's
// partials, whichever is larger.
size_t gemv_mfma_scratch_bytes(uint32_t dtype, int n_tok, int in_dim, int out_dim) {
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    const size_t ntp = n_tok <= 16 ? 16 : 32;
    const int sk = mfs_splits_for(dtype, n_tok, in_dim, out_dim);
    const size_t part = sk > 1 ? (size_t)sk * (size_t)n_tok * (size_t)out_dim * 4 : 0;
    const size_t staged = al(2 * ntp * (size_t)in_dim * 2) + al(ntp * 4) + part;
    // the one-pass kernel: only its slices' partial outputs
    int rows, ks;
    mfo_choose_dt(dtype, n_tok, in_dim, out_dim, rows, ks);
    const size_t one = rows ? al((size_t)(in_dim / ks) * (size_t)n_tok * (size_t)out_dim * 4) : 0;
    return one > staged ? one : staged;
}

template <class F>
static hipError_t mfs_go(const uint8_t *w, const float *x, uint8_t *scratch, float *y, int n_tok,
                         int in_dim, int out_dim, int sk, hipStream_t s) {
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    // 8 image columns up to 8 tokens: half the activation bytes every
    // workgroup reads (C1 14336 x 4096 Q6_K at 8 tokens reads the image 448
    // times)
    const int ntp = n_tok <= 8 ? 8 : n_tok <= 16 ? 16 : 32;
    const size_t plane_bytes = (size_t)ntp * in_dim * 2;
    _Float16 *xh = reinterpret_cast<_Float16 *>(scratch);
    float *unscale = reinterpret_cast<float *>(scratch + al(2 * plane_bytes));
    float *part = reinterpret_cast<float *>(scratch + al(2 * plane_bytes) + al((size_t)ntp * 4));
    constexpr int lds = MfsGeo<F>::LDS;
    constexpr int lds8 = MfsGeo<F, kMfsPackWaves>::LDS;
    // the attribute once per kernel (thread-safe static initialisation)
    static const hipError_t attr1 = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemv_mfs<F, 1>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    static const hipError_t attr2 = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemv_mfs<F, 2>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    static const hipError_t attr3 = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemv_mfs<F, 1, true, kMfsPackWaves>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds8);
    if (attr1 != hipSuccess) return attr1;
    if (attr2 != hipSuccess) return attr2;
    if (attr3 != hipSuccess) return attr3;
    k_mf_x<F><<<(unsigned)ntp, kMfxThreads, 0, s>>>(x, xh, unscale, n_tok, in_dim, ntp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)sk, (unsigned)((out_dim + kMfsRows - 1) / kMfsRows));
    float *dst = sk > 1 ? part : y;
    if (ntp == 8)
        k_gemv_mfs<F, 1, true, kMfsPackWaves><<<grid, 64 * kMfsPackWaves, lds8, s>>>(
            w, xh, (uint32_t)plane_bytes, unscale, dst, n_tok, in_dim, out_dim, ntp);
    else if (ntp == 16)
        k_gemv_mfs<F, 1><<<grid, 256, lds, s>>>(w, xh, (uint32_t)plane_bytes, unscale, dst, n_tok,
                                                in_dim, out_dim, ntp);
    else
        k_gemv_mfs<F, 2><<<grid, 256, lds, s>>>(w, xh, (uint32_t)plane_bytes, unscale, dst, n_tok,
                                                in_dim, out_dim, ntp);
    e = hipGetLastError();
    if (e != hipSuccess || sk == 1) return e;
    const int n = n_tok * out_dim;
    k_mfs_sum<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(part, y, n, sk);
    return hipGetLastError();
}

template <class F, int NT, int NK, int RT>
static hipError_t mf_go(const uint8_t *w, size_t w_bytes, const float *x, uint8_t *scratch, float *y,
                        int n_tok, int in_dim, int out_dim, hipStream_t s) {
    constexpr int ntp = NT * 16;
    const size_t plane_bytes = (size_t)ntp * in_dim * 2;
    _Float16 *xh = reinterpret_cast<_Float16 *>(scratch);
    float *unscale = reinterpret_cast<float *>(scratch + (2 * plane_bytes + 255) / 256 * 256);
    k_mf_x<F><<<ntp, kMfxThreads, 0, s>>>(x, xh, unscale, n_tok, in_dim, ntp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int rows_wg = 16 * RT;
    k_gemv_mf<F, NT, NK, RT><<<(unsigned)((out_dim + rows_wg - 1) / rows_wg), 64 * NK, 0, s>>>(
        w, (uint32_t)w_bytes, xh, (uint32_t)plane_bytes, unscale, y, n_tok, in_dim, out_dim);
    return hipGetLastError();
}

// 5..8 tokens of tall matrices (out_dim >= 8192) whose f16 activations fit
// in LDS take the fused kernel (C1 14336x4096 at 8 tokens: 24 vs 29 us); the
// rest the two-launch kernel, which is faster on short matrices and does not
// need x in LDS.
template <class F>
static hipError_t mf_dispatch(const uint8_t *w, size_t w_bytes, const float *x, uint8_t *scratch,
                              float *y, int n_tok, int in_dim, int out_dim, hipStream_t s) {
    // the staged kernel wherever it applies (16-byte aligned weights: its
    // LDS copies move 16-byte pieces); it is the faster on every measured
    // shape (C1 14336 x 4096 Q6_K at 8 tokens: 21.8 vs 30.1 us)
    if (((uintptr_t)w & 15) == 0) {
        int rows, ks;
        mfo_choose<F>(n_tok, in_dim, out_dim, rows, ks);
        if (rows) return mfo_go<F>(w, x, scratch, y, n_tok, in_dim, out_dim, rows, ks, s);
    }
    if constexpr (kMfsStaged<F>) {
        const int sk = mfs_dense_splits<F>(n_tok, in_dim, out_dim);
        if (sk > 0 && ((uintptr_t)w & 15) == 0)
            return mfs_go<F>(w, x, scratch, y, n_tok, in_dim, out_dim, sk, s);
    }
    const int cus = device_cus();
    // (not IQ2_XXS: its operand tables are staged in LDS by mf_rows)
    if constexpr (!std::is_same<F, MIQ2>::value) {
        if (n_tok <= 8 && out_dim >= 8192 && mfb_xp(n_tok, in_dim, 16) != 0 &&
            mfb_lds_bytes<F>(n_tok, in_dim, out_dim, cus, 16) <= kMfbMaxLds)
            return mfb_xp_go<F, 16, 2>(w, w_bytes, x, y, n_tok, in_dim, out_dim, cus, s);
    }
    // Every workgroup reads the whole activation image, so more rows per
    // workgroup read it fewer times; 4 row tiles (4 wavefronts over K) where
    // that still leaves 224 or more workgroups (C1 14336 x 4096 Q4_K: 20.6 vs
    // 23.7 us at 16 tokens, 23.4 vs 28.3 us at 32), one row tile over 8
    // wavefronts otherwise (4096-row matrices take 1.4-2x longer with 4).
    if (out_dim >= 224 * 64) {
        if (n_tok <= 16) return mf_go<F, 1, 4, 4>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
        return mf_go<F, 2, 4, 4>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    }
    if (n_tok <= 16) return mf_go<F, 1, 8, 1>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    return mf_go<F, 2, 8, 1>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
}

// Any pairing of Q4_K, Q6_K, Q8_0, Q2_K and IQ2_XXS experts with both
// dimensions multiples of 256 (Q2_K and IQ2_XXS, the DS-V4 expert formats,
// on mf_rows: no staged layout). The weights are exact and the activations of each of the two
// GEMVs (x, then the SwiGLU output) reach the matrix cores as hi + lo f16
// planes, so the chained error stays at fp32 level.
static bool mfma_format(uint32_t t) {
    return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0 || t == T_Q2_K || t == T_IQ2_XXS;
}
bool moe_mfma_supported(uint32_t dt_gu, uint32_t dt_d, int n_embd, int n_ff) {
    return mfma_format(dt_gu) && mfma_format(dt_d) && n_embd > 0 && n_ff > 0 &&
           n_embd % 256 == 0 && n_ff % 256 == 0;
}

size_t moe_mfma_scratch_bytes(int n_pairs, int n_expert, int n_embd, int n_ff) {
    const int bw = mfg_width(n_pairs, n_expert);
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    // the batch list, then the x image (at most n_pairs tokens) and the
    // SwiGLU image (one row per slot), two f16 planes and a scale per row
    return mfg_batch_bytes(n_pairs, n_expert, bw) + al((size_t)n_pairs * n_embd * 4) +
           al((size_t)n_pairs * 4) + al((size_t)n_pairs * n_ff * 4) + al((size_t)n_pairs * 4);
}

bool moe_mfma_fits(int n_pairs, int n_embd, int n_ff) {
    // image offsets are 32-bit: two planes of n_pairs rows
    return (size_t)n_pairs * (size_t)(n_embd > n_ff ? n_embd : n_ff) * 4 <= 0xFFFFFFFFu;
}

// The grouped GEMV of one matrix pair (w1 given: gate and up) or matrix over
// the batches, against the per-row image xh of n_rows rows.
template <class F>
static hipError_t mfg_gemv(const uint8_t *w0, const uint8_t *w1, size_t w_stride,
                           const _Float16 *xh, const float *us, int n_rows, const int *tok,
                           const MfgBatch *bat, const int *n_bat, int max_b, float *y0, float *y1,
                           int in_dim, int out_dim, int bw, hipStream_t s) {
    const uint32_t plane = (uint32_t)((size_t)n_rows * in_dim * 2);
    // weights staged through LDS where the layout allows (16-byte aligned
    // expert matrices, in_dim a multiple of 1024, of 2048 for Q6_K)
    // (Q2_K and IQ2_XXS: 8-slot batches only; with 16-slot batches the
    // unstaged kernel measured faster, 5075 vs 5443 us for DS-V4 routed
    // experts at 2048 tokens)
    constexpr bool dsv4 = std::is_same<F, MQ2K>::value || std::is_same<F, MIQ2>::value;
    if constexpr (kMfsStaged<F>) {
    if (mfs_splits<F>(in_dim, out_dim) > 0 && (!dsv4 || bw == 8) &&
        (((uintptr_t)w0 | (uintptr_t)(w1 ? w1 : w0) | (uintptr_t)w_stride) & 15) == 0) {
        if (bw == 8) {
            // Q4_K: 64-row blocks (each workgroup reads the batch's image once
            // for twice the weight bytes); two still fit a CU
            constexpr int rows = std::is_same<F, MQ4K>::value ? kMfgPackRowsQ4K : kMfsRows;
            constexpr int lds = MfsGeo<F, kMfsPackWaves, rows>::LDS;
            static const hipError_t attr =
                hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_mfgs<F, true, rows>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, lds);
            if (attr != hipSuccess) return attr;
            const dim3 g((unsigned)((out_dim + rows - 1) / rows), (unsigned)max_b, w1 ? 2u : 1u);
            k_gemv_mfgs<F, true, rows><<<g, 64 * kMfsPackWaves, lds, s>>>(
                w0, w1, w_stride, xh, plane, us, tok, bat, n_bat, y0, y1, in_dim, out_dim);
        } else {
            constexpr int lds = MfsGeo<F>::LDS;
            static const hipError_t attr =
                hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_mfgs<F, false, kMfsRows>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, lds);
            if (attr != hipSuccess) return attr;
            const dim3 g((unsigned)((out_dim + kMfsRows - 1) / kMfsRows), (unsigned)max_b,
                         w1 ? 2u : 1u);
            k_gemv_mfgs<F, false, kMfsRows><<<g, 256, lds, s>>>(
                w0, w1, w_stride, xh, plane, us, tok, bat, n_bat, y0, y1, in_dim, out_dim);
        }
        return hipGetLastError();
    }
    }
    constexpr int NK = 4, RT = 4;
    const dim3 g((unsigned)((out_dim + 16 * RT - 1) / (16 * RT)), (unsigned)max_b, w1 ? 2u : 1u);
    k_gemv_mfg<F, NK, RT><<<g, 64 * NK, 0, s>>>(w0, w1, w_stride, xh, plane, us, tok, bat, n_bat,
                                                y0, y1, in_dim, out_dim);
    return hipGetLastError();
}

// The SwiGLU image of the down projection, one workgroup per slot (n_alloc
// rows allocated, *n_rows routed).
template <class F>
static hipError_t mfg_swiglu_image(const float *hg, const float *hu, const int *n_rows,
                                   int n_alloc, float clamp, _Float16 *xh, float *us, int in_dim,
                                   hipStream_t s) {
    // 256 threads for rows of up to 2048 elements (one 8-element piece per
    // thread), 512 up to 8192, else kMfxThreads
    const dim3 g((unsigned)n_alloc);
    if (in_dim <= 2048)
        k_mfg_xs<F, 256><<<g, 256, 0, s>>>(hg, hu, n_rows, clamp, xh, us, in_dim);
    else if (in_dim <= 8192)
        k_mfg_xs<F, 512><<<g, 512, 0, s>>>(hg, hu, n_rows, clamp, xh, us, in_dim);
    else
        k_mfg_xs<F, kMfxThreads><<<g, kMfxThreads, 0, s>>>(hg, hu, n_rows, clamp, xh, us, in_dim);
    return hipGetLastError();
}

#define MFG_DT(dt, call)                            \
    switch (dt) {                                   \
    case T_Q4_K: { using F = MQ4K; return call; }   \
    case T_Q6_K: { using F = MQ6K; return call; }   \
    case T_Q8_0: { using F = MQ8; return call; }    \
    case T_Q2_K: { using F = MQ2K; return call; }   \
    case T_IQ2_XXS: { using F = MIQ2; return call; } \
    default: return hipErrorInvalidValue;           \
    }

static hipError_t mfg_gemv_dt(uint32_t dt, const uint8_t *w0, const uint8_t *w1, size_t w_stride,
                              const _Float16 *xh, const float *us, int n_rows, const int *tok,
                              const MfgBatch *bat, const int *n_bat, int max_b, float *y0,
                              float *y1, int in_dim, int out_dim, int bw, hipStream_t s) {
    MFG_DT(dt, mfg_gemv<F>(w0, w1, w_stride, xh, us, n_rows, tok, bat, n_bat, max_b, y0, y1,
                           in_dim, out_dim, bw, s))
}

static hipError_t mfg_swiglu_image_dt(uint32_t dt, const float *hg, const float *hu,
                                      const int *n_rows, int n_alloc, float clamp, _Float16 *xh,
                                      float *us, int in_dim, hipStream_t s) {
    MFG_DT(dt, mfg_swiglu_image<F>(hg, hu, n_rows, n_alloc, clamp, xh, us, in_dim, s))
}

static hipError_t mfg_route_x_dt(uint32_t dt, const MoeRoute1Args *ra, MfgBatch *bat, int *n_bat,
                                 int bw, const float *x, int n_tok, _Float16 *xh, float *us,
                                 int in_dim, hipStream_t s) {
    const MoeRoute1Args none{};
    const unsigned grid = (unsigned)n_tok + (ra ? 1u : 0u);
    const size_t lds = ra ? (size_t)ra->n_expert * 8 : 0;
    MFG_DT(dt, (k_mfg_route_x<F><<<grid, kScanThreads, lds, s>>>(ra ? *ra : none, bat, n_bat, bw,
                                                                 ra ? 1 : 0, x, xh, us, in_dim),
                hipGetLastError()))
}
#undef MFG_DT

hipError_t launch_moe_mfma(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                           const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                           int n_tok, const MoeRoute1Args *route, const int *off,
                           const int *slot_tok, MfgBatch *bat, int *n_bat, int n_pairs,
                           int n_expert, float *hg, float *hu, float *yd, uint8_t *scratch,
                           int n_embd, int n_ff, float clamp, hipStream_t s) {
    if (!moe_mfma_supported(dt_gu, dt_d, n_embd, n_ff) || !moe_mfma_fits(n_pairs, n_embd, n_ff))
        return hipErrorInvalidValue;
    if (gu_stride > 0xFFFFFFFFu || d_stride > 0xFFFFFFFFu || n_tok > n_pairs)
        return hipErrorInvalidValue;
    if (route && (route->n_pairs > kRoute1Pairs || route->n_expert > kRoute1Experts))
        return hipErrorInvalidValue;
    const int bw = mfg_width(n_pairs, n_expert);  // as the routing that listed the batches
    const int max_b = mfg_max_batches(n_pairs, n_expert, bw);
    uint8_t *p = scratch + mfg_batch_bytes(n_pairs, n_expert, bw);
    auto take = [&](size_t n) {
        uint8_t *r = p;
        p += (n + 255) / 256 * 256;
        return r;
    };
    _Float16 *xh1 = reinterpret_cast<_Float16 *>(take((size_t)n_pairs * n_embd * 4));
    float *us1 = reinterpret_cast<float *>(take((size_t)n_pairs * 4));
    _Float16 *xh2 = reinterpret_cast<_Float16 *>(take((size_t)n_pairs * n_ff * 4));
    float *us2 = reinterpret_cast<float *>(take((size_t)n_pairs * 4));
    hipError_t e;
    // routing (when given) and the x image in one launch
    if ((e = mfg_route_x_dt(dt_gu, route, bat, n_bat, bw, x, n_tok, xh1, us1, n_embd, s)) !=
        hipSuccess)
        return e;
    if ((e = mfg_gemv_dt(dt_gu, gate, up, gu_stride, xh1, us1, n_tok, slot_tok, bat, n_bat, max_b,
                         hg, hu, n_embd, n_ff, bw, s)) != hipSuccess)
        return e;
    // off[n_expert]: the routed slot count
    if ((e = mfg_swiglu_image_dt(dt_d, hg, hu, off + n_expert, n_pairs, clamp, xh2, us2, n_ff,
                                 s)) != hipSuccess)
        return e;
    return mfg_gemv_dt(dt_d, down, nullptr, d_stride, xh2, us2, n_pairs, nullptr, bat, n_bat,
                       max_b, yd, nullptr, n_ff, n_embd, bw, s);
}

bool lora_mfma_supported(uint32_t dtype, int n_tok, int D, int G, int R) {
    return (dtype == T_Q4_K || dtype == T_Q6_K || dtype == T_Q8_0) && n_tok >= 9 && D > 0 &&
           D % 256 == 0 && R > 0 && R % 64 == 0 && (long long)G * R >= 1024;
}

size_t lora_mfma_scratch_bytes(int n_tok, int D, int G) {
    const size_t nb = (size_t)G * ((n_tok + kMfgBatch - 1) / kMfgBatch);
    return (nb * kMfgBatch * (size_t)D * 4 + 255) / 256 * 256 + nb * kMfgBatch * 4;
}

template <class F>
static hipError_t mfl_go(const uint8_t *w, size_t w_bytes, const float *x, int x_stride, float *y,
                         int y_stride, uint8_t *scratch, int n_tok, int D, int G, int R,
                         hipStream_t s) {
    const int nchunks = (n_tok + kMfgBatch - 1) / kMfgBatch;
    const size_t nb = (size_t)G * nchunks;
    _Float16 *xh = reinterpret_cast<_Float16 *>(scratch);
    float *us = reinterpret_cast<float *>(scratch + (nb * kMfgBatch * (size_t)D * 4 + 255) / 256 * 256);
    k_mfl_x<F><<<dim3(kMfgBatch, (unsigned)nb), kMfxThreads, 0, s>>>(x, x_stride, n_tok, D, nchunks, xh, us);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int out_dim = G * R;
    k_gemv_mfl<F><<<dim3((unsigned)(out_dim / 64), (unsigned)nchunks), 256, 0, s>>>(
        w, (uint32_t)w_bytes, xh, us, y, y_stride, n_tok, D, R, out_dim, nchunks);
    return hipGetLastError();
}

hipError_t launch_lora_mfma(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            int x_stride, float *y, int y_stride, uint8_t *scratch, int n_tok,
                            int D, int G, int R, hipStream_t s) {
    if (!lora_mfma_supported(dtype, n_tok, D, G, R) || w_bytes > 0xFFFFFFFFu ||
        (size_t)G * ((n_tok + kMfgBatch - 1) / kMfgBatch) > 65535)
        return hipErrorNotSupported;
    switch (dtype) {
    case T_Q4_K: return mfl_go<MQ4K>(w, w_bytes, x, x_stride, y, y_stride, scratch, n_tok, D, G, R, s);
    case T_Q6_K: return mfl_go<MQ6K>(w, w_bytes, x, x_stride, y, y_stride, scratch, n_tok, D, G, R, s);
    case T_Q8_0: return mfl_go<MQ8>(w, w_bytes, x, x_stride, y, y_stride, scratch, n_tok, D, G, R, s);
    default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemv_mfma(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            uint8_t *scratch, float *y, int n_tok, int in_dim, int out_dim,
                            hipStream_t s) {
    switch (dtype) {
    case T_Q4_K: return mf_dispatch<MQ4K>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    case T_Q6_K: return mf_dispatch<MQ6K>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    case T_Q8_0: return mf_dispatch<MQ8>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    case T_Q2_K: return mf_dispatch<MQ2K>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    case T_IQ2_XXS: return mf_dispatch<MIQ2>(w, w_bytes, x, scratch, y, n_tok, in_dim, out_dim, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rsllm_hip
