/*
 * rsllm_oracle.c — CPU restatement of rsLLM's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity oracle for the HIP kernels and the
 * timed CPU baseline ("port"). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it.
 *
 * Build: oracle/build.sh (gcc -O3 -ffp-contract=off, no -ffast-math, no
 * -march flags). The reference is Rust; rustc never contracts a*b+c into an
 * FMA and never reassociates float sums, and its default x86-64 target has
 * no FMA, so -ffp-contract=off reproduces its evaluation order exactly.
 *
 * Arithmetic is written in the reference's order, operation by operation;
 * each function cites the reference lines it restates (paths relative to
 * the rsLLM tree: crates/<crate>/src/...).
 *
 * Pinning (how each function is checked, in tests/test_oracle_*.py):
 *   orc_f16_to_f32        all 65,536 bit patterns vs numpy float16 widening
 *   orc_q4k_scale_min     brute force over all 2^12 (sc, m) pairs through
 *                         the reference's inverse packer (q4_k.rs:100-124)
 *   orc_dequant_q4_k/q6_k/q8_0/q4_0/q4_1/q5_k/q8_k
 *                         the reference's known-answer tests (q4_k.rs:167-250,
 *                         q6_k.rs:163-264, q8_0.rs:82-170, q4_0.rs:184-213,
 *                         q5_k.rs:166-228, q8_k.rs:94-163, mod.rs:164-304),
 *                         closed forms d*sc*q - dmin*m, and an independent
 *                         numpy restatement over every block of seeded data
 *   orc_matmul_quant_f32  dequant-then-dot against float64 numpy (error
 *                         bound), the reference's Q4_0 tolerance test
 *                         (quant_matmul.rs:189-248), bit-identical results
 *                         for every thread count, error order of :57-92
 *   orc_*q8_0* int8 path  the reference's KATs (q8_0.rs:323-553), exact
 *                         integer dots vs numpy int64, rint ties-to-even
 *   orc_moe_routed        w == 0 skip, clamp KATs (moe.rs:791-833 semantics),
 *                         linearity in the routing weights, float64 recompute
 *   orc_matmul_weight_f32 / orc_matmul_grouped_lora_down
 *                         the reference's tests (weight.rs:329-463: hand
 *                         dot, group isolation, slice alignment and offsets,
 *                         out-shape rejection), float64 recompute of the F32
 *                         arm, the grouped form equal to per-group
 *                         orc_matmul_quant_f32 on the slices
 *   orc_apply_shared_expert
 *                         the reference's clamp test (moe.rs:743-789:
 *                         identity F32 weights, x[0] = 1e3 gives silu(10) *
 *                         10), equality with orc_moe_routed on one expert
 *                         of weight 1, float64 recompute of the F32 form
 */
#define _GNU_SOURCE
#include "rsllm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static __thread size_t g_detail_a, g_detail_b;

void orc_last_detail(size_t *a, size_t *b) {
    if (a) *a = g_detail_a;
    if (b) *b = g_detail_b;
}

static int fail2(int code, size_t a, size_t b) {
    g_detail_a = a;
    g_detail_b = b;
    return code;
}

int orc_num_cores(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

/* ---- f16 -> f32 (exact widening, subnormals kept) ------------------------
 * half::f16::to_f32. A finite f16 is (-1)^s * m * 2^(e-25) with an 11-bit
 * significand m (implicit bit for e > 0); every such value is an f32. NaN
 * keeps its payload in the top mantissa bits with the quiet bit set, which
 * is what both the F16C instruction and half's software path produce. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ff;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m ? (0x00400000u | (m << 13)) : 0);
    } else if (e == 0) {
        float v = ldexpf((float)m, -24); /* subnormal or zero, exact */
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float rd_f16(const uint8_t *p) {
    return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ---- block geometry: rsllm-gguf/src/tensor.rs:128-184 -------------------- */
uint32_t orc_block_elements(uint32_t t) {
    switch (t) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q8_0: return 32;
    case ORC_Q2_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K:
    case ORC_IQ2_XXS: return 256;
    default: return 0;
    }
}

uint32_t orc_block_bytes(uint32_t t) {
    switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q8_0: return 34;
    case ORC_Q2_K: return 84;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_Q8_K: return 292;
    case ORC_IQ2_XXS: return 66;
    default: return 0;
    }
}

/* ---- q4_k_scale_min: rsllm-gguf/src/dequant/mod.rs:48-58 ---------------- */
void orc_q4k_scale_min(int j, const uint8_t q[12], uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Size rule shared by the block dequantizers (q4_k.rs:36-49, q6_k.rs:35-48,
 * q8_0.rs:26-42, q4_0.rs:85-100). */
static int check_blocks(size_t src_len, size_t n, size_t be, size_t bb) {
    if (n % be != 0)
        return fail2(ORC_DEQUANT_SIZE_MISMATCH, src_len, (n + be - 1) / be * bb);
    size_t expected = n / be * bb;
    if (src_len != expected) return fail2(ORC_DEQUANT_SIZE_MISMATCH, src_len, expected);
    return ORC_OK;
}

/* ---- dequant_q4_k: rsllm-gguf/src/dequant/q4_k.rs:35-92 ------------------ */
int orc_dequant_q4_k(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 144);
    if (rc) return rc;
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 144;
        float d = rd_f16(blk);
        float dmin = rd_f16(blk + 2);
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        float *o = dst + b * 256;
        for (int it = 0; it < 4; it++) { /* :66-88 */
            uint8_t sc1, m1, sc2, m2;
            orc_q4k_scale_min(2 * it, scales, &sc1, &m1);
            orc_q4k_scale_min(2 * it + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1;
            float m1f = dmin * (float)m1;
            float d2 = d * (float)sc2;
            float m2f = dmin * (float)m2;
            const uint8_t *q = qs + 32 * it;
            for (int l = 0; l < 32; l++) o[64 * it + l] = d1 * (float)(q[l] & 0x0F) - m1f;
            for (int l = 0; l < 32; l++) o[64 * it + 32 + l] = d2 * (float)(q[l] >> 4) - m2f;
        }
    }
    return ORC_OK;
}

/* ---- dequant_q6_k: rsllm-gguf/src/dequant/q6_k.rs:34-102 ----------------- */
int orc_dequant_q6_k(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 210);
    if (rc) return rc;
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 210;
        float d = rd_f16(blk + 208);
        for (int h = 0; h < 2; h++) { /* :65-98 */
            const uint8_t *ql = blk + 64 * h;
            const uint8_t *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            float *o = dst + b * 256 + 128 * h;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = ((ql[l] & 0x0F) | ((qh[l] & 0x03) << 4)) - 32;
                int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 0x03) << 4)) - 32;
                int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32;
                int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32;
                /* d * f32::from(sc) * (q as f32): left to right */
                o[l] = d * (float)sc[is] * (float)q1;
                o[l + 32] = d * (float)sc[is + 2] * (float)q2;
                o[l + 64] = d * (float)sc[is + 4] * (float)q3;
                o[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
    return ORC_OK;
}

/* ---- dequant_q8_0: rsllm-gguf/src/dequant/q8_0.rs:25-63 ------------------ */
int orc_dequant_q8_0(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 32, 34);
    if (rc) return rc;
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 34;
        float d = rd_f16(blk);
        for (int j = 0; j < 32; j++) dst[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
    return ORC_OK;
}

/* ---- dequant_q4_0: rsllm-gguf/src/dequant/q4_0.rs:44-64 ------------------ */
int orc_dequant_q4_0(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 32, 18);
    if (rc) return rc;
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 18;
        float d = rd_f16(blk);
        for (int j = 0; j < 16; j++) {
            int x0 = (blk[2 + j] & 0x0F) - 8;
            int x1 = (blk[2 + j] >> 4) - 8;
            dst[b * 32 + j] = (float)x0 * d;
            dst[b * 32 + j + 16] = (float)x1 * d;
        }
    }
    return ORC_OK;
}

/* ---- dequant_q4_1: rsllm-gguf/src/dequant/q4_0.rs:66-87 ------------------ */
/* 20-byte blocks [d f16 | m f16 | 16 code bytes]; x * d + m. */
int orc_dequant_q4_1(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 32, 20);
    if (rc) return rc;
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 20;
        float d = rd_f16(blk);
        float m = rd_f16(blk + 2);
        for (int j = 0; j < 16; j++) {
            float x0 = (float)(blk[4 + j] & 0x0F);
            float x1 = (float)(blk[4 + j] >> 4);
            dst[b * 32 + j] = x0 * d + m;
            dst[b * 32 + j + 16] = x1 * d + m;
        }
    }
    return ORC_OK;
}

/* ---- dequant_q5_k: rsllm-gguf/src/dequant/q5_k.rs:34-94 ------------------ */
/* 176-byte blocks [d | dmin | scales 12 | qh 32 | qs 128]. Four rounds, each
 * over a sub-block pair (is, is + 1): the low nibbles of qs[q_off + l] plus
 * 16 where qh[l] & u1, then the high nibbles plus 16 where qh[l] & u2; u1,
 * u2 start at 1, 2 and shift left by 2 per round. */
int orc_dequant_q5_k(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 176);
    if (rc) return rc;
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 176;
        float d = rd_f16(blk);
        float dmin = rd_f16(blk + 2);
        const uint8_t *scales = blk + 4;
        const uint8_t *qh = blk + 16;
        const uint8_t *qs = blk + 48;
        float *o = dst + b * 256;
        int is = 0, q_off = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int it = 0; it < 4; it++) {
            uint8_t sc1, m1, sc2, m2;
            orc_q4k_scale_min(is, scales, &sc1, &m1);
            orc_q4k_scale_min(is + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1;
            float m1f = dmin * (float)m1;
            float d2 = d * (float)sc2;
            float m2f = dmin * (float)m2;
            for (int l = 0; l < 32; l++) {
                uint8_t lo = qs[q_off + l] & 0x0F;
                uint8_t hb = (qh[l] & u1) ? 16 : 0;
                o[l] = d1 * (float)(uint8_t)(lo + hb) - m1f;
            }
            for (int l = 0; l < 32; l++) {
                uint8_t lo = qs[q_off + l] >> 4;
                uint8_t hb = (qh[l] & u2) ? 16 : 0;
                o[32 + l] = d2 * (float)(uint8_t)(lo + hb) - m2f;
            }
            o += 64;
            q_off += 32;
            is += 2;
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
    return ORC_OK;
}

/* ---- dequant_q8_k: rsllm-gguf/src/dequant/q8_k.rs:32-70 ------------------ */
/* 292-byte blocks [d f32 | qs 256 int8 | bsums 32 (unused)]; d * q. */
int orc_dequant_q8_k(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 292);
    if (rc) return rc;
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * 292;
        uint32_t bits = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) |
                        ((uint32_t)blk[3] << 24);
        float d;
        memcpy(&d, &bits, 4);
        for (int i = 0; i < 256; i++) dst[b * 256 + i] = d * (float)(int8_t)blk[4 + i];
    }
    return ORC_OK;
}

/* ---- float arms: rsllm-gguf/src/dequant/float.rs:14-52 ------------------- */
static int dequant_float(uint32_t t, const uint8_t *src, size_t src_len, float *dst, size_t n) {
    size_t w = (t == ORC_F32) ? 4 : 2;
    if (src_len != n * w) return fail2(ORC_DEQUANT_SIZE_MISMATCH, src_len, n * w);
    for (size_t i = 0; i < n; i++) {
        const uint8_t *p = src + i * w;
        uint32_t bits;
        if (t == ORC_F32) {
            bits = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                   ((uint32_t)p[3] << 24);
            memcpy(&dst[i], &bits, 4);
        } else if (t == ORC_F16) {
            dst[i] = rd_f16(p);
        } else {
            bits = ((uint32_t)p[0] | ((uint32_t)p[1] << 8)) << 16;
            memcpy(&dst[i], &bits, 4);
        }
    }
    return ORC_OK;
}

/* ---- dequant_to_f32: rsllm-gguf/src/dequant/mod.rs:69-85 ----------------- */
/* Q2_K, rsllm-gguf/src/dequant/q2_k.rs:39-98: 84-byte blocks [scales 16 |
 * qs 64 | d | dmin]; element e of a block uses sub-block e / 16 (scale nibble
 * low, min nibble high) and 2-bit code (qs[32 (e / 128) + (e % 32)] >>
 * 2 ((e % 128) / 32)) & 3; value (d * sc) * q - dmin * m, evaluated as the
 * reference does: dl = d * sc, ml = dmin * m (both exact), dl * q (exact),
 * then one rounding in the subtraction. */
int orc_dequant_q2_k(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 84);
    if (rc) return rc;
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 84;
        const float d = rd_f16(blk + 80), dmin = rd_f16(blk + 82);
        for (int e = 0; e < 256; e++) {
            const uint8_t sc = blk[e / 16];
            const float dl = d * (float)(sc & 0x0F);
            const float ml = dmin * (float)(sc >> 4);
            const int q = (blk[16 + 32 * (e / 128) + (e % 32)] >> (2 * ((e % 128) / 32))) & 3;
            dst[b * 256 + e] = dl * (float)q - ml;
        }
    }
    return ORC_OK;
}

/* IQ2_XXS codebook (ggml's iq2xxs_grid, the GGUF format constant): entry i
 * holds 8 bytes from {8, 25, 43}; stored here as base-3 numbers (byte j =
 * digit j, 8 -> 0, 25 -> 1, 43 -> 2). */
static const uint16_t kIq2Codes[256] = {
       0,    2,    4,    6,    8,   10,   12,   18,   20,   24,   26,   28,   30,   36,   42,   46,
      48,   54,   56,   62,   74,   82,   84,   90,   94,  108,  138,  150,  162,  164,  182,  218,
     244,  246,  252,  262,  264,  270,  272,  276,  288,  298,  300,  306,  318,  324,  326,  330,
     342,  356,  376,  378,  388,  412,  414,  432,  462,  480,  486,  490,  492,  498,  510,  514,
     516,  522,  524,  546,  570,  594,  650,  660,  730,  732,  738,  748,  756,  774,  786,  792,
     796,  810,  816,  828,  846,  854,  864,  912,  922,  972,  978,  990,  994, 1006, 1026, 1068,
    1100, 1134, 1148, 1216, 1218, 1224, 1242, 1270, 1296, 1300, 1368, 1414, 1458, 1460, 1466, 1488,
    1504, 1512, 1514, 1564, 1572, 1620, 1622, 1702, 1704, 1710, 1728, 1742, 1782, 1810, 1830, 1926,
    1950, 1962, 2010, 2136, 2188, 2190, 2196, 2202, 2206, 2208, 2214, 2220, 2228, 2232, 2242, 2244,
    2250, 2268, 2286, 2314, 2322, 2326, 2350, 2358, 2382, 2390, 2400, 2430, 2436, 2448, 2484, 2500,
    2522, 2532, 2592, 2674, 2676, 2682, 2700, 2704, 2754, 2796, 2800, 2810, 2866, 2898, 2916, 2922,
    2926, 2932, 2934, 2970, 2976, 3000, 3026, 3072, 3142, 3222, 3224, 3248, 3322, 3360, 3402, 3412,
    3418, 3450, 3510, 3570, 3648, 3654, 3672, 3696, 3726, 3766, 3822, 3852, 3888, 3892, 3978, 3980,
    4026, 4160, 4374, 4376, 4382, 4402, 4430, 4458, 4470, 4482, 4546, 4618, 4620, 4626, 4630, 4644,
    4662, 4698, 4730, 4764, 4786, 4806, 4824, 4862, 4944, 5032, 5106, 5112, 5124, 5130, 5176, 5198,
    5238, 5296, 5346, 5366, 5376, 5464, 5644, 5688, 5834, 5868, 5890, 5920, 5994, 6090, 6354, 6402,
};

static uint64_t iq2_grid_entry(int i) {
    static const uint8_t val[3] = {8, 25, 43};
    uint32_t c = kIq2Codes[i];
    uint64_t v = 0;
    for (int j = 0; j < 8; j++) {
        v |= (uint64_t)val[c % 3] << (8 * j);
        c /= 3;
    }
    return v;
}

uint64_t orc_iq2xxs_grid(int i) { return (i >= 0 && i < 256) ? iq2_grid_entry(i) : 0; }

/* IQ2_XXS, rsllm-gguf/src/dequant/iq2_xxs.rs:47-113: 66-byte blocks [d |
 * 8 sub-groups x (u32 grid indices, u32 signs/extra)]. Sub-group g: db = d *
 * (0.5 + (aux1 >> 28)) * 0.25; element 8l + j = db * grid[aux0 byte l][j] *
 * sign, negative when bit j of ksigns(aux1 >> 7l & 127) is set, where
 * ksigns(i) = i with bit 7 = parity of i (the format's sign table). Every
 * product is exact. */
int orc_dequant_iq2_xxs(const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int rc = check_blocks(src_len, n, 256, 66);
    if (rc) return rc;
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 66;
        const float d = rd_f16(blk);
        for (int g = 0; g < 8; g++) {
            const uint8_t *q = blk + 2 + 8 * g;
            const uint32_t aux0 = (uint32_t)q[0] | (uint32_t)q[1] << 8 | (uint32_t)q[2] << 16 |
                                  (uint32_t)q[3] << 24;
            const uint32_t aux1 = (uint32_t)q[4] | (uint32_t)q[5] << 8 | (uint32_t)q[6] << 16 |
                                  (uint32_t)q[7] << 24;
            const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                const uint64_t grid = iq2_grid_entry((aux0 >> (8 * l)) & 0xFF);
                const uint32_t si = (aux1 >> (7 * l)) & 0x7F;
                const uint32_t signs = si | ((uint32_t)__builtin_parity(si) << 7);
                for (int j = 0; j < 8; j++) {
                    const float gv = (float)(int8_t)(grid >> (8 * j));
                    const float sg = (signs >> j) & 1 ? -1.0f : 1.0f;
                    dst[b * 256 + 32 * g + 8 * l + j] = db * gv * sg;
                }
            }
        }
    }
    return ORC_OK;
}

int orc_dequant_to_f32(uint32_t t, const uint8_t *src, size_t src_len, float *dst, size_t n) {
    switch (t) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return dequant_float(t, src, src_len, dst, n);
    case ORC_Q4_0: return orc_dequant_q4_0(src, src_len, dst, n);
    case ORC_Q4_1: return orc_dequant_q4_1(src, src_len, dst, n);
    case ORC_Q4_K: return orc_dequant_q4_k(src, src_len, dst, n);
    case ORC_Q5_K: return orc_dequant_q5_k(src, src_len, dst, n);
    case ORC_Q8_K: return orc_dequant_q8_k(src, src_len, dst, n);
    case ORC_Q6_K: return orc_dequant_q6_k(src, src_len, dst, n);
    case ORC_Q8_0: return orc_dequant_q8_0(src, src_len, dst, n);
    case ORC_Q2_K: return orc_dequant_q2_k(src, src_len, dst, n);
    case ORC_IQ2_XXS: return orc_dequant_iq2_xxs(src, src_len, dst, n);
    default: return fail2(ORC_UNSUPPORTED_DEQUANT, t, 0);
    }
}

/* ---- per-token task pool (rayon par_chunks_mut, parallel.rs:37-54) ------- */
typedef struct {
    void (*fn)(void *ctx, size_t t);
    void *ctx;
    size_t n;
    size_t next;
    pthread_mutex_t mu;
} pool_t;

static void *pool_worker(void *arg) {
    pool_t *p = (pool_t *)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        size_t t = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (t >= p->n) break;
        p->fn(p->ctx, t);
    }
    return NULL;
}

static void run_tasks(size_t n, int n_threads, void (*fn)(void *, size_t), void *ctx) {
    if (n_threads <= 0) n_threads = orc_num_cores();
    if ((size_t)n_threads > n) n_threads = (int)n;
    if (n_threads <= 1) {
        for (size_t t = 0; t < n; t++) fn(ctx, t);
        return;
    }
    pool_t p = {fn, ctx, n, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
    for (int i = 0; i < n_threads; i++) pthread_create(&th[i], NULL, pool_worker, &p);
    for (int i = 0; i < n_threads; i++) pthread_join(th[i], NULL);
    free(th);
}

/* ---- matmul_quant_f32: rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119 -- */
typedef struct {
    float *out;
    const uint8_t *w;
    const float *x;
    size_t in_dim, out_dim, row_bytes, row0, row1;
    uint32_t dtype;
} mm_ctx;

static void mm_token(void *vctx, size_t t) {
    mm_ctx *c = (mm_ctx *)vctx;
    const float *x_row = c->x + t * c->in_dim;
    float *out_row = c->out + t * c->out_dim;
    float *w_row = (float *)calloc(c->in_dim ? c->in_dim : 1, sizeof(float)); /* :99 */
    for (size_t o = c->row0; o < c->row1; o++) {                              /* :100 */
        const uint8_t *wp = c->w + o * c->row_bytes;
        if (orc_dequant_to_f32(c->dtype, wp, c->row_bytes, w_row, c->in_dim) != ORC_OK) {
            out_row[o] = 0.0f; /* :106-108 */
            continue;
        }
        float dot = 0.0f; /* :110-113, sequential, no contraction */
        for (size_t i = 0; i < c->in_dim; i++) dot += w_row[i] * x_row[i];
        out_row[o] = dot; /* :114 overwrite */
    }
    free(w_row);
}

int orc_matmul_quant_f32(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                         const float *x, size_t x_len, size_t n_tok, size_t in_dim,
                         size_t out_dim, uint32_t dtype, int allow_q6k, int n_threads) {
    /* :57-64 dtype guard */
    int ok = dtype == ORC_Q4_K || dtype == ORC_Q2_K || dtype == ORC_IQ2_XXS ||
             dtype == ORC_Q4_0 || dtype == ORC_Q8_0 || (allow_q6k && dtype == ORC_Q6_K);
    if (!ok) return fail2(ORC_SHAPE_MISMATCH, 0, 0);
    size_t be = orc_block_elements(dtype), bb = orc_block_bytes(dtype);
    /* :66-74 */
    if (in_dim % be != 0) return fail2(ORC_NOT_BLOCK_ALIGNED, in_dim, be);
    size_t row_bytes = in_dim / be * bb;
    size_t need;
    /* :78-92, in this order */
    if (__builtin_mul_overflow(out_dim, row_bytes, &need) || w_len != need)
        return fail2(ORC_SHAPE_MISMATCH, 1, 0);
    if (__builtin_mul_overflow(n_tok, in_dim, &need) || x_len != need)
        return fail2(ORC_SHAPE_MISMATCH, 2, 0);
    if (__builtin_mul_overflow(n_tok, out_dim, &need) || out_len != need)
        return fail2(ORC_SHAPE_MISMATCH, 3, 0);
    /* for_each_row_mut asserts row_len > 0 (parallel.rs:44): a panic. */
    if (out_dim == 0) return fail2(ORC_PANIC, 0, 0);
    mm_ctx c = {out, w, x, in_dim, out_dim, row_bytes, 0, out_dim, dtype};
    run_tasks(n_tok, n_threads, mm_token, &c);
    return ORC_OK;
}

int orc_matmul_quant_f32_rows(float *out, const uint8_t *w, const float *x, size_t n_tok,
                              size_t in_dim, size_t out_dim, uint32_t dtype, size_t row0,
                              size_t row1, int n_threads) {
    size_t be = orc_block_elements(dtype), bb = orc_block_bytes(dtype);
    if (!be || in_dim % be || row1 > out_dim || row0 > row1) return ORC_SHAPE_MISMATCH;
    mm_ctx c = {out, w, x, in_dim, out_dim, in_dim / be * bb, row0, row1, dtype};
    run_tasks(n_tok, n_threads, mm_token, &c);
    return ORC_OK;
}

/* ---- matmul_weight_f32: rsllm-models/src/dsv4/weight.rs:113-169 ------------ */
int orc_matmul_weight_f32(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                          const float *x, size_t x_len, size_t n_tok, size_t in_dim,
                          size_t out_dim, uint32_t dtype, int allow_q6k) {
    size_t need;
    if (__builtin_mul_overflow(n_tok, out_dim, &need) || out_len != need) /* :121-127 */
        return fail2(ORC_SHAPE_MISMATCH, 10, 0);
    if (__builtin_mul_overflow(n_tok, in_dim, &need) || x_len != need) /* :128-134 */
        return fail2(ORC_SHAPE_MISMATCH, 11, 0);
    if (dtype == ORC_F32) {
        if (__builtin_mul_overflow(out_dim, in_dim, &need) || w_len != need * 4) /* :141-146 */
            return fail2(ORC_SHAPE_MISMATCH, 12, 0);
        for (size_t t = 0; t < n_tok; t++) { /* :148-157 */
            const float *xr = x + t * in_dim;
            float *orow = out + t * out_dim;
            for (size_t o = 0; o < out_dim; o++) {
                float dot = 0.0f, wv;
                for (size_t i = 0; i < in_dim; i++) {
                    memcpy(&wv, w + (o * in_dim + i) * 4, 4);
                    dot += wv * xr[i];
                }
                orow[o] = dot;
            }
        }
        return ORC_OK;
    }
    int rc = orc_matmul_quant_f32(out, out_len, w, w_len, x, x_len, n_tok, in_dim, out_dim, dtype,
                                  allow_q6k, 1);
    if (rc == ORC_OK || rc == ORC_PANIC) return rc;
    return fail2(ORC_SHAPE_MISMATCH, 13, 0); /* :160-167 map_err */
}

/* ---- matmul_grouped_lora_down: weight.rs:209-266, slices :271-323 ------- */
int orc_matmul_grouped_lora_down(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                                 const float *x, size_t x_len, size_t n_tok, size_t n_groups,
                                 size_t group_dim, size_t rank, uint32_t dtype, int allow_q6k) {
    size_t total_in, total_out, need;
    if (__builtin_mul_overflow(n_groups, group_dim, &total_in) ||
        __builtin_mul_overflow(n_tok, total_in, &need) || x_len != need) /* :219-225 */
        return fail2(ORC_SHAPE_MISMATCH, 20, 0);
    if (__builtin_mul_overflow(n_groups, rank, &total_out) ||
        __builtin_mul_overflow(n_tok, total_out, &need) || out_len != need) /* :226-232 */
        return fail2(ORC_SHAPE_MISMATCH, 21, 0);
    float *xg = malloc((n_tok * group_dim + 1) * sizeof(float)); /* :239-240 */
    float *og = malloc((n_tok * rank + 1) * sizeof(float));
    int rc = ORC_OK;
    const size_t epg = group_dim * rank;
    for (size_t g = 0; g < n_groups && rc == ORC_OK; g++) { /* :241 */
        for (size_t t = 0; t < n_tok; t++) /* :243-246 gather */
            memcpy(xg + t * group_dim, x + t * total_in + g * group_dim, group_dim * sizeof(float));
        /* grouped_weight_slice (:271-323) */
        const uint8_t *wg;
        size_t wg_len;
        if (dtype == ORC_F32) {
            size_t start = g * epg, end = start + epg;
            if (end > w_len / 4) { rc = fail2(ORC_SHAPE_MISMATCH, 22, g); break; }
            wg = w + start * 4;
            wg_len = epg * 4;
        } else {
            size_t be = orc_block_elements(dtype), bb = orc_block_bytes(dtype);
            if (be == 0) { rc = fail2(ORC_SHAPE_MISMATCH, 13, g); break; } /* not a known type */
            if (epg % be != 0) { rc = fail2(ORC_SHAPE_MISMATCH, 23, g); break; }
            size_t stride = epg / be * bb, start = g * stride, end = start + stride;
            if (end > w_len) { rc = fail2(ORC_SHAPE_MISMATCH, 24, g); break; }
            wg = w + start;
            wg_len = stride;
        }
        rc = orc_matmul_weight_f32(og, n_tok * rank, wg, wg_len, xg, n_tok * group_dim, n_tok,
                                   group_dim, rank, dtype, allow_q6k); /* :248-256 */
        if (rc != ORC_OK) break;
        for (size_t t = 0; t < n_tok; t++) /* :258-261 scatter */
            memcpy(out + t * total_out + g * rank, og + t * rank, rank * sizeof(float));
    }
    free(xg);
    free(og);
    return rc;
}

/* ---- quantize_q8_0_activation: rsllm-backend-cpu/src/ops/q8_0.rs:42-88 --- */
int orc_quantize_q8_0_activation(const float *x, size_t n, int8_t *xq, size_t xq_len,
                                 float *scale, size_t scale_len) {
    size_t blocks = (n + 31) / 32;
    if (xq_len != blocks * 32) return fail2(ORC_SHAPE_MISMATCH, 1, 0);
    if (scale_len != blocks) return fail2(ORC_SHAPE_MISMATCH, 2, 0);
    for (size_t b = 0; b < blocks; b++) {
        size_t i0 = b * 32;
        size_t bn = n - i0 < 32 ? n - i0 : 32;
        float amax = 0.0f;
        for (size_t i = 0; i < bn; i++) {
            float v = x[i0 + i];
            if (!isfinite(v)) return fail2(ORC_NON_FINITE_INPUT, i0 + i, 0);
            float ax = fabsf(v);
            if (ax > amax) amax = ax;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        scale[b] = d;
        for (size_t i = 0; i < bn; i++) {
            /* round_ties_even then `as i32` (saturating, NaN -> 0), then
             * clamp. x * id can be inf or NaN when d is subnormal and 1/d
             * overflows. */
            float r = rintf(x[i0 + i] * id);
            int v;
            if (r != r) v = 0;
            else if (r >= 2147483647.0f) v = 2147483647;
            else if (r <= -2147483648.0f) v = -2147483647 - 1;
            else v = (int)r;
            if (v < -128) v = -128;
            if (v > 127) v = 127;
            xq[i0 + i] = (int8_t)v;
        }
        for (size_t i = bn; i < 32; i++) xq[i0 + i] = 0;
    }
    return ORC_OK;
}

/* ---- quantize_q8_0_batch: q8_0.rs:95-129 --------------------------------- */
int orc_quantize_q8_0_batch(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                            float *scale, size_t scale_len, size_t n_tok, size_t in_dim) {
    size_t blocks = (in_dim + 31) / 32;
    if (x_len != n_tok * in_dim) return fail2(ORC_SHAPE_MISMATCH, 1, 0);
    if (xq_len != n_tok * blocks * 32) return fail2(ORC_SHAPE_MISMATCH, 2, 0);
    if (scale_len != n_tok * blocks) return fail2(ORC_SHAPE_MISMATCH, 3, 0);
    /* try_for_each over tokens: the first failing token's error is reported;
     * with one token failing, every thread schedule gives the same code. */
    for (size_t t = 0; t < n_tok; t++) {
        int rc = orc_quantize_q8_0_activation(x + t * in_dim, in_dim, xq + t * blocks * 32,
                                              blocks * 32, scale + t * blocks, blocks);
        if (rc) return rc;
    }
    return ORC_OK;
}

/* ---- block_scale_finite: q8_0.rs:133-146 --------------------------------- */
static inline float block_scale_finite(const uint8_t *blk) {
    float s = rd_f16(blk);
    return isfinite(s) ? s : 0.0f;
}

/* ---- dot_q8_0_row_scalar: q8_0.rs:163-193 -------------------------------- */
float orc_dot_q8_0_row_scalar(const uint8_t *row, const int8_t *xq, const float *xscale,
                              size_t in_dim) {
    size_t blocks = (in_dim + 31) / 32;
    float acc = 0.0f;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * 34;
        float ws = block_scale_finite(blk);
        const int8_t *wq = (const int8_t *)(blk + 2);
        size_t i0 = b * 32;
        size_t bn = in_dim - i0 < 32 ? in_dim - i0 : 32;
        int32_t dot = 0;
        for (size_t i = 0; i < bn; i++) dot += (int32_t)wq[i] * (int32_t)xq[i0 + i];
        acc += ws * xscale[b] * (float)dot; /* (ws * xs) * dot, then += */
    }
    return acc;
}

/* ---- matmul_q8_0_batch: q8_0.rs:217-263 ---------------------------------- */
typedef struct {
    float *out;
    const uint8_t *w;
    const int8_t *xq;
    const float *xs;
    size_t in_dim, out_dim, blocks;
} mq_ctx;

static void mq_token(void *vctx, size_t t) {
    mq_ctx *c = (mq_ctx *)vctx;
    size_t stride = c->blocks * 34;
    for (size_t o = 0; o < c->out_dim; o++)
        c->out[t * c->out_dim + o] = orc_dot_q8_0_row_scalar(
            c->w + o * stride, c->xq + t * c->blocks * 32, c->xs + t * c->blocks, c->in_dim);
}

int orc_matmul_q8_0_batch(float *out, size_t out_len, const uint8_t *w, size_t w_len,
                          const int8_t *xq, size_t xq_len, const float *xscale,
                          size_t xscale_len, size_t n_tok, size_t in_dim, size_t out_dim,
                          int n_threads) {
    size_t blocks = (in_dim + 31) / 32;
    if (w_len != out_dim * blocks * 34) return fail2(ORC_SHAPE_MISMATCH, 1, 0);
    if (xq_len != n_tok * blocks * 32) return fail2(ORC_SHAPE_MISMATCH, 2, 0);
    if (xscale_len != n_tok * blocks) return fail2(ORC_SHAPE_MISMATCH, 3, 0);
    if (out_len != n_tok * out_dim) return fail2(ORC_SHAPE_MISMATCH, 4, 0);
    if (out_dim == 0) return fail2(ORC_PANIC, 0, 0);
    mq_ctx c = {out, w, xq, xscale, in_dim, out_dim, blocks};
    run_tasks(n_tok, n_threads, mq_token, &c);
    return ORC_OK;
}

/* ---- sigmoid / silu: rsllm-backend-cpu/src/ops/scalar.rs:57-75 ----------- */
static float sigmoid_stable(float x) {
    if (x >= 0.0f) {
        float e = expf(-x);
        return 1.0f / (1.0f + e);
    }
    float e = expf(x);
    return e / (1.0f + e);
}

float orc_silu(float x) { return x * sigmoid_stable(x); }
float orc_sigmoid(float x) { return sigmoid_stable(x); }

/* apply_swiglu_clamp, moe.rs:515-531: only when c > 1e-6; gate from above,
 * up both sides; NaN passes (every comparison with NaN is false). */
void orc_swiglu_clamp(float *h_gate, float *h_up, size_t n, float c) {
    if (c <= 1e-6f) return;
    for (size_t j = 0; j < n; j++)
        if (h_gate[j] > c) h_gate[j] = c;
    for (size_t j = 0; j < n; j++) {
        if (h_up[j] > c) h_up[j] = c;
        else if (h_up[j] < -c) h_up[j] = -c;
    }
}

/* ---- shared expert: apply_shared_expert moe.rs:422-455 ----------------------
 * check_moe_shapes (:557-573: x then out), then per token apply_expert_swiglu
 * (:479-502): gate and up through matmul_weight_f32, the clamp, silu(g) * u
 * (scalar.rs:80-86), down through matmul_weight_f32 into out_t (overwritten).
 * Errors: ORC_SHAPE_MISMATCH detail a = 30 (x), 31 (out), else those of
 * orc_matmul_weight_f32 with detail b = 0 (gate), 1 (up), 2 (down). */
int orc_apply_shared_expert(float *out, size_t out_len, const float *x, size_t x_len,
                            const uint8_t *gate, size_t gate_len, uint32_t dt_gate,
                            const uint8_t *up, size_t up_len, uint32_t dt_up,
                            const uint8_t *down, size_t down_len, uint32_t dt_down, size_t n_tok,
                            size_t n_embd, size_t n_ff, float clamp) {
    size_t need;
    if (__builtin_mul_overflow(n_tok, n_embd, &need) || x_len != need)
        return fail2(ORC_SHAPE_MISMATCH, 30, 0);
    if (out_len != need) return fail2(ORC_SHAPE_MISMATCH, 31, 0);
    float *h_gate = (float *)malloc(sizeof(float) * (n_ff + 1));
    float *h_up = (float *)malloc(sizeof(float) * (n_ff + 1));
    float *h_act = (float *)malloc(sizeof(float) * (n_ff + 1));
    int rc = ORC_OK;
    size_t a, b;
    for (size_t t = 0; t < n_tok && rc == ORC_OK; t++) {
        const float *x_t = x + t * n_embd;
        rc = orc_matmul_weight_f32(h_gate, n_ff, gate, gate_len, x_t, n_embd, 1, n_embd, n_ff,
                                   dt_gate, 1);
        if (rc) { orc_last_detail(&a, &b); fail2(rc, a, 0); break; }
        rc = orc_matmul_weight_f32(h_up, n_ff, up, up_len, x_t, n_embd, 1, n_embd, n_ff, dt_up,
                                   1);
        if (rc) { orc_last_detail(&a, &b); fail2(rc, a, 1); break; }
        orc_swiglu_clamp(h_gate, h_up, n_ff, clamp);
        for (size_t j = 0; j < n_ff; j++) h_act[j] = orc_silu(h_gate[j]) * h_up[j];
        rc = orc_matmul_weight_f32(out + t * n_embd, n_embd, down, down_len, h_act, n_ff, 1, n_ff,
                                   n_embd, dt_down, 1);
        if (rc) { orc_last_detail(&a, &b); fail2(rc, a, 2); break; }
    }
    free(h_gate);
    free(h_up);
    free(h_act);
    return rc;
}

/* ---- routed experts: moe.rs:479-531 and :648-707 -------------------------- */
int orc_moe_routed(float *out, const float *x, size_t n_tok, size_t n_embd, size_t n_ff,
                   const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                   uint32_t dtype_gate_up, uint32_t dtype_down, size_t n_expert,
                   const int32_t *ids, const float *weights, size_t k, float clamp) {
    size_t be_gu = orc_block_elements(dtype_gate_up), bb_gu = orc_block_bytes(dtype_gate_up);
    size_t be_d = orc_block_elements(dtype_down), bb_d = orc_block_bytes(dtype_down);
    if (!be_gu || !be_d || n_embd % be_gu || n_ff % be_d) return ORC_NOT_BLOCK_ALIGNED;
    size_t gu_stride = n_ff * (n_embd / be_gu * bb_gu);   /* expert stride, moe.rs:86-94 */
    size_t d_stride = n_embd * (n_ff / be_d * bb_d);
    float *h_gate = (float *)malloc(sizeof(float) * n_ff);
    float *h_up = (float *)malloc(sizeof(float) * n_ff);
    float *h_act = (float *)malloc(sizeof(float) * n_ff);
    float *eo = (float *)malloc(sizeof(float) * n_embd);
    int rc = ORC_OK;
    for (size_t t = 0; t < n_tok && rc == ORC_OK; t++) {
        const float *x_t = x + t * n_embd;
        float *out_t = out + t * n_embd;
        for (size_t i = 0; i < k; i++) {
            int32_t e = ids[t * k + i];
            float we = weights[t * k + i];
            if (we == 0.0f) continue; /* :681-683 */
            if (e < 0 || (size_t)e >= n_expert) { rc = ORC_SHAPE_MISMATCH; break; }
            /* apply_expert_swiglu :488-500 */
            rc = orc_matmul_quant_f32(h_gate, n_ff, gate + (size_t)e * gu_stride, gu_stride, x_t,
                                      n_embd, 1, n_embd, n_ff, dtype_gate_up, 1, 1);
            if (!rc)
                rc = orc_matmul_quant_f32(h_up, n_ff, up + (size_t)e * gu_stride, gu_stride, x_t,
                                          n_embd, 1, n_embd, n_ff, dtype_gate_up, 1, 1);
            if (rc) break;
            orc_swiglu_clamp(h_gate, h_up, n_ff, clamp);
            for (size_t j = 0; j < n_ff; j++) h_act[j] = orc_silu(h_gate[j]) * h_up[j];
            rc = orc_matmul_quant_f32(eo, n_embd, down + (size_t)e * d_stride, d_stride, h_act,
                                      n_ff, 1, n_ff, n_embd, dtype_down, 1, 1);
            if (rc) break;
            for (size_t j = 0; j < n_embd; j++) out_t[j] += we * eo[j]; /* :700-702 */
        }
    }
    free(h_gate);
    free(h_up);
    free(h_act);
    free(eo);
    return rc;
}
