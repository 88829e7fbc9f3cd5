// Prefill GEMM: out[t, o] = sum_i deq(W)[o, i] * x[t, i] for a Q4_K, Q8_0 or
// Q6_K weight W [out_dim x in_dim] and bf16 or f32 activations x [n_tok x
// in_dim], fp32 output.
//
// The reference computes this as matmul_quant_f32 (backend-cpu/src/ops/
// quant_matmul.rs:45-119): every weight row is dequantised once per token and
// dotted in f32. Here it is one dense contraction on the CDNA4 matrix cores:
//
// 1. k_prefill_x / k_prefill_x_f32: per token t, x is scaled by 2^e_t so that
//    max|x_t| lands in [2^14, 2^15) and converted to f16. bf16 has an 8-bit
//    significand, so that conversion is exact for every element within 2^-29
//    of the token's maximum; f32 is rounded once (2^-11 relative). 2^-e_t is
//    kept to undo the scaling in the epilogue.
// 2. The GEMM dequantises W in registers to f16, w = f16(d*sc_j) * q -
//    f16(dmin*m_j) (packed f16 FMA, q exact), straight into the operands of
//    v_mfma_f32_16x16x32_f16 against the f16 activations; products
//    accumulate in fp32. The f16 weight rounding (about 2^-11 relative per
//    weight) keeps the output within about 4e-4 of the reference, inside the
//    1e-3 budget. The weights are the MFMA A operand and the activations the
//    B operand, so every lane ends with 4 consecutive outputs of one token.
//    k_prefill_q4k_w8 runs it: a workgroup of 8 wavefronts covers 256 weight
//    rows x 128 tokens, two wavefronts per SIMD that split K between them
//    (described at the kernel). k_prefill_q8_w8 (w = f16(d) * q) and
//    k_prefill_q6_w8 (w = f16(d*sc) * (q - 32)) keep that workgroup and
//    change only the weight stage and the dequantisation.
// 3. Range guard. d and dmin are f16 and sc, m, q integers, so every exact
//    intermediate of a weight's dequantisation is a multiple of 2^-24 (f16's
//    subnormal spacing): its f16 rounding is exact below 2^-13 and within
//    2^-11 relative everywhere. The one failure is overflow past 65504 (d above
//    about 69 for Q4_K, 16 for Q6_K, 511 for Q8_0), which turns the row's
//    outputs into inf/NaN. The epilogue checks what it stores; a workgroup
//    that stored a non-finite value runs its tile again with each row's
//    weights scaled by a power of two 2^-E that keeps them in range, and
//    stores again with the 2^E put back (see kPfNeedHi).
#include "kernels.h"

#include <algorithm>
#include <climits>

#include "../../include/rsllm_hip.h"

namespace rsllm_hip {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPfTok = 128;    // tokens per workgroup
constexpr int kPfRowsWg = 256;  // weight rows per workgroup

// ---- activation pre-pass: bf16 -> scaled f16 ----------------------------------
// One workgroup (256 threads) per token; each thread moves 16-byte pieces (8
// elements). Up to kPxCache pieces per thread (in_dim <= 16384) stay in
// registers between the max pass and the conversion, so the token is read
// once; longer rows are read twice. in_dim is a multiple of 256.
constexpr int kPxCache = 8;

__device__ __forceinline__ uint32_t px_absmax_bits(const uint4 v) {
    // |bf16| bit patterns order like the magnitudes (finite values)
    const uint32_t a = max(v.x & 0x7FFF7FFFu, v.y & 0x7FFF7FFFu);
    const uint32_t b = max(v.z & 0x7FFF7FFFu, v.w & 0x7FFF7FFFu);
    const uint32_t c = max(a, b);
    return max(c & 0xFFFFu, c >> 16);
}

__device__ __forceinline__ uint4 px_convert(const uint4 v, float up) {
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const _Float16 lo = (_Float16)(__uint_as_float(in[k] << 16) * up);
        const _Float16 hi = (_Float16)(__uint_as_float(in[k] & 0xFFFF0000u) * up);
        o[k] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
               ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ __launch_bounds__(256) void k_prefill_x(const uint16_t *__restrict__ x,
                                                   _Float16 *__restrict__ xh,
                                                   float *__restrict__ unscale, int in_dim) {
    __shared__ uint32_t red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const uint4 *xt = reinterpret_cast<const uint4 *>(x + (size_t)t * in_dim);
    uint4 *ht = reinterpret_cast<uint4 *>(xh + (size_t)t * in_dim);
    const int n8 = in_dim >> 3;  // 16-byte pieces in the row (a multiple of 32)
    const bool cached = n8 <= 256 * kPxCache;
    uint4 c[kPxCache];
    uint32_t mbits = 0;
    if (cached) {
#pragma unroll
        for (int i = 0; i < kPxCache; i++) {
            const int idx = i * 256 + tid;
            if (idx < n8) {
                c[i] = xt[idx];
                mbits = max(mbits, px_absmax_bits(c[i]));
            }
        }
    } else {
        for (int idx = tid; idx < n8; idx += 256) mbits = max(mbits, px_absmax_bits(xt[idx]));
    }
    // NaN patterns (above 0x7F80) do not pick the scale; infinity does
    if (mbits > 0x7F80u) mbits = 0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mbits = max(mbits, (uint32_t)__shfl_xor((int)mbits, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mbits;
    __syncthreads();
    mbits = max(max(red[0], red[1]), max(red[2], red[3]));
    const float amax = __uint_as_float(mbits << 16);
    // e: amax * 2^e in [2^14, 2^15) for finite nonzero amax (exponent from the bits)
    int e = 0;
    if (amax > 0.f && amax <= 3.4e38f) {
        const int ex = (int)((__float_as_uint(amax) >> 23) & 0xFF) - 127;
        e = 14 - (ex < -126 ? -126 : ex);
        if (e > 120) e = 120;
    }
    const float up = __uint_as_float((uint32_t)(127 + e) << 23);
    if (tid == 0) unscale[t] = __uint_as_float((uint32_t)(127 - e) << 23);
    if (cached) {
#pragma unroll
        for (int i = 0; i < kPxCache; i++) {
            const int idx = i * 256 + tid;
            if (idx < n8) ht[idx] = px_convert(c[i], up);
        }
    } else {
        for (int idx = tid; idx < n8; idx += 256) ht[idx] = px_convert(xt[idx], up);
    }
}

// f32 activations (the reference's own prefill input, engine_impl.rs:277 ->
// weight.rs:161-163 -> quant_matmul.rs:45 with n_tok = T): the same scaled
// f16 image. Each element is rounded once to f16 (at most 2^-11 relative);
// pieces of 8 elements (two 16-byte loads), up to kPxCache per thread kept
// in registers between the max pass and the conversion (in_dim <= 16384).
__global__ __launch_bounds__(256) void k_prefill_x_f32(const float *__restrict__ x,
                                                       _Float16 *__restrict__ xh,
                                                       float *__restrict__ unscale, int in_dim) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float4 *xt = reinterpret_cast<const float4 *>(x + (size_t)t * in_dim);
    uint4 *ht = reinterpret_cast<uint4 *>(xh + (size_t)t * in_dim);
    const int n8 = in_dim >> 3;
    const bool cached = n8 <= 256 * kPxCache;
    float4 c[kPxCache][2];
    auto amax8 = [](const float4 &a, const float4 &b) {
        const float m0 = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
        const float m1 = fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)));
        return fmaxf(m0, m1);  // NaN lanes drop out of fmaxf
    };
    float m = 0.f;
    if (cached) {
#pragma unroll
        for (int i = 0; i < kPxCache; i++) {
            const int idx = i * 256 + tid;
            if (idx < n8) {
                c[i][0] = xt[2 * idx];
                c[i][1] = xt[2 * idx + 1];
                m = fmaxf(m, amax8(c[i][0], c[i][1]));
            }
        }
    } else {
        for (int idx = tid; idx < n8; idx += 256) m = fmaxf(m, amax8(xt[2 * idx], xt[2 * idx + 1]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // e: amax * 2^e in [2^14, 2^15) for finite nonzero amax
    int e = 0;
    if (amax > 0.f && amax <= 3.4e38f) {
        const int ex = (int)((__float_as_uint(amax) >> 23) & 0xFF) - 127;
        e = 14 - (ex < -126 ? -126 : ex);
        if (e > 120) e = 120;
    }
    const float up = __uint_as_float((uint32_t)(127 + e) << 23);
    if (tid == 0) unscale[t] = __uint_as_float((uint32_t)(127 - e) << 23);
    auto cvt = [&](const float4 &a, const float4 &b) {
        h8 h;
        h[0] = (_Float16)(a.x * up); h[1] = (_Float16)(a.y * up);
        h[2] = (_Float16)(a.z * up); h[3] = (_Float16)(a.w * up);
        h[4] = (_Float16)(b.x * up); h[5] = (_Float16)(b.y * up);
        h[6] = (_Float16)(b.z * up); h[7] = (_Float16)(b.w * up);
        return __builtin_bit_cast(uint4, h);
    };
    if (cached) {
#pragma unroll
        for (int i = 0; i < kPxCache; i++) {
            const int idx = i * 256 + tid;
            if (idx < n8) ht[idx] = cvt(c[i][0], c[i][1]);
        }
    } else {
        for (int idx = tid; idx < n8; idx += 256) ht[idx] = cvt(xt[2 * idx], xt[2 * idx + 1]);
    }
}

// ---- GEMM -------------------------------------------------------------------------
// Eight f16 weights of one chunk: qs bytes b0..b7 are dwords d0 (b0..b3) and
// d1 (b4..b7); `hi` selects the high nibbles. w = q * dsc - dm.
// A byte 0..15 read as fp8 e4m3 is q * 2^-9 exactly (subnormal for q < 8,
// exponent 1 above), and v_cvt_scalef32_pk_f16_fp8 applies its scale as a
// power of two, so a scale of 2^9 yields the integer q in f16 exactly — two
// weights per instruction.
__device__ __forceinline__ h8 pf_dequant8(uint32_t d0, uint32_t d1, bool hi, h2 dsc, h2 dm) {
    return dequant_q4x8_f16(d0, d1, hi, dsc, dm);
}

// ---- weight range guard -------------------------------------------------------------
// Every block has a bound N on its weights and on every f16 intermediate of
// their dequantisation: 945 |d| + 63 |dmin| for Q4_K (sc, m <= 63, q <=
// 15), 4096 |d| for Q6_K (|sc| <= 128, |q - 32| <= 32), 128 |d| for Q8_0.
// A second pass scales row r's weights by 2^-E_r, E_r = max(0, k - 14) for
// the row's largest N = m 2^k (m in [0.5, 1)) over the blocks of the
// workgroup's K range, so N 2^-E < 2^15 and no f16 value passes 2^15 (1 +
// 2^-11)^2 < 65504. With E_r > 0 a scaled scale is no longer a multiple of
// 2^-24 and an f16 rounding may be off by 2^(E_r - 25) <= 2^-38 N absolute.
constexpr float kPfNeedHi = 32768.0f;
__device__ __forceinline__ int pf_row_exponent(float n) {
    if (!(n > kPfNeedHi && n <= 3.4e38f)) return 0;
    int k;
    (void)frexpf(n, &k);  // n = m 2^k, m in [0.5, 1)
    return k - 14;
}
// LDS words after a GEMM's stages: the workgroup's flag, then E of its 256 rows
constexpr int kPfGuardBytes = 16 + 4 * kPfRowsWg;

// ---- 8-wavefront GEMM: two K groups per workgroup -----------------------------
// The workgroup covers 256 weight rows x 128 tokens with 8 wavefronts: wave w
// owns rows 64 (w & 3) .. + 63 for all 128 tokens (8 x 4 MFMA tiles in VGPRs)
// and K group w >> 2, which takes every other quarter (64 elements) of each
// super-block: group g computes quarters g and 2 + g. Each weight is
// dequantised once per workgroup and used for 128 tokens, and every SIMD holds
// two wavefronts,
// one of each group, so one wavefront's dequantisation, LDS waits and barrier
// drain run while the other issues MFMAs (a VALU instruction in an MFMA's own
// wavefront stalls the matrix pipe on gfx950). The two groups' partial sums
// are added once, through LDS, before the store.
//
// K order inside a quarter u (sub-blocks 2u, 2u + 1, elements 64u .. 64u + 63
// of the super-block): MFMA chunk c is sub-block 2u + c, lane group q holds
// its positions 8q .. 8q + 7. A lane's weights for both chunks are the 8 qs
// bytes 32u + 8q .. + 7 (low nibbles chunk 0, high nibbles chunk 1); the
// activations of chunk c are elements 64u + 32c + 8q .. + 7, 16 contiguous
// bytes of the f16 image.
//
// LDS:
// - weights: the 256 rows' whole blocks of one super-block (144 bytes each,
//   row-major: the 144-byte row stride spreads 16 rows over distinct banks),
//   shared by both groups, two super-blocks deep. A row's block is contiguous
//   in HBM, so each 1 KB DMA instruction reads whole cache lines of about 7
//   rows instead of 16 bytes from each of 64;
// - activations: per group and step 128 tokens x 128 bytes (16-byte slot k of
//   token row t holds piece k ^ ((t >> 1) & 7), so the operand reads of 16
//   tokens hit 16 distinct bank groups), two steps deep;
// - per group the f16 (d*sc_j, dmin*m_j) of its four sub-blocks, 16 bytes per
//   row, each thread converting its own row's header once per super-block.
constexpr int kP8Blk = kPfRowsWg * kQ4kBytes;        // 36 KB: one super-block of 256 rows
constexpr int kP8Act = kPfTok * 128;                 // 16 KB: one group's activations of a step
constexpr int kP8ActOff = 2 * kP8Blk;                // activation buffers (group, step parity)
constexpr int kP8ScOff = kP8ActOff + 4 * kP8Act;     // scale records, 16 bytes per row per group
constexpr int kP8Lds = kP8ScOff + 2 * kPfRowsWg * 16;  // 144 KB
constexpr int kP8WPieces = kP8Blk / 1024;            // 36 weight DMA instructions per super-block
static_assert(kP8WPieces <= 40, "at most five weight DMA instructions per wavefront");
static_assert(2 * 4 * 16 * 64 * 16 <= kP8Lds, "the epilogue's exchange fits");

// LDS byte address of a pointer into a __shared__ array
__device__ __forceinline__ uint32_t p8_lds(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p;
}
// 16 bytes per lane from global to LDS: lane i copies base + voff_i to LDS
// address lds + 16 i (base and lds uniform). Written out by hand, so the
// compiler tracks no LDS write for it and inserts no wait for it: the
// kernel's own waits (p8_barrier_*) order every copy against its readers.
// The memory clobber keeps LDS accesses on their side of it; M0 is restored.
// base and lds are wave-uniform by construction; readfirstlane makes them
// scalar operands however the compiler placed them.
__device__ __forceinline__ void p8_dma(const void *base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(size_t)base;
    const uint64_t bs = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b) |
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32);
    const uint32_t ls = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(bs), "s"(ls)
                 : "memory");
}
// Wait for this wavefront's own copies except the newest n (n = 0 or 5) and
// for its LDS accesses, then the workgroup barrier.
__device__ __forceinline__ void p8_barrier_vm0() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void p8_barrier_vm5() {
    asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A GEMM workgroup's tile, K split and destination. A 3D grid (row tiles,
// token tiles, S) gives every tile S K splits: split z >= 1 stores its sums
// to slice z - 1 of `part` (n_tok x ld_out each), which k_prefill_sum adds
// into `out` in split order. A 1D grid (tail_s > 0; used when the tiles
// leave a last partial round of at most half the CUs) gives tiles 0 ..
// n_full - 1 (row tile fastest) one workgroup each and each later tile
// tail_s splits, split z of tail tile j at block n_full + j tail_s + z:
// split 0 stores to `out`, split z >= 1 to compact slice (z - 1) n_tail + j
// of `part` (kPfTok token rows of kPfRowsWg floats), which
// k_prefill_sum_tail adds in split order. The sums of token t, row o go to
// out[(t - t_org) ld + o - n_org].
struct PfTile {
    int n0, t0;  // first row, first token
    int z, nz;   // K split, splits of this tile
    float *out;
    int ld, t_org, n_org;
};
__device__ __forceinline__ PfTile pf_tile(float *out, float *part, int n_tok, int ld_out, int rt,
                                          int n_full, int tail_s) {
    PfTile p;
    if (tail_s == 0) {
        p.n0 = blockIdx.x * kPfRowsWg;
        p.t0 = blockIdx.y * kPfTok;
        p.z = blockIdx.z;
        p.nz = gridDim.z;
        p.out = p.z > 0 ? part + (size_t)(p.z - 1) * n_tok * ld_out : out;
        p.ld = ld_out;
        p.t_org = p.n_org = 0;
        return p;
    }
    const int b = blockIdx.x;
    int tile = b;
    p.z = 0;
    p.nz = 1;
    if (b >= n_full) {
        const int j = (b - n_full) / tail_s;
        tile = n_full + j;
        p.z = b - n_full - j * tail_s;
        p.nz = tail_s;
    }
    p.n0 = tile % rt * kPfRowsWg;
    p.t0 = tile / rt * kPfTok;
    p.out = out;
    p.ld = ld_out;
    p.t_org = p.n_org = 0;
    if (p.z > 0) {
        const int n_tail = ((int)gridDim.x - n_full) / tail_s;
        p.out = part + ((size_t)(p.z - 1) * n_tail + (tile - n_full)) * (kPfTok * kPfRowsWg);
        p.ld = kPfRowsWg;
        p.t_org = p.t0;
        p.n_org = p.n0;
    }
    return p;
}

// The end of an 8-wavefront workgroup (256 rows x 128 tokens, two K groups
// holding partial sums of the same outputs): group kg keeps token tiles
// 4 kg .. 4 kg + 3 and hands the other four to the partner wavefront (same
// rows, other group) through LDS (128 KB of the kernel's LDS, free once every
// copy has landed and every stage read is done); each lane then adds both
// groups' sums of its outputs, scales them by the token's 2^-e and stores
// them: lane (r16, q) holds outputs 16 nt + 4q .. + 3 of token 16 mt + r16.
// First pass (erow null): a lane that stores a non-finite value raises
// *flag. Second pass: output o of row r is scaled by 2^(erow[r] - e_t) in
// one step (erow: the workgroup's 256 row exponents in LDS).
__device__ __forceinline__ void p8_epilogue(f4 (&acc)[8][4], uint8_t *smem, int kg, int wr,
                                            int lane, int n0, int t0, const PfTile &tile,
                                            const float *unscale, int n_tok, int out_dim,
                                            const int *erow, int *flag) {
    const int r16 = lane & 15, q = lane >> 4;
    p8_barrier_vm0();
    f4 *xch = reinterpret_cast<f4 *>(smem);
    auto xidx = [=](int g, int i) { return ((g * 4 + wr) * 16 + i) * 64 + lane; };
    if (kg == 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) xch[xidx(0, i)] = acc[4 + (i >> 2)][i & 3];
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) xch[xidx(1, i)] = acc[i >> 2][i & 3];
    }
    __syncthreads();
    f4 res[4][4];
    if (kg == 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) res[i >> 2][i & 3] = acc[i >> 2][i & 3] + xch[xidx(1, i)];
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) res[i >> 2][i & 3] = acc[4 + (i >> 2)][i & 3] + xch[xidx(0, i)];
    }
    const int ow = n0 + 64 * wr + 4 * q;
    float *const out = tile.out;
    const int ld_out = tile.ld;
    const bool vec = ((out_dim | ld_out) & 3) == 0 && ((uintptr_t)out & 15) == 0;
    bool bad = false;  // a stored value is inf or NaN
#pragma unroll
    for (int ml = 0; ml < 4; ml++) {
        const int t = t0 + 16 * (4 * kg + ml) + r16;
        if (t >= n_tok) continue;
        const float us = unscale[t];
        float *orow = out + (size_t)(t - tile.t_org) * ld_out;
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int o = ow + 16 * nt;
            f4 v = res[ml][nt] * us;
            if (erow) {
                // us = 2^-e_t exactly (a normal power of two)
                const int eu = (int)((__float_as_uint(us) >> 23) & 0xFFu) - 127;
                const int lr = 64 * wr + 16 * nt + 4 * q;
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = ldexpf(res[ml][nt][i], erow[lr + i] + eu);
            }
            const int oc = o - tile.n_org;  // column in the destination
            if (vec && o + 3 < out_dim) {
                *reinterpret_cast<f4 *>(orow + oc) = v;
                if (!erow)
                    bad |= !(__builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) &&
                             __builtin_isfinite(v[2]) && __builtin_isfinite(v[3]));
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (o + i < out_dim) {
                        orow[oc + i] = v[i];
                        if (!erow) bad |= !__builtin_isfinite(v[i]);
                    }
            }
        }
    }
    if (bad) *flag = 1;
}

template <int PAR, bool MORE, bool SCALED = false> struct p8_step {
    static constexpr int par = PAR;         // step parity within the super-block
    static constexpr bool more = MORE;      // a next step exists
    static constexpr bool scaled = SCALED;  // a second pass: row exponents apply
};

// Between the passes of a GEMM workgroup: every stored value is checked and
// every stage read; returns whether any was inf or NaN (uniform).
__device__ __forceinline__ bool pf_again(const int *flag) {
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*flag) != 0;
}

//
// K split: split z of a tile's S covers super-blocks [z nbt / S, (z + 1)
// nbt / S) of the nbt in a row and stores its sums where pf_tile says.
__global__ __launch_bounds__(512) void k_prefill_q4k_w8(const uint8_t *__restrict__ w_arg,
                                                        const _Float16 *__restrict__ xh_arg,
                                                        const float *__restrict__ unscale,
                                                        float *__restrict__ out_arg,
                                                        float *__restrict__ part, int n_tok,
                                                        int in_dim, int out_dim, int ld_out,
                                                        int rt, int n_full, int tail_s) {
    __shared__ __align__(16) uint8_t smem[kP8Lds + kPfGuardBytes];
    // range guard: the workgroup's flag, its rows' exponents (after the
    // stages)
    int *const flag = reinterpret_cast<int *>(smem + kP8Lds);
    int *const erow_lds = flag + 4;
    if (threadIdx.x == 0) *flag = 0;  // before the prologue's barrier
    // one pass of the workgroup: setup, the tile, the epilogue
    auto body = [&](auto pass_c) __attribute__((always_inline)) {
        int erow = 0;  // this thread's scale row's exponent (0 in the first pass)
        // the second pass re-derives every per-lane value from an opaque copy
        // of the thread index, so none of the first pass's stays live across
        // its epilogue
        int tid = threadIdx.x;
        if constexpr (decltype(pass_c)::value) asm volatile("" : "+v"(tid));
        const int lane = tid & 63;
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wr = wv & 3, kg = wv >> 2;
        const int r16 = lane & 15, q = lane >> 4;
        const PfTile tile = pf_tile(out_arg, part, n_tok, ld_out, rt, n_full, tail_s);
        const int n0 = tile.n0, t0 = tile.t0;
        const int nbt = in_dim >> 8;  // super-blocks in a row
        const int z = tile.z, nz = tile.nz;
        const int kb0 = (int)((long)z * nbt / nz);
        const int nb = (int)((long)(z + 1) * nbt / nz) - kb0;  // super-blocks of this split (>= 1)
        const int ns = 2 * nb;                                 // steps of one K group
        // this K split's weights and activations (the arguments stay
        // unchanged for the second pass)
        const uint8_t *const w = w_arg + (size_t)kb0 * kQ4kBytes;
        const _Float16 *const xh = xh_arg + (size_t)kb0 * 256;
        uint8_t *const act = smem + kP8ActOff + 2 * kg * kP8Act;  // this group's two step buffers
        uint8_t *const scl = smem + kP8ScOff + kg * kPfRowsWg * 16;
        const uint32_t row_bytes = (uint32_t)nbt * (uint32_t)kQ4kBytes;

        // DMA sources (bytes from a uniform base). Activations: instruction p
        // moves token rows 8 (4 wr + p) .. + 7 of this group's quarter, lane i to
        // row 8 (4 wr + p) + i / 8, slot i % 8. Rows past n_tok repeat the last
        // token (their outputs are not stored).
        uint32_t xoff[4];
    #pragma unroll
        for (int p = 0; p < 4; p++) {
            const int tl = 8 * (4 * wr + p) + (lane >> 3);
            const int pc = (lane & 7) ^ ((tl >> 1) & 7);
            const int t = min(t0 + tl, n_tok - 1);
            xoff[p] = 2u * ((uint32_t)t * (uint32_t)in_dim + 64 * kg + 32 * (pc >> 2) + 8 * (pc & 3));
        }
        // Weights: instruction i = wv + 8k moves 16-byte pieces j = 64 i + lane of
        // the stage, row j / 9, piece j % 9. Instructions past the last repeat it
        // (same bytes to the same place), so every wavefront issues five.
        uint32_t woff[5];
    #pragma unroll
        for (int k = 0; k < 5; k++) {
            const int i = min(wv + 8 * k, kP8WPieces - 1);
            const int j = 64 * i + lane, row = j / 9;
            woff[k] = (uint32_t)min(n0 + row, out_dim - 1) * row_bytes + 16u * (uint32_t)(j % 9);
        }
        const uint32_t lds_act = p8_lds(act), lds_w = p8_lds(smem);
        // piece p of group step s (clamped to the last) into the buffer of step parity s % 2
        auto dma_act = [&](int s, int p) {
            const uint32_t dst = lds_act + (uint32_t)((s & 1) * kP8Act + 1024 * (4 * wr + p));
            s = min(s, ns - 1);
            p8_dma(xh + (s >> 1) * 256 + 128 * (s & 1), xoff[p], dst);
        };
        // piece k of super-block sb (clamped to the last) into weight stage sb % 2
        auto dma_w = [&](int sb, int k) {
            const uint32_t dst = lds_w + (uint32_t)((sb & 1) * kP8Blk + 1024 * min(wv + 8 * k, kP8WPieces - 1));
            sb = min(sb, nb - 1);
            p8_dma(w + (size_t)sb * kQ4kBytes, woff[k], dst);
        };
        // header of this thread's row in a weight stage -> scale records of the
        // group's four sub-blocks: 16 bytes, {d*sc, d*sc'} {dmin*m, dmin*m'} for
        // the even step (sub-blocks 2 kg, 2 kg + 1), then for the odd step (4 +
        // 2 kg, 5 + 2 kg) (q4_k_scale_min, dequant/mod.rs:48-58)
        auto scales_from_header = [&](const uint8_t *wbuf, auto scaled_c) {
            const int row = 64 * wr + lane;
            const uint4 hd = *reinterpret_cast<const uint4 *>(wbuf + kQ4kBytes * row);
            float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
            if constexpr (decltype(scaled_c)::value) {
                d = ldexpf(d, -erow);
                dmin = ldexpf(dmin, -erow);
            }
            const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, m_lo = hd.z & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
            const int b = 16 * kg;  // bit offset of byte 2 kg
            uint32_t rec[4];
    #pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const uint32_t sw = (hf ? sc_hi : sc_lo) >> b, mw = (hf ? m_hi : m_lo) >> b;
                const _Float16 a0 = (_Float16)(d * (float)(sw & 0xFFu));
                const _Float16 a1 = (_Float16)(d * (float)((sw >> 8) & 0xFFu));
                const _Float16 m0 = (_Float16)(dmin * (float)(mw & 0xFFu));
                const _Float16 m1 = (_Float16)(dmin * (float)((mw >> 8) & 0xFFu));
                rec[2 * hf] = __builtin_bit_cast(uint32_t, h2{a0, a1});
                rec[2 * hf + 1] = __builtin_bit_cast(uint32_t, h2{m0, m1});
            }
            *reinterpret_cast<uint4 *>(scl + 16 * row) = make_uint4(rec[0], rec[1], rec[2], rec[3]);
        };
        const int qbyte = 16 + 32 * kg + 8 * q;  // the lane's qs bytes in a block, step parity 0
        const int aswz = (r16 >> 1) & 7;
        // this lane's qs bytes and scale records of row tile nt at step parity hf
        uint2 qs[4], sc[4];
        auto load_weights = [&](const uint8_t *wbuf, int hf) {
    #pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const int row = 64 * wr + 16 * nt + r16;
                qs[nt] = *reinterpret_cast<const uint2 *>(wbuf + kQ4kBytes * row + qbyte + 64 * hf);
                sc[nt] = *reinterpret_cast<const uint2 *>(scl + 16 * row + 8 * hf);
            }
        };
        auto dequant = [&](int c, int nt) -> h8 {
            const h2 d2 = __builtin_bit_cast(h2, sc[nt].x), m2 = __builtin_bit_cast(h2, sc[nt].y);
            return pf_dequant8(qs[nt].x, qs[nt].y, c != 0, c ? d2.yy : d2.xx, c ? m2.yy : m2.xx);
        };
        auto read_a = [&](const uint8_t *buf, int c, int mt) -> h8 {
            return *reinterpret_cast<const h8 *>(buf + (16 * mt + r16) * 128 + 16 * ((4 * c + q) ^ aswz));
        };

        f4 acc[8][4];
        h8 bq[4], a0, a1;

        // One step s (super-block sb = s / 2, step parity PAR = s % 2): 16 groups
        // (2 chunks x 8 token tiles) of 4 MFMAs. Operand reads run two groups
        // ahead, across the step boundary; chunk 1's weights are dequantised
        // during chunk 0, the next step's chunk 0 in groups 14, 15. In group 14
        // every wavefront has this step's operands in registers and waits for
        // its own copies the next step needs (its activations; on the last step
        // of a super-block also the next super-block's weights): after the
        // barrier those are readable, this step's activation buffer takes step
        // s + 2 (groups 14, 15), and after the last step of a super-block its
        // weight stage takes super-block sb + 2 (groups 1, 3, .., 9 of the next
        // step; super-block 1 in step 0). The weight copies are issued after the
        // activation copies of the step after, so an even step waits only for the
        // older activation pieces (vmcnt(5)).
        auto step = [&](int s, auto tag) __attribute__((always_inline)) {
            constexpr int PAR = decltype(tag)::par;
            constexpr bool MORE = decltype(tag)::more;
            const int sb = s >> 1;
            const uint8_t *buf = act + PAR * kP8Act;
            const uint8_t *nbuf = act + (1 - PAR) * kP8Act;
            h8 b1[4];
    #pragma unroll
            for (int g = 0; g < 16; g++) {
                const int c = g >> 3, mt = g & 7;
                __builtin_amdgcn_sched_barrier(0);
                if (MORE && PAR == 0 && (g & 1) && g < 10) dma_w(sb + 1, g >> 1);
                if (MORE && g == 14) {
                    if (PAR) p8_barrier_vm0();
                    else p8_barrier_vm5();
                    if (PAR)
                        scales_from_header(smem + ((sb + 1) & 1) * kP8Blk,
                                           std::integral_constant<bool, decltype(tag)::scaled>{});
                    load_weights(smem + ((sb + PAR) & 1) * kP8Blk, 1 - PAR);
                }
                h8 a2 = a1;
                if (g + 2 < 16) a2 = read_a(buf, (g + 2) >> 3, (g + 2) & 7);
                else if (MORE) a2 = read_a(nbuf, 0, g - 14);
                if (MORE && g >= 14) {
                    dma_act(s + 2, 2 * (g - 14));
                    dma_act(s + 2, 2 * (g - 14) + 1);
                }
                const h8 acur = a0;
                const h8 *bw = c ? b1 : bq;
    #pragma unroll
                for (int nt = 0; nt < 4; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bw[nt], acur, acc[mt][nt], 0, 0, 0);
                if (c == 0 && (mt & 1)) b1[mt >> 1] = dequant(1, mt >> 1);
                if (MORE && g >= 14) {
                    bq[2 * (g - 14)] = dequant(0, 2 * (g - 14));
                    bq[2 * (g - 14) + 1] = dequant(0, 2 * (g - 14) + 1);
                }
                a0 = a1;
                a1 = a2;
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        if constexpr (decltype(pass_c)::value) {
            // E of this thread's scale row from its blocks' bounds
            // E of this thread's scale row from its blocks' bounds
            const int r = min(n0 + 64 * wr + lane, out_dim - 1);
            const uint8_t *hp = w + (size_t)r * row_bytes;
            float m = 0.f;
            for (int b = 0; b < nb; b++) {
                const uint32_t h = *reinterpret_cast<const uint32_t *>(hp + (size_t)b * kQ4kBytes);
                m = fmaxf(m, 945.f * fabsf(f16_to_f32(h & 0xFFFFu)) + 63.f * fabsf(f16_to_f32(h >> 16)));
            }
            erow = pf_row_exponent(m);
            if (kg == 0) erow_lds[64 * wr + lane] = erow;
        }
        // one pass over the tile: the first with E = 0, a second (scaled) with
        // this thread's row exponent erow
        auto run = [&](auto scaled_c) __attribute__((always_inline)) {
            constexpr bool SC = decltype(scaled_c)::value;
    #pragma unroll
            for (int mt = 0; mt < 8; mt++)
    #pragma unroll
                for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

            // prologue: super-block 0 and step 0 in, step 1 in flight, step 0's
            // chunk-0 operands ready
    #pragma unroll
            for (int k = 0; k < 5; k++) dma_w(0, k);
    #pragma unroll
            for (int p = 0; p < 4; p++) dma_act(0, p);
            p8_barrier_vm0();
    #pragma unroll
            for (int p = 0; p < 4; p++) dma_act(1, p);  // ns >= 2; super-block 1 in step 0
            scales_from_header(smem, scaled_c);
            load_weights(smem, 0);
    #pragma unroll
            for (int nt = 0; nt < 4; nt++) bq[nt] = dequant(0, nt);
            a0 = read_a(act, 0, 0);
            a1 = read_a(act, 0, 1);

            for (int sb = 0; sb + 1 < nb; sb++) {
                step(2 * sb, p8_step<0, true, SC>{});
                step(2 * sb + 1, p8_step<1, true, SC>{});
            }
            step(ns - 2, p8_step<0, true, SC>{});
            step(ns - 1, p8_step<1, false, SC>{});
        };
        run(pass_c);
        if constexpr (!decltype(pass_c)::value)
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, nullptr, flag);
        else
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, erow_lds,
                        nullptr);
    };
    body(std::false_type{});
    if (pf_again(flag)) body(std::true_type{});
}

// ---- Q8_0 weights ----------------------------------------------------------------
// k_prefill_q8_w8: the workgroup of k_prefill_q4k_w8 (256 rows x 128 tokens,
// 8 wavefronts, two K groups on alternate quarters of each 256 elements, the
// same activation stages, epilogue and K split) on Q8_0 weights in this
// backend's device layout: super-tiles of 8 blocks [qs 8 x 32 | d 8 x 2], 272
// bytes per 256 elements of a row. A super-tile of 256 rows is 68 KB, too
// large to keep two beside the activations, so the weights are staged per
// K-group step with the activations: the quarter's two blocks' qs (64 bytes
// per row; the four 16-byte pieces of row r in slot p ^ ((r >> 2) & 3), so
// the operand reads of 16 rows hit distinct banks) and the row's 16-byte d
// run. Chunk c of quarter u is block 2u + c; lane group q holds its bytes
// 8q .. 8q + 7. w = f16(d * q): the byte ^ 0x80 paired with 0x64 is
// 1152 + q exactly in f16, minus 1152 leaves q, and one multiply by the f16
// d rounds once (about 2^-11 relative, as the Q4_K weights).
constexpr int kQ8Qs = kPfRowsWg * 64;            // 16 KB
constexpr int kQ8D = kPfRowsWg * 16;             // 4 KB
constexpr int kQ8Stage = kP8Act + kQ8Qs + kQ8D;  // 36 KB per group step
constexpr int kQ8Lds = 4 * kQ8Stage;             // 144 KB
static_assert(2 * 4 * 16 * 64 * 16 <= kQ8Lds, "the epilogue's exchange fits");

__global__ __launch_bounds__(512) void k_prefill_q8_w8(const uint8_t *__restrict__ w_arg,
                                                       const _Float16 *__restrict__ xh_arg,
                                                       const float *__restrict__ unscale,
                                                       float *__restrict__ out_arg,
                                                       float *__restrict__ part, int n_tok,
                                                       int in_dim, int out_dim, int ld_out,
                                                       int rt, int n_full, int tail_s) {
    __shared__ __align__(16) uint8_t smem[kQ8Lds + kPfGuardBytes];
    // range guard: the workgroup's flag, its rows' exponents (after the
    // stages)
    int *const flag = reinterpret_cast<int *>(smem + kQ8Lds);
    int *const erow_lds = flag + 4;
    if (threadIdx.x == 0) *flag = 0;  // before the prologue's barrier
    // one pass of the workgroup: setup, the tile, the epilogue
    auto body = [&](auto pass_c) __attribute__((always_inline)) {
        int erow = 0;  // this thread's scale row's exponent (0 in the first pass)
        // the second pass re-derives every per-lane value from an opaque copy
        // of the thread index, so none of the first pass's stays live across
        // its epilogue
        int tid = threadIdx.x;
        if constexpr (decltype(pass_c)::value) asm volatile("" : "+v"(tid));
        const int lane = tid & 63;
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wr = wv & 3, kg = wv >> 2;
        const int r16 = lane & 15, q = lane >> 4;
        const PfTile tile = pf_tile(out_arg, part, n_tok, ld_out, rt, n_full, tail_s);
        const int n0 = tile.n0, t0 = tile.t0;
        const int nbt = in_dim >> 8;  // super-tiles in a row
        const int z = tile.z, nz = tile.nz;
        const int kb0 = (int)((long)z * nbt / nz);
        const int nb = (int)((long)(z + 1) * nbt / nz) - kb0;
        const int ns = 2 * nb;
        // this K split's weights and activations (the arguments stay
        // unchanged for the second pass)
        const uint8_t *const w = w_arg + (size_t)kb0 * 272;
        const _Float16 *const xh = xh_arg + (size_t)kb0 * 256;
        uint8_t *const stg = smem + 2 * kg * kQ8Stage;  // this group's two step buffers
        const uint32_t row_bytes = (uint32_t)nbt * 272u;

        // DMA sources (bytes from a uniform base). Activations as in
        // k_prefill_q4k_w8. qs: instruction p moves rows 16 (4 wr + p) .. + 15,
        // lane i to row 16 (4 wr + p) + i / 4, slot i % 4 (holding piece
        // (i % 4) ^ ((row >> 2) & 3) of the quarter's 64 bytes). d: lane i moves
        // row 64 wr + i's 16-byte d run. Both cover exactly this wavefront's rows.
        uint32_t xoff[4], qoff[4];
    #pragma unroll
        for (int p = 0; p < 4; p++) {
            const int tl = 8 * (4 * wr + p) + (lane >> 3);
            const int pc = (lane & 7) ^ ((tl >> 1) & 7);
            const int t = min(t0 + tl, n_tok - 1);
            xoff[p] = 2u * ((uint32_t)t * (uint32_t)in_dim + 64 * kg + 32 * (pc >> 2) + 8 * (pc & 3));
            const int row = 16 * (4 * wr + p) + (lane >> 2);
            const int piece = (lane & 3) ^ ((row >> 2) & 3);
            qoff[p] = (uint32_t)min(n0 + row, out_dim - 1) * row_bytes + 64u * kg + 16u * piece;
        }
        const uint32_t doff = (uint32_t)min(n0 + 64 * wr + lane, out_dim - 1) * row_bytes + 256u;
        const uint32_t lds_stg = p8_lds(stg);
        // piece p (0..8) of group step s (clamped to the last) into the buffer of
        // step parity s % 2: 0..3 activations, 4..7 qs, 8 the d run
        auto dma = [=](int s, int p) {
            const uint32_t buf = lds_stg + (uint32_t)((s & 1) * kQ8Stage);
            s = min(s, ns - 1);
            const int sb = s >> 1, hf = s & 1;
            if (p < 4)
                p8_dma(xh + sb * 256 + 128 * hf, xoff[p], buf + 1024 * (4 * wr + p));
            else if (p < 8)
                p8_dma(w + (size_t)sb * 272 + 128 * hf, qoff[p - 4], buf + kP8Act + 1024 * (4 * wr + p - 4));
            else
                p8_dma(w + (size_t)sb * 272, doff, buf + kP8Act + kQ8Qs + 1024 * wr);
        };
        const int sw = (r16 >> 2) & 3;
        const int qb0 = 16 * ((q >> 1) ^ sw) + 8 * (q & 1);        // chunk 0: piece q / 2
        const int qb1 = 16 * ((2 + (q >> 1)) ^ sw) + 8 * (q & 1);  // chunk 1: piece 2 + q / 2
        const int aswz = (r16 >> 1) & 7;
        uint2 qs0[4], qs1[4];
        uint32_t dd[4];  // f16 d of blocks 2u, 2u + 1
        auto load_weights = [&](const uint8_t *buf, int hf) {
    #pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const int row = 64 * wr + 16 * nt + r16;
                qs0[nt] = *reinterpret_cast<const uint2 *>(buf + kP8Act + 64 * row + qb0);
                qs1[nt] = *reinterpret_cast<const uint2 *>(buf + kP8Act + 64 * row + qb1);
                dd[nt] = *reinterpret_cast<const uint32_t *>(buf + kP8Act + kQ8Qs + 16 * row +
                                                             4 * (2 * hf + kg));
            }
        };
        auto dequant = [&](int c, int nt) -> h8 {
            const uint2 b = c ? qs1[nt] : qs0[nt];
            const h2 d2 = __builtin_bit_cast(h2, dd[nt]);
            const h2 ds = c ? d2.yy : d2.xx;
            const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
            h8 r;
    #pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t bb = (u ? b.y : b.x) ^ 0x80808080u;
                const h2 w01 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, bb, 0x04010400u)) - bias) * ds;
                const h2 w23 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, bb, 0x04030402u)) - bias) * ds;
                r[4 * u] = w01[0];
                r[4 * u + 1] = w01[1];
                r[4 * u + 2] = w23[0];
                r[4 * u + 3] = w23[1];
            }
            return r;
        };
        // second pass: the two d of this thread's row (64 wr + lane) that its
        // group uses in the step held in buf (parity hf) are rewritten in place
        // as f16(d 2^-E); the readers of that dword are lanes of this wavefront
        auto scale_d = [&](uint8_t *buf, int hf) {
            uint32_t *dp = reinterpret_cast<uint32_t *>(buf + kP8Act + kQ8Qs + 16 * (64 * wr + lane) +
                                                        4 * (2 * hf + kg));
            const uint32_t dv = *dp;
            const h2 sd = {(_Float16)ldexpf(f16_to_f32(dv & 0xFFFFu), -erow),
                           (_Float16)ldexpf(f16_to_f32(dv >> 16), -erow)};
            *dp = __builtin_bit_cast(uint32_t, sd);
        };
        auto read_a = [&](const uint8_t *buf, int c, int mt) -> h8 {
            return *reinterpret_cast<const h8 *>(buf + (16 * mt + r16) * 128 + 16 * ((4 * c + q) ^ aswz));
        };

        f4 acc[8][4];
        h8 bq[4], a0, a1;

        // One step: as in k_prefill_q4k_w8, with the weights in the step's
        // buffer: in group 14 every wavefront waits for its own copies of step
        // s + 1, after the barrier reads that step's weights and first operands,
        // and this step's buffer takes step s + 2 (pieces 0..5 in groups 14, 15,
        // 6..8 in groups 0, 2, 4 of the next step).
        auto step = [&](int s, auto tag) __attribute__((always_inline)) {
            constexpr int PAR = decltype(tag)::par;
            constexpr bool MORE = decltype(tag)::more;
            const uint8_t *buf = stg + PAR * kQ8Stage;
            const uint8_t *nbuf = stg + (1 - PAR) * kQ8Stage;
            h8 b1[4];
    #pragma unroll
            for (int g = 0; g < 16; g++) {
                const int c = g >> 3, mt = g & 7;
                __builtin_amdgcn_sched_barrier(0);
                if (MORE && g < 6 && (g & 1) == 0 && s >= 1) dma(s + 1, 6 + (g >> 1));
                if (MORE && g == 14) {
                    p8_barrier_vm0();
                    if constexpr (decltype(tag)::scaled) scale_d(const_cast<uint8_t *>(nbuf), 1 - PAR);
                    load_weights(nbuf, 1 - PAR);
                }
                h8 a2 = a1;
                if (g + 2 < 16) a2 = read_a(buf, (g + 2) >> 3, (g + 2) & 7);
                else if (MORE) a2 = read_a(nbuf, 0, g - 14);
                if (MORE && g >= 14) {
                    dma(s + 2, 3 * (g - 14));
                    dma(s + 2, 3 * (g - 14) + 1);
                    dma(s + 2, 3 * (g - 14) + 2);
                }
                const h8 acur = a0;
                const h8 *bw = c ? b1 : bq;
    #pragma unroll
                for (int nt = 0; nt < 4; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bw[nt], acur, acc[mt][nt], 0, 0, 0);
                if (c == 0 && (mt & 1)) b1[mt >> 1] = dequant(1, mt >> 1);
                if (MORE && g >= 14) {
                    bq[2 * (g - 14)] = dequant(0, 2 * (g - 14));
                    bq[2 * (g - 14) + 1] = dequant(0, 2 * (g - 14) + 1);
                }
                a0 = a1;
                a1 = a2;
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        if constexpr (decltype(pass_c)::value) {
            // E of this thread's scale row from its blocks' bounds
            const int r = min(n0 + 64 * wr + lane, out_dim - 1);
            const uint8_t *rp = w + (size_t)r * row_bytes + 256;  // the d run of super-tile 0
            float m = 0.f;
            for (int b = 0; b < nb; b++) {
                const uint4 dr = *reinterpret_cast<const uint4 *>(rp + (size_t)b * 272);
                const uint32_t dw[4] = {dr.x, dr.y, dr.z, dr.w};
    #pragma unroll
                for (int i = 0; i < 4; i++)
                    m = fmaxf(m, 128.f * fmaxf(fabsf(f16_to_f32(dw[i] & 0xFFFFu)),
                                               fabsf(f16_to_f32(dw[i] >> 16))));
            }
            erow = pf_row_exponent(m);
            if (kg == 0) erow_lds[64 * wr + lane] = erow;
        }
        // one pass over the tile: the first with E = 0, a second (scaled) with
        // this thread's row exponent erow
        auto run = [&](auto scaled_c) __attribute__((always_inline)) {
            constexpr bool SC = decltype(scaled_c)::value;
    #pragma unroll
            for (int mt = 0; mt < 8; mt++)
    #pragma unroll
                for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

            // prologue: step 0 in, step 1 in flight, step 0's chunk-0 operands ready
    #pragma unroll
            for (int p = 0; p < 9; p++) dma(0, p);
            p8_barrier_vm0();
    #pragma unroll
            for (int p = 0; p < 9; p++) dma(1, p);  // ns >= 2
            if constexpr (SC) scale_d(stg, 0);
            load_weights(stg, 0);
    #pragma unroll
            for (int nt = 0; nt < 4; nt++) bq[nt] = dequant(0, nt);
            a0 = read_a(stg, 0, 0);
            a1 = read_a(stg, 0, 1);

            for (int sb = 0; sb + 1 < nb; sb++) {
                step(2 * sb, p8_step<0, true, SC>{});
                step(2 * sb + 1, p8_step<1, true, SC>{});
            }
            step(ns - 2, p8_step<0, true, SC>{});
            step(ns - 1, p8_step<1, false, SC>{});
        };
        run(pass_c);
        if constexpr (!decltype(pass_c)::value)
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, nullptr, flag);
        else
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, erow_lds,
                        nullptr);
    };
    body(std::false_type{});
    if (pf_again(flag)) body(std::true_type{});
}

// ---- Q6_K weights -----------------------------------------------------------------
// k_prefill_q6_w8: the same workgroup on Q6_K weights in the device layout
// (super-tiles of 8 blocks [ql 8 x 128 | qh 8 x 64 | scales 8 x 16 | d 8 x 2],
// 1680 bytes per 2048 elements of a row; rows of whole super-tiles, in_dim a
// multiple of 2048). Element 128 h + 32 j + l of a block (q6_k.rs:65-92) is
// the low (j < 2) or high nibble of ql[64 h + 32 (j & 1) + l] with bits 2j,
// 2j + 1 of qh[32 h + l] above it, minus 32, times d * sc[8 h + 2 j + l / 16].
// Group kg's step at half h takes j = 2 kg + c for its chunks c, so both
// groups read the same half-block in a step: one weight stage per step,
// shared by the 8 wavefronts, 128 bytes per row (the half's 64 ql and 32 qh
// bytes, the block's 16 scales, the super-tile's 16-byte d run), its 16-byte
// slot s of row r at slot s ^ ((r & 15) >> 1) so the 8-byte operand reads of
// 16 rows hit distinct banks. Each thread turns its own row's scales into
// f16 (d * sc) for its group once per step. Lane group q's 8 weights of a
// chunk: the 6-bit codes (ql nibble | qh bits << 4), paired with 0x64 as
// f16 1024 + code, minus 1056 (exact q - 32), times f16(d * sc) (one
// rounding, as the Q4_K weights).
constexpr int kQ6W = kPfRowsWg * 128;              // 32 KB: a step's weight stage
constexpr int kQ6ActOff = 2 * kQ6W;                // activations: (group, step parity)
constexpr int kQ6ScOff = kQ6ActOff + 4 * kP8Act;   // scale records: 8 bytes per row per group
constexpr int kQ6Lds = kQ6ScOff + 2 * kPfRowsWg * 8;  // 132 KB
static_assert(2 * 4 * 16 * 64 * 16 <= kQ6Lds, "the epilogue's exchange fits");

__global__ __launch_bounds__(512) void k_prefill_q6_w8(const uint8_t *__restrict__ w,
                                                       const _Float16 *__restrict__ xh_arg,
                                                       const float *__restrict__ unscale,
                                                       float *__restrict__ out_arg,
                                                       float *__restrict__ part, int n_tok,
                                                       int in_dim, int out_dim, int ld_out,
                                                       int rt, int n_full, int tail_s) {
    __shared__ __align__(16) uint8_t smem[kQ6Lds + kPfGuardBytes];
    // range guard: the workgroup's flag, its rows' exponents (after the
    // stages)
    int *const flag = reinterpret_cast<int *>(smem + kQ6Lds);
    int *const erow_lds = flag + 4;
    if (threadIdx.x == 0) *flag = 0;  // before the prologue's barrier
    // one pass of the workgroup: setup, the tile, the epilogue
    auto body = [&](auto pass_c) __attribute__((always_inline)) {
        int erow = 0;  // this thread's scale row's exponent (0 in the first pass)
        // the second pass re-derives every per-lane value from an opaque copy
        // of the thread index, so none of the first pass's stays live across
        // its epilogue
        int tid = threadIdx.x;
        if constexpr (decltype(pass_c)::value) asm volatile("" : "+v"(tid));
        const int lane = tid & 63;
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wr = wv & 3, kg = wv >> 2;
        const int r16 = lane & 15, q = lane >> 4;
        const PfTile tile = pf_tile(out_arg, part, n_tok, ld_out, rt, n_full, tail_s);
        const int n0 = tile.n0, t0 = tile.t0;
        const int nbt = in_dim >> 8;  // blocks in a row (a multiple of 8)
        const int z = tile.z, nz = tile.nz;
        const int kb0 = (int)((long)z * nbt / nz);
        const int nb = (int)((long)(z + 1) * nbt / nz) - kb0;
        const int ns = 2 * nb;
        // this K split's activations (the arguments stay unchanged for the
        // second pass)
        const _Float16 *const xh = xh_arg + (size_t)kb0 * 256;
        uint8_t *const act = smem + kQ6ActOff + 2 * kg * kP8Act;  // this group's two step buffers
        uint8_t *const scl = smem + kQ6ScOff + kg * kPfRowsWg * 8;
        const uint32_t row_bytes = (uint32_t)(nbt >> 3) * 1680u;

        // Copies, 16 bytes a lane, lane l to LDS row 8 R + l / 8 (a token of
        // this group's activations, a weight row of the stage), 16-byte slot
        // l % 8. Piece p of wavefront (wr or wv) covers R = 2 (4 (w >> 1) + p) +
        // (w & 1), so a row's swizzle ((row & 15) >> 1 = 4 (w & 1) + l / 16), and
        // with it what a lane copies, is the same for all four pieces: a column
        // piece of the activations; for the weights field slot f = (l % 8) ^
        // swizzle (0..3 ql, 4..5 qh, 6 the scales, 7 the d run) at byte
        // base(f) + (b % 8) stride(f) + h half(f) of the super-tile of block b, h
        // the half-block. Rows past the matrix repeat its last row: the row
        // offset is min(l / 8, lim) rows from a clamped first row, lim passed
        // through an empty asm at each copy so the compiler keeps no per-piece
        // offsets in registers.
        const int lr = lane >> 3;
        const int aswz_dma = 4 * (wr & 1) + (lane >> 4), wswz_dma = 4 * (wv & 1) + (lane >> 4);
        const int pc = (lane & 7) ^ aswz_dma;
        const uint32_t xcol = 2u * (64 * kg + 32 * (pc >> 2) + 8 * (pc & 3));
        const int f = (lane & 7) ^ wswz_dma;
        const uint32_t wfld = f < 4 ? 16u * f : f < 6 ? 1024u + 16u * (f - 4) : f == 6 ? 1536u : 1664u;
        const uint32_t wmul = (f < 4 ? 128u : f < 6 ? 64u : f == 6 ? 16u : 0u) |
                              ((f < 4 ? 64u : f < 6 ? 32u : 0u) << 16);  // stride | half << 16
        // this wavefront's first copy destinations, held in scalar registers
        // (from an asm result) so no vector register keeps them
        uint32_t lds_act, lds_w;
        asm("s_mov_b32 %0, %1"
            : "=s"(lds_act)
            : "s"(__builtin_amdgcn_readfirstlane(p8_lds(act) + 8192 * (wr >> 1) + 1024 * (wr & 1))));
        asm("s_mov_b32 %0, %1"
            : "=s"(lds_w)
            : "s"(__builtin_amdgcn_readfirstlane(p8_lds(smem) + 8192 * (wv >> 1) + 1024 * (wv & 1))));
        // piece p (0..7) of group step s into the buffers of step parity par
        // (s % 2, a constant at every call, so the half-block is one): 0..3 this
        // group's activations, 4..7 the shared weight stage. A step past the end
        // reloads the last block's half par, which no one reads.
        auto dma = [=](int s, int p, auto par_c) {
            constexpr int par = decltype(par_c)::value;
            const int b = kb0 + (min(s, ns - 1) >> 1);  // block of the row
            if (p < 4) {
                const int R = 2 * (4 * (wr >> 1) + p) + (wr & 1);
                const int t = min(t0 + 8 * R, n_tok - 1);
                int lim = n_tok - 1 - t;
                asm volatile("" : "+s"(lim));
                const uint32_t o = (uint32_t)min(lr, lim) * (2u * (uint32_t)in_dim) + xcol;
                p8_dma(xh + (size_t)t * in_dim + (b - kb0) * 256 + 128 * par, o,
                       lds_act + (uint32_t)(par * kP8Act + 2048 * p));
            } else {
                const int R = 2 * (4 * (wv >> 1) + p - 4) + (wv & 1);
                const int r = min(n0 + 8 * R, out_dim - 1);
                int lim = out_dim - 1 - r;
                asm volatile("" : "+s"(lim));
                uint32_t o = (uint32_t)min(lr, lim) * row_bytes + (uint32_t)(b & 7) * (wmul & 0xFFFFu) + wfld;
                if (par) o += wmul >> 16;
                p8_dma(w + (size_t)r * row_bytes + (size_t)(b >> 3) * 1680, o,
                       lds_w + (uint32_t)(par * kQ6W + 2048 * (p - 4)));
            }
        };
        using par0 = std::integral_constant<int, 0>;
        using par1 = std::integral_constant<int, 1>;
        const int sw = r16 >> 1;
        const int qlb0 = 16 * ((0 + (q >> 1)) ^ sw) + 8 * (q & 1);  // ql, chunk 0: field slot q / 2
        const int aswz = (r16 >> 1) & 7;
        // this thread's row's scales -> records for its group at half h:
        // {f16(d sc[8h + 4kg]), f16(d sc[8h + 4kg + 2])} for lane groups q < 2,
        // {f16(d sc[8h + 4kg + 1]), f16(d sc[8h + 4kg + 3])} for q >= 2
        auto scales_of_step = [&](const uint8_t *wbuf, int b, int h, auto scaled_c) {
            const int row = 64 * wr + lane;
            const int rs = (row & 15) >> 1;
            const uint32_t sc4 = *reinterpret_cast<const uint32_t *>(wbuf + 128 * row + 16 * (6 ^ rs) + 8 * h + 4 * kg);
            float d = f16_to_f32(*reinterpret_cast<const uint16_t *>(wbuf + 128 * row + 16 * (7 ^ rs) + 2 * (b & 7)));
            if constexpr (decltype(scaled_c)::value) d = ldexpf(d, -erow);
            auto f = [&](int i) { return (_Float16)(d * (float)(int8_t)(sc4 >> (8 * i))); };
            const h2 lo = {f(0), f(2)}, hi = {f(1), f(3)};
            *reinterpret_cast<uint2 *>(scl + 8 * row) =
                make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
        };
        // a lane's raw operands of chunk c, token tile nt: 8 ql bytes, the 8 qh
        // bytes, (f16 scale of chunk 0, of chunk 1)
        struct q6w {
            uint2 ql, qh;
            uint32_t sc;
        };
        // one per-lane base (row 64 wr + r16 of stage 0, the chunk-0 ql field):
        // the chunk-1 ql and the qh fields are at base ^ 32 and base ^ 64 (slots
        // q / 2 + 2 and + 4 under the swizzle), token tile nt and the stage are
        // immediate offsets. The empty asm at each use keeps the compiler from
        // holding the derived addresses in registers across the loop.
        const uint32_t wq_base = 128u * (uint32_t)(64 * wr + r16) + (uint32_t)qlb0;  // from smem
        const uint32_t ws_base = (uint32_t)(scl - smem) + 8u * (uint32_t)(64 * wr + r16) + 4u * (uint32_t)(q >> 1);
        auto read_w = [&](int par, int c, int nt) -> q6w {
            uint32_t a = wq_base, sa = ws_base;
            asm volatile("" : "+v"(a), "+v"(sa));
            const uint32_t o = (uint32_t)par * kQ6W + 2048u * nt;
            return {*reinterpret_cast<const uint2 *>(smem + ((c ? a ^ 32u : a) + o)),
                    *reinterpret_cast<const uint2 *>(smem + ((a ^ 64u) + o)),
                    *reinterpret_cast<const uint32_t *>(smem + (sa + 128u * nt))};
        };
        const int nsh = 4 * kg;  // ql nibble shift; qh bits 2j = nsh + 2c
        auto dequant = [&](const q6w &v, int c) -> h8 {
            const int sh = nsh + 2 * c;  // qh bits of this chunk
            const h2 d2 = __builtin_bit_cast(h2, v.sc);
            const h2 ds = c ? d2.yy : d2.xx;
            const h2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};
            h8 r;
    #pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t lw = ((u ? v.ql.y : v.ql.x) >> nsh) & 0x0F0F0F0Fu;
                const uint32_t hw = ((u ? v.qh.y : v.qh.x) >> sh) & 0x03030303u;
                const uint32_t code = lw | (hw << 4);
                const h2 w01 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, code, 0x04010400u)) - bias) * ds;
                const h2 w23 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, code, 0x04030402u)) - bias) * ds;
                r[4 * u] = w01[0];
                r[4 * u + 1] = w01[1];
                r[4 * u + 2] = w23[0];
                r[4 * u + 3] = w23[1];
            }
            return r;
        };
        auto read_a = [&](const uint8_t *buf, int c, int mt) -> h8 {
            return *reinterpret_cast<const h8 *>(buf + (16 * mt + r16) * 128 + 16 * ((4 * c + q) ^ aswz));
        };

        f4 acc[8][4];
        h8 bq[4], a0;

        // One step: as in k_prefill_q8_w8, the weights in the shared stage of
        // the step's parity: in group 14 every wavefront waits for its own
        // copies of step s + 1, after the barrier decodes its row's scales of
        // step s + 1 and reads that step's chunk-0 weights, and this step's
        // buffers take step s + 2 (pieces 0..5 in groups 14, 15, 6..7 in groups
        // 0, 2 of the next step). Chunk 1's raw weights of token tile i are read
        // in group 2 i, dequantised in group 2 i + 1.
        auto step = [&](int s, auto tag) __attribute__((always_inline)) {
            constexpr int PAR = decltype(tag)::par;
            constexpr bool MORE = decltype(tag)::more;
            const uint8_t *buf = act + PAR * kP8Act;
            const uint8_t *nbuf = act + (1 - PAR) * kP8Act;
            const uint8_t *nwbuf = smem + (1 - PAR) * kQ6W;
            h8 b1[4], a15;
            q6w rw;
    #pragma unroll
            for (int g = 0; g < 16; g++) {
                const int c = g >> 3, mt = g & 7;
                __builtin_amdgcn_sched_barrier(0);
                if (MORE && g < 4 && (g & 1) == 0 && s >= 1)
                    dma(s + 1, 6 + (g >> 1), std::integral_constant<int, 1 - PAR>{});
                if (c == 0 && (mt & 1) == 0) rw = read_w(PAR, 1, mt >> 1);
                q6w rn0, rn1;
                if (MORE && g == 14) p8_barrier_vm0();
                if (MORE && g == 14)
                    scales_of_step(nwbuf, kb0 + ((s + 1) >> 1), 1 - PAR,
                                   std::integral_constant<bool, decltype(tag)::scaled>{});
                if (MORE && g >= 14) {
                    rn0 = read_w(1 - PAR, 0, 2 * (g - 14));
                    rn1 = read_w(1 - PAR, 0, 2 * (g - 14) + 1);
                }
                // the activation operand one group ahead, except that group 13
                // also reads group 15's, so every read of this step's buffer
                // precedes the barrier of group 14 (after which it takes step
                // s + 2), and group 15 reads the next step's first
                h8 a1 = a0;
                if (g < 13) a1 = read_a(buf, (g + 1) >> 3, (g + 1) & 7);
                if (g == 13) {
                    a1 = read_a(buf, 1, 6);
                    a15 = read_a(buf, 1, 7);
                }
                if (g == 14) a1 = a15;
                if (MORE && g == 15) a1 = read_a(nbuf, 0, 0);
                if (MORE && g >= 14) {
                    dma(s + 2, 3 * (g - 14), std::integral_constant<int, PAR>{});
                    dma(s + 2, 3 * (g - 14) + 1, std::integral_constant<int, PAR>{});
                    dma(s + 2, 3 * (g - 14) + 2, std::integral_constant<int, PAR>{});
                }
                const h8 acur = a0;
                const h8 *bw = c ? b1 : bq;
    #pragma unroll
                for (int nt = 0; nt < 4; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bw[nt], acur, acc[mt][nt], 0, 0, 0);
                if (c == 0 && (mt & 1)) b1[mt >> 1] = dequant(rw, 1);
                if (MORE && g >= 14) {
                    bq[2 * (g - 14)] = dequant(rn0, 0);
                    bq[2 * (g - 14) + 1] = dequant(rn1, 0);
                }
                a0 = a1;
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        if constexpr (decltype(pass_c)::value) {
            // E of this thread's scale row from its blocks' bounds
            const int r = min(n0 + 64 * wr + lane, out_dim - 1);
            const uint8_t *rp = w + (size_t)r * row_bytes + 1664;  // d runs
            float m = 0.f;
            for (int b = kb0; b < kb0 + nb; b++) {
                const uint16_t h = *reinterpret_cast<const uint16_t *>(rp + (size_t)(b >> 3) * 1680 + 2 * (b & 7));
                m = fmaxf(m, 4096.f * fabsf(f16_to_f32(h)));
            }
            erow = pf_row_exponent(m);
            if (kg == 0) erow_lds[64 * wr + lane] = erow;
        }
        // one pass over the tile: the first with E = 0, a second (scaled) with
        // this thread's row exponent erow
        auto run = [&](auto scaled_c) __attribute__((always_inline)) {
            constexpr bool SC = decltype(scaled_c)::value;
    #pragma unroll
            for (int mt = 0; mt < 8; mt++)
    #pragma unroll
                for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

            // prologue: step 0 in, step 1 in flight, step 0's chunk-0 operands ready
    #pragma unroll
            for (int p = 0; p < 8; p++) dma(0, p, par0{});
            p8_barrier_vm0();
    #pragma unroll
            for (int p = 0; p < 8; p++) dma(1, p, par1{});  // ns >= 2
            scales_of_step(smem, kb0, 0, scaled_c);
    #pragma unroll
            for (int nt = 0; nt < 4; nt++) bq[nt] = dequant(read_w(0, 0, nt), 0);
            a0 = read_a(act, 0, 0);

            for (int sb = 0; sb + 1 < nb; sb++) {
                step(2 * sb, p8_step<0, true, SC>{});
                step(2 * sb + 1, p8_step<1, true, SC>{});
            }
            step(ns - 2, p8_step<0, true, SC>{});
            step(ns - 1, p8_step<1, false, SC>{});
        };
        run(pass_c);
        if constexpr (!decltype(pass_c)::value)
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, nullptr, flag);
        else
            p8_epilogue(acc, smem, kg, wr, lane, n0, t0, tile, unscale, n_tok, out_dim, erow_lds,
                        nullptr);
    };
    body(std::false_type{});
    if (pf_again(flag)) body(std::true_type{});
}

// out[i] += part[z][i] for z = 0 .. nz - 1 in order (n floats per slice)
__global__ __launch_bounds__(256) void k_prefill_sum(float *__restrict__ out,
                                                     const float *__restrict__ part, size_t n,
                                                     int nz) {
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const bool vec = (n & 3) == 0 && ((uintptr_t)out & 15) == 0;  // part is 16-byte aligned
    if (vec && i4 * 4 + 3 < n) {
        f4 v = *reinterpret_cast<const f4 *>(out + i4 * 4);
        for (int z = 0; z < nz; z++) v += *reinterpret_cast<const f4 *>(part + z * n + i4 * 4);
        *reinterpret_cast<f4 *>(out + i4 * 4) = v;
    } else {
        // this thread's four elements (fewer at the end)
        for (size_t i = i4 * 4; i < n && i < i4 * 4 + 4; i++) {
            float v = out[i];
            for (int z = 0; z < nz; z++) v += part[z * n + i];
            out[i] = v;
        }
    }
}

// out[t][o] += the compact slices 1 .. nz - 1 of the tail tiles in split
// order (block (i, j): float4s 256 i .. 256 i + 255 of tail tile j, a tile
// being kPfTok token rows of kPfRowsWg floats; slice z - 1 of tile j at
// part + ((z - 1) n_tail + j) kPfTok kPfRowsWg)
__global__ __launch_bounds__(256) void k_prefill_sum_tail(float *__restrict__ out,
                                                          const float *__restrict__ part,
                                                          int n_tok, int out_dim, int ld_out,
                                                          int rt, int n_full, int n_tail, int nz) {
    constexpr int kTile = kPfTok * kPfRowsWg;
    const int j = blockIdx.y, tile = n_full + j;
    const int i4 = blockIdx.x * 256 + threadIdx.x;
    const int tl = i4 / (kPfRowsWg / 4), oc = i4 % (kPfRowsWg / 4) * 4;
    const int t = tile / rt * kPfTok + tl, o = tile % rt * kPfRowsWg + oc;
    if (t >= n_tok || o >= out_dim) return;
    const size_t slice = (size_t)n_tail * kTile;
    const float *p = part + (size_t)j * kTile + tl * kPfRowsWg + oc;
    float *y = out + (size_t)t * ld_out + o;
    if (o + 3 < out_dim && (ld_out & 3) == 0 && ((uintptr_t)out & 15) == 0) {
        f4 v = *reinterpret_cast<const f4 *>(y);
        for (int z = 1; z < nz; z++) v += *reinterpret_cast<const f4 *>(p + (z - 1) * slice);
        *reinterpret_cast<f4 *>(y) = v;
    } else {
        for (int i = 0; i < 4 && o + i < out_dim; i++) {
            float v = y[i];
            for (int z = 1; z < nz; z++) v += p[(z - 1) * slice + i];
            y[i] = v;
        }
    }
}

// How a call's GEMM covers its tiles (256 rows x 128 tokens each, one
// workgroup per CU, 256 CUs):
// * grids of fewer than 128 workgroups split K into nz splits, as many as
//   keep the grid within one round of 256 workgroups (a partial second round
//   costs more than the split gains), each split keeping at least two
//   super-blocks, at most 16;
// * grids of more than one round whose last round holds R <= 128 tiles
//   split those R tiles into tail_s splits each (tail_s R <= 256, the same
//   limits), so the last round runs tail_s R shorter workgroups;
// either only where the partial sums keep the whole workspace within the
// no-allocation entry point's maximum (so a call that fits it without
// splitting still fits). Calls that need more than one launch (32-bit
// offsets, below) are not split.
struct PfPlan {
    int nz = 1;                  // K splits of every tile (3D grid)
    int tail_s = 0;              // K splits of each tail tile (1D grid), or 0
    int n_full = 0, n_tail = 0;  // whole tiles, tail tiles (tail_s > 0)
};
constexpr size_t kPfCUs = 256;
static PfPlan prefill_plan(int n_tok, int in_dim, int out_dim) {
    PfPlan p;
    const size_t rt = (size_t)(out_dim + kPfRowsWg - 1) / kPfRowsWg;
    const size_t tt = ((size_t)n_tok + kPfTok - 1) / kPfTok;
    const size_t grid = rt * tt, nbt = (size_t)in_dim / 256;
    if (nbt < 4) return p;
    const size_t row_bytes = nbt * 272;  // the larger of Q8_0's and Q4_K's row bytes
    if ((size_t)out_dim * row_bytes > UINT32_MAX || (size_t)n_tok * in_dim * 2 > INT32_MAX) return p;
    const size_t base = ((size_t)n_tok * in_dim * 2 + 15) / 16 * 16 + tt * kPfTok * 4;
    if (grid < kPfCUs / 2) {
        size_t nz = std::min<size_t>({kPfCUs / grid, nbt / 2, 16});
        while (nz > 1 && base + (nz - 1) * (size_t)n_tok * out_dim * 4 > RSLLM_HIP_NOALLOC_SCRATCH_BYTES)
            nz--;
        p.nz = (int)nz;
        return p;
    }
    const size_t r = grid % kPfCUs;
    if (grid < kPfCUs || r == 0 || r > kPfCUs / 2) return p;
    size_t s = std::min<size_t>({kPfCUs / r, nbt / 2, 16});
    while (s > 1 && base + (s - 1) * r * kPfTok * kPfRowsWg * 4 > RSLLM_HIP_NOALLOC_SCRATCH_BYTES) s--;
    if (s > 1) {
        p.tail_s = (int)s;
        p.n_tail = (int)r;
        p.n_full = (int)(grid - r);
    }
    return p;
}

size_t prefill_scratch_bytes(int n_tok, int in_dim, int out_dim) {
    // f16 activations, one f32 unscale per token padded to whole 128-token
    // tiles (16-byte aligned), then the partial sums of splits 1 .. S - 1
    const size_t tiles = ((size_t)n_tok + kPfTok - 1) / kPfTok;
    const PfPlan p = prefill_plan(n_tok, in_dim, out_dim);
    const size_t part = p.tail_s ? (size_t)(p.tail_s - 1) * p.n_tail * kPfTok * kPfRowsWg
                                 : (size_t)(p.nz - 1) * n_tok * out_dim;
    return ((size_t)n_tok * in_dim * 2 + 15) / 16 * 16 + tiles * kPfTok * 4 + part * 4;
}

// One GEMM launch on the pre-pass's image (partial sums in part)
static hipError_t prefill_gemm(uint32_t dtype, const uint8_t *w, const _Float16 *xh,
                               const float *unscale, float *out, float *part, const PfPlan &p,
                               int n_tok, int in_dim, int out_dim, int ld_out, hipStream_t s) {
    const dim3 grid = p.tail_s ? dim3((unsigned)(p.n_full + p.n_tail * p.tail_s))
                               : dim3((unsigned)((out_dim + kPfRowsWg - 1) / kPfRowsWg),
                                      (unsigned)((n_tok + kPfTok - 1) / kPfTok), (unsigned)p.nz);
    const int rt = (out_dim + kPfRowsWg - 1) / kPfRowsWg;
    if (dtype == T_Q8_0)
        k_prefill_q8_w8<<<grid, 512, 0, s>>>(w, xh, unscale, out, part, n_tok, in_dim, out_dim, ld_out,
                                             rt, p.n_full, p.tail_s);
    else if (dtype == T_Q6_K)
        k_prefill_q6_w8<<<grid, 512, 0, s>>>(w, xh, unscale, out, part, n_tok, in_dim, out_dim, ld_out,
                                             rt, p.n_full, p.tail_s);
    else
        k_prefill_q4k_w8<<<grid, 512, 0, s>>>(w, xh, unscale, out, part, n_tok, in_dim, out_dim,
                                              ld_out, rt, p.n_full, p.tail_s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.tail_s) {
        k_prefill_sum_tail<<<dim3(kPfTok * kPfRowsWg / 4 / 256, (unsigned)p.n_tail), 256, 0, s>>>(
            out, part, n_tok, out_dim, ld_out, rt, p.n_full, p.n_tail, p.tail_s);
        return hipGetLastError();
    }
    if (p.nz == 1) return hipSuccess;
    const size_t n = (size_t)n_tok * out_dim;
    k_prefill_sum<<<(unsigned)((n + 1023) / 1024), 256, 0, s>>>(out, part, n, p.nz - 1);
    return hipGetLastError();
}

// The pre-pass, then the GEMM; x is bf16 (x_bf16) or f32 (x_f32). The
// kernels address weights with 32-bit byte offsets and the activation image
// with 32-bit byte offsets too, so a call whose weights pass 4 GiB or whose
// image passes 2 GiB runs as several launches over row and token ranges
// (whole 256-row and 128-token tiles).
static hipError_t prefill_run(uint32_t dtype, const uint8_t *w, const uint16_t *x_bf16,
                              const float *x_f32, uint8_t *scratch, float *out, int n_tok,
                              int in_dim, int out_dim, hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    const size_t row_bytes = dtype == T_Q6_K ? (size_t)(in_dim / 2048) * 1680
                                             : (size_t)(in_dim / 256) * (dtype == T_Q8_0 ? 272 : kQ4kBytes);
    const size_t rows_max = (size_t)UINT32_MAX / row_bytes / kPfRowsWg * kPfRowsWg;
    const size_t toks_max = (size_t)INT32_MAX / ((size_t)in_dim * 2) / kPfTok * kPfTok;
    if (rows_max == 0 || toks_max == 0) return hipErrorInvalidValue;
    const size_t tiles = ((size_t)n_tok + kPfTok - 1) / kPfTok;
    const size_t xb = ((size_t)n_tok * in_dim * 2 + 15) / 16 * 16;
    _Float16 *xh = reinterpret_cast<_Float16 *>(scratch);
    float *unscale = reinterpret_cast<float *>(scratch + xb);
    float *part = unscale + tiles * kPfTok;
    if (x_f32)
        k_prefill_x_f32<<<(unsigned)n_tok, 256, 0, s>>>(x_f32, xh, unscale, in_dim);
    else
        k_prefill_x<<<(unsigned)n_tok, 256, 0, s>>>(x_bf16, xh, unscale, in_dim);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const PfPlan plan = prefill_plan(n_tok, in_dim, out_dim);
    for (size_t t0 = 0; t0 < (size_t)n_tok; t0 += toks_max) {
        const int nt = (int)std::min(toks_max, (size_t)n_tok - t0);
        for (size_t r0 = 0; r0 < (size_t)out_dim; r0 += rows_max) {
            const int nr = (int)std::min(rows_max, (size_t)out_dim - r0);
            e = prefill_gemm(dtype, w + r0 * row_bytes, xh + t0 * in_dim, unscale + t0,
                             out + t0 * out_dim + r0, part, plan, nt, in_dim, nr, out_dim, s);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

hipError_t launch_prefill_q4k(const uint8_t *w, size_t w_bytes, const uint16_t *x_bf16,
                              uint8_t *scratch, float *out, int n_tok, int in_dim, int out_dim,
                              hipStream_t s) {
    (void)w_bytes;
    return prefill_run(T_Q4_K, w, x_bf16, nullptr, scratch, out, n_tok, in_dim, out_dim, s);
}

hipError_t launch_prefill_f32(uint32_t dtype, const uint8_t *w, const float *x, uint8_t *scratch,
                              float *out, int n_tok, int in_dim, int out_dim, hipStream_t s) {
    if (dtype != T_Q4_K && dtype != T_Q8_0 && !(dtype == T_Q6_K && in_dim % 2048 == 0))
        return hipErrorInvalidValue;
    return prefill_run(dtype, w, nullptr, x, scratch, out, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
