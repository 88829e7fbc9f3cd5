// Prefill GEMM: out[t, o] = sum_i deq(W)[o, i] * x[t, i] for a Q4_K weight W
// [out_dim x in_dim] and bf16 activations x [n_tok x in_dim], fp32 output.
//
// The reference computes this as matmul_quant_f32 on f32(bf16 x)
// (backend-cpu/src/ops/quant_matmul.rs:45-119): every weight row is
// dequantised once per token and dotted in f32. Here it is one dense
// contraction on the CDNA4 matrix cores:
//
// 1. k_prefill_x: per token t, x is scaled by 2^e_t so that max|x_t| lands in
//    [2^14, 2^15) and converted to f16. bf16 has an 8-bit significand, so the
//    conversion is exact for every element within 2^-29 of the token's
//    maximum; 2^-e_t is kept to undo the scaling in the epilogue.
// 2. k_prefill_q4k: W is dequantised in registers to f16,
//    w = f16(d*sc_j) * q - f16(dmin*m_j) (packed f16 FMA, q exact), straight
//    into the operands of v_mfma_f32_16x16x32_f16 against the f16
//    activations; products accumulate in fp32. The f16 weight rounding
//    (about 2^-11 relative per weight) keeps the output within about 3e-4
//    of the reference, inside the 1e-3 budget.
//
// Tiling: a workgroup is 4 wavefronts and covers 256 weight rows x TOK
// tokens (TOK = 128, or 64 when the 128-token grid would leave most CUs
// idle); a wavefront owns 64 rows (4 MFMA tiles) x TOK tokens (TOK / 16
// tiles), accumulators held in VGPRs. Every weight is dequantised once per
// workgroup and used for all TOK tokens: the larger tile halves the
// dequantisation per MFMA, the smaller one fits two workgroups per CU (80
// KiB of LDS instead of 112). The weights are the MFMA A operand and the
// activations the B operand, so every lane ends with 4 consecutive outputs of
// one token. The K loop runs in steps of
// half a super-block (128 elements). Each step's activations (TOK tokens x
// 128 f16), weight bytes (256 rows x the 64 qs bytes of that half,
// 16 KB) and block headers (256 rows x 16 bytes) are copied global->LDS by
// DMA into one of two stage buffers while the other is computed. Each
// thread turns its own row's header into f16 (d*sc_j, dmin*m_j) once per
// step and leaves them in LDS for the lanes that dequantise that row.
//
// K order: inside a super-block, MFMA chunk c (0..7) gives lane group q
// (lanes 16q..16q+15) sub-block 2q + (c & 1), positions 8 * (c >> 1) .. + 7,
// so a lane's weights for one half are 16 contiguous qs bytes (low nibbles
// for even c, high for odd c); the activation stage is laid out in the same
// order. Half h holds positions 16h .. 16h + 15 of every sub-block.
#include "kernels.h"

namespace rsllm_hip {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPfTok = 128;                      // largest token tile (tokens per workgroup)
constexpr int kPfRowsWave = 64;                  // weight rows per wavefront
constexpr int kPfRowsWg = 4 * kPfRowsWave;       // weight rows per workgroup
constexpr int kPfQsBytes = kPfRowsWg * 64;      // weight qs stage: 256 rows x 64 bytes
constexpr int kPfHdBytes = kPfRowsWg * 16;      // weight header stage: 256 rows x 16 bytes
constexpr int kPfNStage = 2;                    // stage buffers
// LDS of the TOK-token workgroup: two stages of (TOK rows x 128 f16
// activations, qs, headers), then the f16 block scales (256 rows x 32 bytes):
// 114688 bytes at TOK = 128, 81920 at TOK = 64
constexpr int pf_lds(int tok) {
    return kPfNStage * (tok * 256 + kPfQsBytes + kPfHdBytes) + kPfRowsWg * 32;
}

typedef __attribute__((address_space(3))) void lds_void;

// 16-byte global->LDS DMA (a non-template wrapper: the builtin called
// directly inside a kernel template keeps the host pass from emitting that
// kernel's stub)
__device__ __forceinline__ void pf_dma16(const void *g, uint8_t *l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)l, 16, 0, 0);
}

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

struct pf_true { static constexpr bool value = true; };
struct pf_false { static constexpr bool value = false; };

// dword i (0..3) of a uint4 for a compile-time i
__device__ __forceinline__ uint32_t pf_u4(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int TOK>
__global__ __launch_bounds__(256) void k_prefill_q4k(const uint8_t *__restrict__ w,
                                                     const _Float16 *__restrict__ xh,
                                                     const float *__restrict__ unscale,
                                                     float *__restrict__ out, int n_tok, int in_dim,
                                                     int out_dim) {
    // token tiles per workgroup, activation DMA instructions per wavefront,
    // DMA instructions per stage and wavefront, operand groups per step
    constexpr int MT = TOK / 16, XP = TOK / 16, NP = XP + 5, NG = 4 * MT;
    constexpr int kXBytes = TOK * 256, kStage = kXBytes + kPfQsBytes + kPfHdBytes;
    constexpr int kScOff = kPfNStage * kStage;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * kPfRowsWg;  // first weight row of the workgroup
    const int t0 = blockIdx.y * TOK;
    const int nb = in_dim >> 8;
    const int nsteps = 2 * nb;

    // DMA sources. Activations: instruction p of this wave moves token rows
    // 4g .. 4g + 3 (g = 8 wv + p), lane i to row 4g + i / 16, slot i % 16;
    // slot s of token row tl holds chunk k = s ^ (tl & 15), i.e. elements
    // 32 (k >> 1) + 16h + 8 (k & 1) .. + 7 of the super-block. Rows past
    // n_tok repeat the last token (their outputs are not stored).
    uint32_t xoff[XP];
#pragma unroll
    for (int p = 0; p < XP; p++) {
        const int tl = 4 * (XP * wv + p) + (lane >> 4);
        const int k = (lane & 15) ^ (tl & 15);
        const int t = min(t0 + tl, n_tok - 1);
        xoff[p] = (uint32_t)t * (uint32_t)in_dim + 32u * (k >> 1) + 8u * (k & 1);
    }
    // Weight qs: instruction p (g = 4 wv + p) moves pieces j = 64 g + i, row
    // j / 4, slot j % 4 holding qs piece k = slot ^ ((row >> 2) & 3) (bytes
    // 32k + 16h .. + 15 of the block), so the operand reads below hit 16
    // distinct bank groups. Headers: one instruction per wave, lane i moves
    // the header of row 64 wv + i. Both cover exactly this wave's own rows.
    uint32_t qoff[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int j = 64 * (4 * wv + p) + lane;
        const int row = j >> 2, k = (j & 3) ^ ((row >> 2) & 3);
        const uint32_t rowg = (uint32_t)min(n0 + row, out_dim - 1);
        qoff[p] = rowg * (uint32_t)nb * 144u + 16u + 32u * k;
    }
    const uint32_t hoff = (uint32_t)min(n0 + 64 * wv + lane, out_dim - 1) * (uint32_t)nb * 144u;
    // DMA instruction p (0..NP - 1) of stage st into buf: 0..XP - 1
    // activations, XP..XP + 3 qs, XP + 4 headers.
    auto dma_piece = [&](int st, uint8_t *buf, int p) {
        const int s = st >> 1, h = st & 1;
        if (p < XP)
            pf_dma16(xh + xoff[p] + s * 256 + 16 * h, buf + 1024 * (XP * wv + p));
        else if (p < XP + 4)
            pf_dma16(w + qoff[p - XP] + s * 144 + 16 * h, buf + kXBytes + 1024 * (4 * wv + p - XP));
        else
            pf_dma16(w + hoff + s * 144, buf + kXBytes + kPfQsBytes + 1024 * wv);
    };
    // activation operand of group g (chunk g / MT of the step, token tile
    // g % MT): elements of sub-block 2q + (c & 1) at positions 16h + 8 (c >> 1)
    // .. + 7.
    auto read_a = [&](const uint8_t *buf, int g) -> h8 {
        const int c = g / MT, mt = g % MT;
        const int k = 2 * (2 * q + (c & 1)) + (c >> 1);
        return *reinterpret_cast<const h8 *>(buf + (mt * 16 + r16) * 256 + ((k ^ r16) << 4));
    };
    // this lane's weight rows in the stage: wave rows 16 nt + r16; qs piece
    // q sits in slot q ^ ((row >> 2) & 3) = q ^ (r16 >> 2) (rows 16 nt + r16)
    const int wrow = wv * kPfRowsWave + r16;
    const int qslot = q ^ (r16 >> 2);

    f4 acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

    // f16 scales of this lane's sub-blocks 2q, 2q + 1: .x = (d*sc_2q,
    // d*sc_2q+1), .y = (dmin*m_2q, dmin*m_2q+1)
    uint2 sc[4];
    uint4 qs[4];
    h8 bq[4];
    uint8_t *const scl = smem + kScOff;
    auto load_step_weights = [&](const uint8_t *buf) {
        // this thread's row 64 wv + lane: header -> 16 f16 scales into LDS,
        // record layout per q: {d*sc_2q, d*sc_2q+1, dmin*m_2q, dmin*m_2q+1}
        // (q4_k_scale_min, dequant/mod.rs:48-58, on four bytes at a time)
        {
            const uint4 hd = *reinterpret_cast<const uint4 *>(buf + kXBytes + kPfQsBytes + 16 * (64 * wv + lane));
            const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
            const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, m_lo = hd.z & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
            uint32_t rec[8];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                // sub-blocks 2qq, 2qq + 1: bytes of the low (j < 4) or high word
                const uint32_t sw = qq < 2 ? sc_lo : sc_hi, mw = qq < 2 ? m_lo : m_hi;
                const int b = 2 * (qq & 1);
                const _Float16 a0 = (_Float16)(d * (float)((sw >> (8 * b)) & 0xFFu));
                const _Float16 a1 = (_Float16)(d * (float)((sw >> (8 * b + 8)) & 0xFFu));
                const _Float16 m0 = (_Float16)(dmin * (float)((mw >> (8 * b)) & 0xFFu));
                const _Float16 m1 = (_Float16)(dmin * (float)((mw >> (8 * b + 8)) & 0xFFu));
                rec[2 * qq] = __builtin_bit_cast(uint32_t, h2{a0, a1});
                rec[2 * qq + 1] = __builtin_bit_cast(uint32_t, h2{m0, m1});
            }
            uint4 *dst = reinterpret_cast<uint4 *>(scl + 32 * (64 * wv + lane));
            dst[0] = make_uint4(rec[0], rec[1], rec[2], rec[3]);
            dst[1] = make_uint4(rec[4], rec[5], rec[6], rec[7]);
        }
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int row = wrow + 16 * nt;
            qs[nt] = *reinterpret_cast<const uint4 *>(buf + kXBytes + row * 64 + qslot * 16);
            sc[nt] = *reinterpret_cast<const uint2 *>(scl + row * 32 + q * 8);
        }
    };
    // B operands of chunk c (0..3) of the current step
    auto dequant = [&](int c, int nt) -> h8 {
        const int run = c >> 1;  // bytes 8 run .. 8 run + 7 of the lane's 16
        const h2 d2 = __builtin_bit_cast(h2, sc[nt].x), m2 = __builtin_bit_cast(h2, sc[nt].y);
        const h2 ds = (c & 1) ? d2.yy : d2.xx;
        const h2 dm = (c & 1) ? m2.yy : m2.xx;
        return pf_dequant8(pf_u4(qs[nt], 2 * run), pf_u4(qs[nt], 2 * run + 1), (c & 1) != 0, ds,
                           dm);
    };

    // Stage st + 1 is in flight while step st is computed: its DMA is issued
    // right after the barrier in step st - 1, into the buffer step st - 1
    // used. The last step's DMA repeats the last stage into a buffer nothing
    // reads again.
    auto sbuf = [&](int st) { return smem + (st & 1) * kStage; };
#pragma unroll
    for (int p = 0; p < NP; p++) dma_piece(0, sbuf(0), p);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; p++) dma_piece(1, sbuf(1), p);  // nsteps >= 2 (in_dim >= 256)
    load_step_weights(sbuf(0));
#pragma unroll
    for (int nt = 0; nt < 4; nt++) bq[nt] = dequant(0, nt);
    h8 a0 = read_a(sbuf(0), 0), a1 = read_a(sbuf(0), 1);

    // One K step: NG groups (4 chunks x MT token tiles) of 4 MFMAs. Operand
    // reads run two groups ahead (across the step boundary), weight operands
    // are dequantised one chunk ahead (chunk 3 prepares the next step's chunk
    // 0 from the next stage's weight rows). The DMA of stage st + 2 is
    // spread so the CU's return path is never flooded: instructions 0..3
    // after the barrier in groups NG - 2, NG - 1 of step st, 4..NP - 1 one
    // per group in groups 0..NP - 5 of step st + 1. MORE: a next step exists.
    auto step = [&](int st, auto more_tag) {
        constexpr bool more = decltype(more_tag)::value;
        uint8_t *buf = sbuf(st);
        const uint8_t *nbuf = sbuf(st + 1);
        h8 bn[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            __builtin_amdgcn_sched_barrier(0);
            if (more && c == 3) {
                // stage st + 1: this wave's own weight rows are in once its
                // own DMA has completed
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
                load_step_weights(nbuf);
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int g = MT * c + mt;
                if (more && g <= NP - 5)  // rest of stage st + 1
                    dma_piece(min(st + 1, nsteps - 1), buf + (nbuf - buf), 4 + g);
                if (more && g == NG - 2) {
                    // every wave has its operands up to group NG - 1 in
                    // registers and its stage-(st+1) DMA complete: the next
                    // stage's activation rows become readable and `buf` is
                    // free for stage st + 2 (the last stage again when there
                    // is none; nothing reads it then)
                    __syncthreads();
                }
                if (more && g >= NG - 2) {
                    dma_piece(min(st + 2, nsteps - 1), buf, 2 * (g - (NG - 2)));
                    dma_piece(min(st + 2, nsteps - 1), buf, 2 * (g - (NG - 2)) + 1);
                }
                h8 a2 = a1;
                if (g + 2 < NG) a2 = read_a(buf, g + 2);
                else if (more) a2 = read_a(nbuf, g + 2 - NG);
                const h8 acur = a0;
#pragma unroll
                for (int nt = 0; nt < 4; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bq[nt], acur, acc[mt][nt], 0, 0, 0);
                // the next chunk's 4 weight operands, spread over the groups
                if (MT == 8 ? (mt & 1) : true) {
                    const int nt = MT == 8 ? (mt >> 1) : mt;
                    if (c < 3) bn[nt] = dequant(c + 1, nt);
                    else if (more) bn[nt] = dequant(0, nt);
                }
                a0 = a1;
                a1 = a2;
            }
            // per group: 4 MFMAs, one operand read, the group's share of
            // the dequantisation (VPS VALU instructions after each MFMA)
            constexpr int VPS = MT == 8 ? 2 : 3;
#pragma unroll
            for (int i = 0; i < MT; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
                __builtin_amdgcn_sched_group_barrier(0x002, VPS, 0);  // VALU
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPS, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPS, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPS, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (c < 3 || more) {
#pragma unroll
                for (int nt = 0; nt < 4; nt++) bq[nt] = bn[nt];
            }
        }
    };
    for (int st = 0; st + 1 < nsteps; st++) step(st, pf_true{});
    step(nsteps - 1, pf_false{});

    // The weights are the MFMA A operand, so tile (mt, nt) has weight rows
    // as its rows: lane (r16, q) holds outputs o = 16 nt + 4q + i (i = 0..3)
    // of token t = 16 mt + r16 — four consecutive outputs of one token, one
    // 16-byte store. The unscale vector is padded to whole 128-token tiles,
    // which cover whole 64-token tiles too.
    float us[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) us[mt] = unscale[t0 + mt * 16 + r16];
    const int ow = n0 + wv * kPfRowsWave + 4 * q;
    const bool vec = (out_dim & 3) == 0;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int t = t0 + mt * 16 + r16;
        if (t >= n_tok) continue;
        float *orow = out + (size_t)t * out_dim;
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int o = ow + 16 * nt;
            const f4 v = acc[mt][nt] * us[mt];
            if (vec && o + 3 < out_dim) {
                *reinterpret_cast<f4 *>(orow + o) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (o + i < out_dim) orow[o + i] = v[i];
            }
        }
    }
}

size_t prefill_scratch_bytes(int n_tok, int in_dim) {
    // f16 activations, then one f32 unscale per token padded to whole
    // 128-token tiles (16-byte aligned)
    const size_t tiles = ((size_t)n_tok + kPfTok - 1) / kPfTok;
    return ((size_t)n_tok * in_dim * 2 + 15) / 16 * 16 + tiles * kPfTok * 4;
}

// The GEMM on TOK-token workgroup tiles (the dynamic LDS size set once)
template <int TOK>
static hipError_t prefill_gemm(const uint8_t *w, const _Float16 *xh, const float *unscale,
                               float *out, int n_tok, int in_dim, int out_dim, hipStream_t s) {
    static const hipError_t attr = hipFuncSetAttribute(
        (const void *)k_prefill_q4k<TOK>, hipFuncAttributeMaxDynamicSharedMemorySize, pf_lds(TOK));
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((out_dim + kPfRowsWg - 1) / kPfRowsWg),
                    (unsigned)((n_tok + TOK - 1) / TOK));
    k_prefill_q4k<TOK><<<grid, 256, pf_lds(TOK), s>>>(w, xh, unscale, out, n_tok, in_dim, out_dim);
    return hipGetLastError();
}

// The GEMM on the pre-pass's image; x is bf16 (x_bf16) or f32 (x_f32).
static hipError_t prefill_q4k(const uint8_t *w, const uint16_t *x_bf16, const float *x_f32,
                              uint8_t *scratch, float *out, int n_tok, int in_dim, int out_dim,
                              hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    const size_t xb = ((size_t)n_tok * in_dim * 2 + 15) / 16 * 16;
    _Float16 *xh = reinterpret_cast<_Float16 *>(scratch);
    float *unscale = reinterpret_cast<float *>(scratch + xb);
    if (x_f32)
        k_prefill_x_f32<<<(unsigned)n_tok, 256, 0, s>>>(x_f32, xh, unscale, in_dim);
    else
        k_prefill_x<<<(unsigned)n_tok, 256, 0, s>>>(x_bf16, xh, unscale, in_dim);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // 128-token tiles unless that grid fills under 160 of the 256 CUs: then
    // 64-token tiles, two workgroups per CU (C4 at T = 100: 52 us instead of
    // 68; at T = 512, 224 workgroups, the 128-token tile is 10% faster)
    const size_t g128 = (size_t)((out_dim + kPfRowsWg - 1) / kPfRowsWg) * (size_t)((n_tok + 127) / 128);
    if (g128 < 160) return prefill_gemm<64>(w, xh, unscale, out, n_tok, in_dim, out_dim, s);
    return prefill_gemm<128>(w, xh, unscale, out, n_tok, in_dim, out_dim, s);
}

hipError_t launch_prefill_q4k(const uint8_t *w, size_t w_bytes, const uint16_t *x_bf16,
                              uint8_t *scratch, float *out, int n_tok, int in_dim, int out_dim,
                              hipStream_t s) {
    (void)w_bytes;
    return prefill_q4k(w, x_bf16, nullptr, scratch, out, n_tok, in_dim, out_dim, s);
}

hipError_t launch_prefill_q4k_f32(const uint8_t *w, const float *x, uint8_t *scratch, float *out,
                                  int n_tok, int in_dim, int out_dim, hipStream_t s) {
    return prefill_q4k(w, nullptr, x, scratch, out, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
