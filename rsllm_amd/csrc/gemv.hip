// Quantized GEMV, batch 1..n: y[t, o] = sum_i deq(W)[o, i] * x[t, i].
//
// Restates matmul_quant_f32 (rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119)
// without materialising dequantised rows; the weight formats and the
// two-limb activation arithmetic are in gemv_formats.h.
//
// Kernels:
//   k_gemv1         batch 1, x quantised in LDS inside the kernel (one launch);
//   k_quant_x       activation pre-pass for larger batches (limbs to scratch);
//   k_gemv          batch 2..32: a wavefront owns RT rows x one K column of 8
//                   units, issues every load of the column at once; the
//                   wavefronts of a workgroup combine per-row partials in LDS;
//   k_gemv_grouped  the same per routed expert (slot lists sorted by expert);
//   k_quant_swiglu  SwiGLU of the gate/up outputs fused with the pre-pass.
#include "gemv_formats.h"

#include <algorithm>

namespace rsllm_hip {

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
    stage_format_tables<F>();
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
// Steps past a wavefront's last tile (its last round of PD) skip their
// arithmetic: on MI355X a step costs about 0.2 us of issue, which showed at
// the end of the kernel. Compiler scheduling barriers keep each
// step's loads ahead of its arithmetic, so the waits before each tile's
// arithmetic leave the later tiles in flight.
//
// Groups. The rows form groups of rows_per_group consecutive rows (one
// group: rows_per_group = out_dim); row r of group g = r / rows_per_group
// dots x columns [g * x_gstride, g * x_gstride + in_dim) of each token.
// Workgroups are dealt group-major, wpg per group: workgroup b serves group
// b / wpg and takes that group's rows b % wpg + wpg * l, and its LDS image
// holds only that group's x. Token t of x starts at x + t * x_stride (x_dim
// readable values from there); y[t, r] is at y + t * y_stride + r.
// Weights: one matrix of out_dim rows at w; or, with w1 set, two matrices of
// rows_per_group rows each (group 0 at w, group 1 at w1, w1_bytes long), as
// an FFN's gate and up projections of one x (x_gstride 0).
struct Gemv1Shape {
    int in_dim, out_dim, x_dim, x_stride, y_stride, rows_per_group, wpg;
    int x_gstride;
    const uint8_t *w1;
    uint32_t w1_bytes;
};

template <class F, int NW, int PD, int GPT, int BT = 1, bool UNI = false>
__global__ __launch_bounds__(64 * NW) void k_gemv1(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                  const float *__restrict__ x,
                                                  float *__restrict__ y, Gemv1Shape sh,
                                                  int n_tok) {
    const int in_dim = sh.in_dim, out_dim = sh.out_dim;
    extern __shared__ uint4 xl[];
    stage_format_tables<F, false>();  // before the barrier that ends the x prologue
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    constexpr int kThreads = 64 * NW;
    const int lane = threadIdx.x & 63, k = lane & 7, ks = lane >> 3;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nunits = F::units(in_dim), ncols = (nunits + 7) >> 3;
    const int per_tok = ncols * 64 * kHalves;                           // limb groups per token
    const int n_groups = per_tok * BT;
    const uint32_t tok_fields = (uint32_t)ncols * F::kXF * 64;          // uint4 per token in LDS
    const int wpg = sh.wpg, R = sh.rows_per_group;
    const int gsel = blockIdx.x / wpg;                                   // this workgroup's group
    const int r0 = blockIdx.x - gsel * wpg;
    const int row_base = gsel * R;
    const int nrows = r0 < R ? (R - r0 + wpg - 1) / wpg : 0;            // this workgroup's rows
    const int my_rows = nrows > wv ? (nrows - wv + NW - 1) / NW : 0;   // this wavefront's rows
    const int T = my_rows * ncols;                                       // its tiles
    // the matrix this workgroup's rows belong to: its rows, and the first
    // global row in it
    const bool pair = sh.w1 != nullptr;
    const __amdgpu_buffer_rsrc_t rw =
        pair && gsel ? make_rsrc(sh.w1, sh.w1_bytes) : make_rsrc(w, w_bytes);
    const int mrows = pair ? R : out_dim, mbase = pair ? row_base : 0;
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(w, 0);
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x, ((uint32_t)(n_tok - 1) * (uint32_t)sh.x_stride + (uint32_t)sh.x_dim) * 4u);

    // limb group g (token g / per_tok) -> first element offset in x, or -1
    auto group_off = [&](int g) {
        const int t = g / per_tok, rem = g - t * per_tok;
        const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        const int kk = ln & 7, unit = col * 8 + (ln >> 3);
        const bool ok = g < n_groups && t < n_tok && unit < nunits && F::valid(unit, kk, in_dim);
        return ok ? t * sh.x_stride + gsel * sh.x_gstride +
                        (half ? F::elem_hi(unit, kk) : F::elem_lo(unit, kk))
                  : -1;
    };
    auto row_of = [&](int j) { return row_base + r0 + wpg * (wv + NW * j); };
    typename F::Slice buf[PD];
    // UNI (rows of whole 8-unit groups, F::kUniform): per-lane offsets
    // fixed, the tile's base a scalar offset
    uint32_t loff[F::kNO];
    if constexpr (UNI) F::lane_offs(loff, ks, k);
    // Tiles are loaded in order through a cursor (row lj of this wavefront's
    // list, column lc), advanced after each load.
    // Loads are never branched over (the compiler would then wait for every
    // load in flight where the paths join): a tile past the wavefront's last
    // one is read through a zero-length buffer resource, which returns zeros
    // without memory traffic.
    int lj = 0, lc = 0;
    auto load_next = [&](typename F::Slice &sl, bool real) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t r = real ? rw : rnull;
        const int row = min(row_of(lj), out_dim - 1) - mbase;
        if constexpr (UNI) {
            F::load_u(sl, r, loff, F::tile_base((uint32_t)row, (uint32_t)lc, in_dim));
        } else {
            const int unit = min(lc * 8 + ks, nunits - 1);
            F::load(sl, r, row, unit, k, in_dim, mrows);
        }
        // arithmetic updates (a conditional store to one of two captured
        // variables is lowered through memory)
        const bool wrap = lc + 1 == ncols;
        lj += wrap ? 1 : 0;
        lc = wrap ? 0 : lc + 1;
    };

    // Prologue: x loads, the first tiles, then quantisation into LDS (token
    // t's columns at t * tok_fields; tokens past n_tok quantise zeros). Group
    // indices past n_groups store into one spare column.
    uint4 xv[GPT][4];
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        if (wv * 64 + i * kThreads >= n_groups) continue;
        const int e = group_off(threadIdx.x + i * kThreads);
        const uint32_t off = e >= 0 ? (uint32_t)e * 4u : 0x80000000u;  // past the end: zeros
#pragma unroll
        for (int q = 0; q < 4; q++) xv[i][q] = bload16(rx, off + 16u * q, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PD - 1; j++) load_next(buf[j], j < T);
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
        const int t = gg / per_tok, rem = gg - t * per_tok;
        const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        uint4 *b = xl + t * tok_fields + col * F::kXF * 64 + ln;
        b[(half ? 3 : 0) * 64] = h;
        b[(half ? 4 : 1) * 64] = l;
        reinterpret_cast<float2 *>(b + 2 * 64)[half] = make_float2(sc, sum);
    }
    __syncthreads();

    float acc[BT];
#pragma unroll
    for (int tk = 0; tk < BT; tk++) acc[tk] = 0.f;
    // One tile's arithmetic; the row's total is stored after its last column.
    int col = 0, j = 0;
    auto step = [&](const typename F::Slice &sl) __attribute__((always_inline)) {
        const int unit = col * 8 + ks;
        const bool ok = unit < nunits && F::valid(unit, k, in_dim);
#pragma unroll
        for (int tk = 0; tk < BT; tk++) {
            XSlice xs;
            const uint4 *bx = xl + tk * tok_fields + col * F::kXF * 64 + lane;
            xs.hlo = bx[0];
            xs.llo = bx[64];
            xs.meta = bx[128];
            if (F::kXF == 5) {
                xs.hhi = bx[192];
                xs.lhi = bx[256];
            }
            const float d = F::dot(sl, k, xs);
            acc[tk] += ok ? d : 0.f;
        }
        const bool last = col == ncols - 1;
        if (last) {
#pragma unroll
            for (int tk = 0; tk < BT; tk++) {
                const float tot = wave_sum_dpp(acc[tk]);
                if (lane == 0 && tk < n_tok) y[(size_t)tk * sh.y_stride + row_of(j)] = tot;
                acc[tk] = 0.f;
            }
        }
        j += last ? 1 : 0;
        col = last ? 0 : col + 1;
    };
    // Rounds of PD steps: step t uses slot t % PD and loads tile t + PD - 1
    // into the slot step t - 1 used; steps past T (the last round's) load
    // through the null resource and skip their arithmetic.
    for (int t0 = 0; t0 < T; t0 += PD) {
#pragma unroll
        for (int jj = 0; jj < PD; jj++) {
            load_next(buf[(jj + PD - 1) % PD], t0 + jj + PD - 1 < T);
            __builtin_amdgcn_sched_barrier(0);
            if (t0 + jj < T) step(buf[jj]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// LDS of k_gemv1: the quantised x (bt tokens x the columns of one group's
// in_dim) plus one spare column.
template <class F>
static size_t gemv1_lds_bytes(int in_dim, int bt = 1) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    return (size_t)(bt * ncols + 1) * F::kXF * 1024;
}

// Groups of x per thread the prologue needs (1, 2 or 4; 0 = too long).
template <class F>
static int gemv1_gpt(int in_dim, int nw, int bt = 1) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    const int groups = bt * ncols * 64 * (F::kXF == 5 ? 2 : 1);
    const int gpt = (groups + 64 * nw - 1) / (64 * nw);
    return gpt <= 1 ? 1 : gpt <= 2 ? 2 : gpt <= 4 ? 4 : 0;
}

template <class F, int NW, int PD, int GPT, int BT, bool UNI>
static hipError_t gemv1_launch(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                               const Gemv1Shape &sh, int n_tok, int n_wg, hipStream_t s) {
    // the attribute once per kernel (thread-safe static initialisation)
    static const hipError_t attr = hipFuncSetAttribute(
        (const void *)k_gemv1<F, NW, PD, GPT, BT, UNI>, hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)(kGemv1MaxLds - kFormatTableLds<F>));
    if (attr != hipSuccess) return attr;
    // n_wg workgroups dealt over the groups (at least one per group, at most
    // one per row)
    Gemv1Shape g = sh;
    const int n_grp = sh.out_dim / sh.rows_per_group;
    g.wpg = max(1, min(n_wg / n_grp, sh.rows_per_group));
    k_gemv1<F, NW, PD, GPT, BT, UNI>
        <<<(unsigned)(n_grp * g.wpg), 64 * NW, gemv1_lds_bytes<F>(sh.in_dim, BT), s>>>(
            w, (uint32_t)w_bytes, x, y, g, n_tok);
    return hipGetLastError();
}

template <class F, int NW, int PD, int GPT, int BT>
static hipError_t gemv1_go(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                           const Gemv1Shape &sh, int n_tok, int n_wg, hipStream_t s) {
    // rows of whole 8-unit groups take the scalar-offset tile loads
    if constexpr (F::kUniform)
        if ((sh.in_dim / F::kEPU) % 8 == 0)
            return gemv1_launch<F, NW, PD, GPT, BT, true>(w, w_bytes, x, y, sh, n_tok, n_wg, s);
    return gemv1_launch<F, NW, PD, GPT, BT, false>(w, w_bytes, x, y, sh, n_tok, n_wg, s);
}

template <class F, int NW, int PD, int BT = 1>
static hipError_t gemv1_gpt_go(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                               const Gemv1Shape &sh, int n_tok, int n_wg, hipStream_t s) {
    switch (gemv1_gpt<F>(sh.in_dim, NW, BT)) {
    case 1: return gemv1_go<F, NW, PD, 1, BT>(w, w_bytes, x, y, sh, n_tok, n_wg, s);
    case 2: return gemv1_go<F, NW, PD, 2, BT>(w, w_bytes, x, y, sh, n_tok, n_wg, s);
    case 4: return gemv1_go<F, NW, PD, 4, BT>(w, w_bytes, x, y, sh, n_tok, n_wg, s);
    default: return hipErrorInvalidValue;
    }
}

static Gemv1Shape plain_shape(int n_tok, int in_dim, int out_dim) {
    (void)n_tok;
    return Gemv1Shape{in_dim, out_dim, in_dim, in_dim, out_dim, out_dim, 1, in_dim, nullptr, 0};
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
    stage_format_tables<F>();
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

// Routes for more than 32 tokens (prefill, n_tok = T): Q4_K and Q8_0 with
// in_dim a multiple of 256, and Q6_K with rows of whole 8-block super-tiles
// (in_dim a multiple of 2048), take the prefill GEMM; other Q6_K rows with
// in_dim a multiple of 256, and Q2_K and IQ2_XXS (the DS-V4 expert formats)
// with in_dim a multiple of 256, the exact matrix-core GEMV over 32-token
// chunks (one weight pass per 32 tokens instead of per 8 on the int8-limb
// GEMV).
enum class Prefill { none, gemm, mfma_chunks };
static Prefill prefill_route(uint32_t dtype, int n_tok, int in_dim) {
    if (n_tok <= 32 || in_dim <= 0 || in_dim % 256 != 0) return Prefill::none;
    if (dtype == T_Q4_K || dtype == T_Q8_0) return Prefill::gemm;
    if (dtype == T_Q6_K) return in_dim % 2048 == 0 ? Prefill::gemm : Prefill::mfma_chunks;
    if (dtype == T_Q2_K || dtype == T_IQ2_XXS) return Prefill::mfma_chunks;
    return Prefill::none;
}

size_t gemv_work_bytes(uint32_t dtype, int n_tok, int in_dim, int out_dim) {
    switch (prefill_route(dtype, n_tok, in_dim)) {
    case Prefill::gemm:
        // the GEMM, or the int8-limb GEMV where w or x is not 16-byte aligned
        return std::max(prefill_scratch_bytes(n_tok, in_dim, out_dim),
                        gemv_scratch_bytes(dtype, n_tok, in_dim));
    case Prefill::mfma_chunks: return gemv_mfma_scratch_bytes(dtype, 32, in_dim, out_dim);
    default: break;
    }
    size_t b = gemv_scratch_bytes(dtype, n_tok, in_dim);
    if (gemv_mfma_supported(dtype, n_tok, in_dim, out_dim)) {
        const size_t m = gemv_mfma_scratch_bytes(dtype, n_tok, in_dim, out_dim);
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
static hipError_t gemv1(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                        const Gemv1Shape &sh, hipStream_t s) {
    const int cus = device_cus();
    if (w_bytes >= ((size_t)32 << 20)) {
        if (sh.out_dim >= 2 * sh.in_dim) return gemv1_gpt_go<F, 8, 2>(w, w_bytes, x, y, sh, 1, 2 * cus, s);
        return gemv1_gpt_go<F, 8, 3>(w, w_bytes, x, y, sh, 1, cus, s);
    }
    return gemv1_gpt_go<F, 16, 2>(w, w_bytes, x, y, sh, 1, cus, s);
}

// Wavefronts per workgroup of the batched kernel for BT tokens. Eight
// tokens of a five-field x image (every format but Q8_0) take 8 wavefronts:
// a 1024-thread workgroup caps a thread at 128 VGPRs, and eight tokens'
// accumulators and x slices then spill to scratch (3-5x slower on MI355X).
template <class F>
constexpr int gemv1_batch_nw(int bt) {
    return bt == 8 && F::kXF == 5 ? 8 : 16;
}

template <class F>
static bool gemv1_fits_f(int in_dim, int bt) {
    return gemv1_lds_bytes<F>(in_dim, bt) <= kGemv1MaxLds - kFormatTableLds<F> &&
           gemv1_gpt<F>(in_dim, bt == 1 ? 8 : gemv1_batch_nw<F>(bt), bt) != 0;
}

// Tokens the fused kernel takes as one batch (x of all of them in LDS):
// 1, 2, 4 or 8; 0 if n_tok does not fit.
template <class F>
static int gemv1_bt(int n_tok, int in_dim) {
    const int bt = n_tok <= 1 ? 1 : n_tok <= 2 ? 2 : n_tok <= 4 ? 4 : n_tok <= 8 ? 8 : 0;
    return bt && gemv1_fits_f<F>(in_dim, bt) ? bt : 0;
}

// 2..8 tokens: one workgroup per CU, two tiles in flight, 16 wavefronts
// (8 for gemv1_batch_nw's case); sweeps of the C0-C2 shapes at 2, 4 and 8
// tokens.
template <class F>
static hipError_t gemv1_batch(const uint8_t *w, size_t w_bytes, const float *x, float *y,
                              const Gemv1Shape &sh, int n_tok, hipStream_t s) {
    const int cus = device_cus();
    switch (gemv1_bt<F>(n_tok, sh.in_dim)) {
    case 2: return gemv1_gpt_go<F, 16, 2, 2>(w, w_bytes, x, y, sh, n_tok, cus, s);
    case 4: return gemv1_gpt_go<F, 16, 2, 4>(w, w_bytes, x, y, sh, n_tok, cus, s);
    case 8:
        return gemv1_gpt_go<F, gemv1_batch_nw<F>(8), 2, 8>(w, w_bytes, x, y, sh, n_tok, cus, s);
    default: return hipErrorInvalidValue;
    }
}

#define GEMV_FORMATS(X)                                                                            \
    X(T_Q4_K, FQ4K) X(T_Q6_K, FQ6K) X(T_Q8_0, FQ8<false>) X(T_Q4_0, FQ8<true>) X(T_Q2_K, FQ2K)     \
    X(T_IQ2_XXS, FIQ2XXSK)

static int gemv1_tokens(uint32_t dtype, int n_tok, int in_dim) {
#define X(T, F) if (dtype == T) return gemv1_bt<F>(n_tok, in_dim);
    GEMV_FORMATS(X)
#undef X
    return 0;
}

// ---- f32 weights (WeightBlob::F32) ----------------------------------------------
// y[t * y_stride + r] = sum_i w[r * in_dim + i] * x[t * x_stride + g(r) * in_dim + i],
// g(r) = r / rows_per_group: matmul_weight_f32's F32 arm (weight.rs:139-158)
// and, with groups, matmul_grouped_lora_down over F32 blobs. Rows are dealt
// as in k_gemv1 and streamed whole: a tile is 256 consecutive elements (lane
// l takes l, l + 64, l + 128, l + 192: four coalesced dword loads), PD tiles
// in flight, fp32 FMA; tokens in chunks of BT (one weight pass per chunk).
template <int NW, int PD, int BT>
__global__ __launch_bounds__(64 * NW) void k_gemv_f32(const float *__restrict__ w,
                                                     const float *__restrict__ x,
                                                     float *__restrict__ y, Gemv1Shape sh,
                                                     int n_wg, int n_tok) {
    const int in_dim = sh.in_dim, out_dim = sh.out_dim;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = blockIdx.x;
    const int nrows = (out_dim - r0 + n_wg - 1) / n_wg;
    const int my_rows = nrows > wv ? (nrows - wv + NW - 1) / NW : 0;
    const int ncols = (in_dim + 255) >> 8;
    const int T = my_rows * ncols;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)((size_t)out_dim * in_dim * 4u));
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(w, 0);
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x, ((uint32_t)(n_tok - 1) * (uint32_t)sh.x_stride + (uint32_t)sh.x_dim) * 4u);
    auto row_of = [&](int j) { return r0 + n_wg * (wv + NW * j); };
    struct Tile {
        float v[4];
    };
    for (int t_base = 0; t_base < n_tok; t_base += BT) {
        Tile buf[PD];
        auto load_tile = [&](Tile &tl, int t) {
            const int j = t / ncols, col = t - j * ncols;
            const uint32_t rowoff = (uint32_t)min(row_of(j), out_dim - 1) * (uint32_t)in_dim;
            const __amdgpu_buffer_rsrc_t r = t < T ? rw : rnull;
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int e = col * 256 + m * 64 + lane;
                const uint32_t off = e < in_dim ? (rowoff + (uint32_t)e) * 4u : 0x80000000u;
                tl.v[m] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
            }
        };
#pragma unroll
        for (int jj = 0; jj < PD - 1; jj++) load_tile(buf[jj], jj);
        float acc[BT];
#pragma unroll
        for (int tk = 0; tk < BT; tk++) acc[tk] = 0.f;
        int col = 0, j = 0;
        for (int t0 = 0; t0 < T; t0 += PD) {
#pragma unroll
            for (int jj = 0; jj < PD; jj++) {
                const int t = t0 + jj;
                load_tile(buf[(jj + PD - 1) % PD], t + PD - 1);
                __builtin_amdgcn_sched_barrier(0);
                const int row = min(row_of(j), out_dim - 1);
                const uint32_t xg = (uint32_t)(row / sh.rows_per_group) * (uint32_t)in_dim;
#pragma unroll
                for (int tk = 0; tk < BT; tk++) {
                    const uint32_t xt = (uint32_t)(t_base + tk) * (uint32_t)sh.x_stride + xg;
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const int e = col * 256 + m * 64 + lane;
                        const bool ok = e < in_dim && t < T && t_base + tk < n_tok;
                        const uint32_t off = ok ? (xt + (uint32_t)e) * 4u : 0x80000000u;
                        const float xv = __uint_as_float(
                            (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rx, (int)off, 0, 0));
                        acc[tk] = fmaf(buf[jj].v[m], xv, acc[tk]);
                    }
                }
                if (col == ncols - 1) {
#pragma unroll
                    for (int tk = 0; tk < BT; tk++) {
                        const float tot = wave_sum_dpp(acc[tk]);
                        if (lane == 0 && t < T && t_base + tk < n_tok)
                            y[(size_t)(t_base + tk) * sh.y_stride + row_of(j)] = tot;
                        acc[tk] = 0.f;
                    }
                    col = 0;
                    j++;
                } else {
                    col++;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

hipError_t launch_gemv_f32(const float *w, const float *x, float *y, int n_tok, int in_dim,
                           int out_dim, int x_dim, int x_stride, int y_stride, int rows_per_group,
                           hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    const Gemv1Shape sh{in_dim, out_dim, x_dim, x_stride, y_stride, rows_per_group,
                        0,      in_dim,  nullptr, 0};
    const int n_wg = min(device_cus(), out_dim);
    // x offsets are 32-bit byte offsets: launch in token chunks of < 2 GiB of x
    const size_t per = ((size_t)1 << 29) / (size_t)(x_stride > 0 ? x_stride : 1);
    const int chunk = per == 0 ? 1 : per > (size_t)n_tok ? n_tok : (int)per;
    for (int t0 = 0; t0 < n_tok; t0 += chunk) {
        k_gemv_f32<16, 2, 4><<<(unsigned)n_wg, 64 * 16, 0, s>>>(
            w, x + (size_t)t0 * x_stride, y + (size_t)t0 * y_stride, sh, n_wg,
            min(chunk, n_tok - t0));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Quantized rows with strided / grouped x and y through k_gemv1, tokens in
// chunks of up to 8 (one group's x for a chunk in LDS; each chunk is one
// pass over the weights). hipErrorNotSupported: one group's x is too long for
// LDS even for one token.
bool gemv_rows_fits(uint32_t dtype, int in_dim) { return gemv1_tokens(dtype, 1, in_dim) != 0; }

// k_gemv1 over token chunks of up to 8 (the largest whose x fits in LDS).
static hipError_t gemv1_chunks(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                               float *y, int n_tok, const Gemv1Shape &sh, hipStream_t s) {
    for (int t0 = 0; t0 < n_tok;) {
        int c = n_tok - t0 < 8 ? n_tok - t0 : 8;
        while (c > 1 && gemv1_tokens(dtype, c, sh.in_dim) == 0) c = (c + 1) / 2;
        const float *xc = x + (size_t)t0 * sh.x_stride;
        float *yc = y + (size_t)t0 * sh.y_stride;
        hipError_t e = hipErrorInvalidValue;
        if (c == 1) {
#define X(T, F) if (dtype == T) e = gemv1<F>(w, w_bytes, xc, yc, sh, s);
            GEMV_FORMATS(X)
#undef X
        } else {
#define X(T, F) if (dtype == T) e = gemv1_batch<F>(w, w_bytes, xc, yc, sh, c, s);
            GEMV_FORMATS(X)
#undef X
        }
        if (e != hipSuccess) return e;
        t0 += c;
    }
    return hipSuccess;
}

hipError_t launch_gemv_rows(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                            float *y, int n_tok, int in_dim, int out_dim, int x_dim, int x_stride,
                            int y_stride, int rows_per_group, hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    if (rows_per_group <= 0 || out_dim % rows_per_group != 0) return hipErrorInvalidValue;
    if (!gemv_rows_fits(dtype, in_dim)) return hipErrorNotSupported;
    const Gemv1Shape sh{in_dim, out_dim, x_dim, x_stride, y_stride, rows_per_group,
                        1,      in_dim,  nullptr, 0};
    return gemv1_chunks(dtype, w, w_bytes, x, y, n_tok, sh, s);
}

hipError_t launch_gemv_pair(uint32_t dtype, const uint8_t *w0, const uint8_t *w1, size_t w_bytes,
                            const float *x, float *y, int n_tok, int in_dim, int rows,
                            int y_stride, hipStream_t s) {
    if (n_tok <= 0 || rows <= 0) return hipSuccess;
    if (!gemv_rows_fits(dtype, in_dim)) return hipErrorNotSupported;
    const Gemv1Shape sh{in_dim, 2 * rows, in_dim, in_dim, y_stride, rows,
                        1,      0,        w1,     (uint32_t)w_bytes};
    return gemv1_chunks(dtype, w0, w_bytes, x, y, n_tok, sh, s);
}

hipError_t launch_gemv(uint32_t dtype, const uint8_t *w, size_t w_bytes, const float *x,
                       uint8_t *xq_scratch, float *y, int n_tok, int in_dim, int out_dim,
                       hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    switch (prefill_route(dtype, n_tok, in_dim)) {
    case Prefill::gemm:
        // the GEMM's global->LDS copies move 16-byte pieces
        if ((((uintptr_t)w | (uintptr_t)x) & 15) == 0)
            return launch_prefill_f32(dtype, w, x, xq_scratch, y, n_tok, in_dim, out_dim, s);
        break;
    case Prefill::mfma_chunks:
        // every chunk, a short tail included, on the matrix cores (which pad
        // a partial token tile), so all tokens get the same exact weights
        for (int t0 = 0; t0 < n_tok; t0 += 32) {
            const int nt = n_tok - t0 < 32 ? n_tok - t0 : 32;
            const hipError_t e =
                launch_gemv_mfma(dtype, w, w_bytes, x + (size_t)t0 * in_dim, xq_scratch,
                                 y + (size_t)t0 * out_dim, nt, in_dim, out_dim, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    default: break;
    }
    if (gemv_mfma_supported(dtype, n_tok, in_dim, out_dim))
        return launch_gemv_mfma(dtype, w, w_bytes, x, xq_scratch, y, n_tok, in_dim, out_dim, s);
    const int bt = gemv1_tokens(dtype, n_tok, in_dim);
    const Gemv1Shape sh = plain_shape(n_tok, in_dim, out_dim);
    if (bt == 1) {
#define X(T, F) if (dtype == T) return gemv1<F>(w, w_bytes, x, y, sh, s);
        GEMV_FORMATS(X)
#undef X
        return hipErrorInvalidValue;
    }
    if (bt > 1) {
#define X(T, F) if (dtype == T) return gemv1_batch<F>(w, w_bytes, x, y, sh, n_tok, s);
        GEMV_FORMATS(X)
#undef X
        return hipErrorInvalidValue;
    }
    hipError_t e = launch_quantize_x(dtype, x, xq_scratch, n_tok, in_dim, s);
    if (e != hipSuccess) return e;
    return launch_gemv_prequant(dtype, w, w_bytes, xq_scratch, y, n_tok, in_dim, out_dim, s);
}

}  // namespace rsllm_hip
