// Routed-expert MoE layer on the GPU:
//   out[t] += sum_i w[t, i] * down[e] ( silu(min(gate[e] x_t, c)) * clamp(up[e] x_t, -c, c) ),
//   e = ids[t, i], for every token t and selected slot i with w[t, i] != 0.
//
// Restates accumulate_moe_outputs (rsllm-models/src/dsv4/moe.rs:648-707) with
// apply_expert_swiglu (:479-502) and apply_swiglu_clamp (:515-531). The
// reference runs three matmul_quant_f32 GEMVs per (token, expert) pair,
// re-reading each selected expert's weights once per token. Here the
// (token, slot) pairs are grouped by expert on the device, and each expert's
// gate/up and down matrices are streamed once per batch of up to 4 of its
// tokens (grouped GEMV, gemv.hip; for Q4_K, Q6_K, Q8_0, Q2_K and IQ2_XXS
// experts whenever the fused pair does not take the call in one go, batches
// of up to 8 or 16 on the matrix cores instead, launch_moe_mfma in
// gemv_mfma.hip, steps 2-6 there):
//   1. routing (k_moe_hist, k_moe_scan, k_moe_scatter, any number of
//      pairs): slots sorted by expert (ties in (t, i) order), per-expert
//      offsets, slot -> token, (t, i) -> slot, the list of active experts;
//      slots with w == 0 are skipped (moe.rs:681-683). Calls of more than
//      kMoeMaxPairs pairs run in token chunks, one pass each.
//   2. activation limbs of x for the gate/up format;
//   3. grouped GEMV, gate and up in one launch -> hg, hu [slot x n_ff];
//   4+5. clamp (only when c > 1e-6; NaN passes), silu(g) * u and the
//      activation limbs for the down format in one pass;
//   6. grouped GEMV, down -> yd [slot x n_embd];
//   7. k_moe_accumulate: out[t, j] += w[t, i] * yd[slot(t, i), j] in i order,
//      as the reference's `out_t[j] += we * expert_out[j]` (no contraction).
#include "gemv_formats.h"
#include "moe_route.h"

namespace rsllm_hip {

// ---- routing: slots sorted by expert -----------------------------------------
// The (t, i) pairs, p = t * k + i, are cut into blocks of 256. A valid pair
// (w != 0, expert id in range) gets slot
//     base[e][b] + (valid pairs of expert e before p in its block b),
// base[e][b] = valid pairs of experts < e, plus those of expert e in blocks
// before b: slots are sorted by expert, ties in pair order, for any number of
// pairs. Three launches: per-block counts and in-block ranks; one workgroup
// scans the counts (expert-major) into the bases and lists the active
// experts and the matrix-core batches; per-pair scatter. Calls of up to
// kRoute1Pairs pairs take the one-launch form k_moe_route1 (one block).
constexpr int kRouteBlock = 256;

inline int route_blocks(int n_pairs) { return (n_pairs + kRouteBlock - 1) / kRouteBlock; }

// hist[e * nblk + b] = valid pairs of expert e in block b; rank[p] = valid
// pairs of p's expert before p in its block.
__global__ __launch_bounds__(kRouteBlock) void k_moe_hist(const int *__restrict__ ids,
                                                          const float *__restrict__ wts,
                                                          int n_pairs, int n_expert,
                                                          int *__restrict__ hist,
                                                          int *__restrict__ rank) {
    extern __shared__ int cnt[];  // n_expert
    __shared__ int eb[kRouteBlock];
    const int tid = threadIdx.x, b = blockIdx.x, nblk = gridDim.x;
    for (int e = tid; e < n_expert; e += kRouteBlock) cnt[e] = 0;
    const int p = b * kRouteBlock + tid;
    int e = -1;
    if (p < n_pairs) {
        const int id = ids[p];
        if (wts[p] != 0.0f && id >= 0 && id < n_expert) e = id;
    }
    eb[tid] = e;
    __syncthreads();
    if (e >= 0) {
        atomicAdd(&cnt[e], 1);
        int r = 0;
        for (int q = 0; q < tid; q++) r += eb[q] == e ? 1 : 0;
        rank[p] = r;
    }
    __syncthreads();
    for (int x = tid; x < n_expert; x += kRouteBlock) hist[(size_t)x * nblk + b] = cnt[x];
}

// One workgroup: hist -> bases (in place); off[e] (n_expert + 1 entries);
// the active experts in ascending order (act, *n_act); and, when bat is
// given, each active expert's slots cut into batches of up to bw (experts
// ascending, batches in slot order; *n_bat of them). `flags` holds n_expert
// + 1 ints of workspace.
__global__ __launch_bounds__(kScanThreads) void k_moe_scan(int *__restrict__ hist, int nblk,
                                                           int n_expert, int *__restrict__ off,
                                                           int *__restrict__ act,
                                                           int *__restrict__ n_act,
                                                           MfgBatch *__restrict__ bat,
                                                           int *__restrict__ n_bat, int bw,
                                                           int *__restrict__ flags) {
    __shared__ int part[kScanThreads];
    const int tid = threadIdx.x;
    const int total = scan_inplace(hist, (size_t)n_expert * nblk, part);
    for (int e = tid; e < n_expert; e += kScanThreads) off[e] = hist[(size_t)e * nblk];
    if (tid == 0) off[n_expert] = total;
    __syncthreads();
    // active experts: positions from a scan of the 0/1 flags
    for (int e = tid; e < n_expert; e += kScanThreads) {
        const int c = (e + 1 < n_expert ? hist[(size_t)(e + 1) * nblk] : total) -
                      hist[(size_t)e * nblk];
        flags[e] = c > 0 ? 1 : 0;
    }
    __syncthreads();
    const int na = scan_inplace(flags, (size_t)n_expert, part);
    for (int e = tid; e < n_expert; e += kScanThreads) {
        const int next = e + 1 < n_expert ? flags[e + 1] : na;
        if (next != flags[e]) act[flags[e]] = e;
    }
    if (tid == 0) *n_act = na;
    if (!bat) return;
    __syncthreads();
    // batches: positions from a scan of ceil(count / bw)
    for (int e = tid; e < n_expert; e += kScanThreads) {
        const int c = off[e + 1] - off[e];
        flags[e] = (c + bw - 1) / bw;
    }
    __syncthreads();
    const int nb = scan_inplace(flags, (size_t)n_expert, part);
    for (int e = tid; e < n_expert; e += kScanThreads) {
        const int c = off[e + 1] - off[e];
        for (int f = 0, j = flags[e]; f < c; f += bw, j++)
            bat[j] = MfgBatch{off[e] + f, c - f < bw ? c - f : bw, e, 0};
    }
    if (tid == 0) *n_bat = nb;
}

// slot_of[p] = the pair's slot, or -1 when it is skipped; slot_tok[slot] = t.
__global__ __launch_bounds__(kRouteBlock) void k_moe_scatter(const int *__restrict__ ids,
                                                             const float *__restrict__ wts,
                                                             int n_pairs, int k, int n_expert,
                                                             const int *__restrict__ base,
                                                             const int *__restrict__ rank,
                                                             int *__restrict__ slot_tok,
                                                             int *__restrict__ slot_of) {
    const int b = blockIdx.x, p = b * kRouteBlock + threadIdx.x;
    if (p >= n_pairs) return;
    const int id = ids[p];
    int slot = -1;
    if (wts[p] != 0.0f && id >= 0 && id < n_expert) {
        slot = base[(size_t)id * gridDim.x + b] + rank[p];
        slot_tok[slot] = p / k;
    }
    slot_of[p] = slot;
}

// The same routing in one workgroup and one launch (moe_route1), for calls
// of up to kRoute1Pairs pairs and kRoute1Experts experts (decode batches).
// Each small launch costs a few microseconds of dependent latency; this
// saves two.
__global__ __launch_bounds__(kScanThreads) void k_moe_route1(const int *__restrict__ ids,
                                                             const float *__restrict__ wts,
                                                             int n_pairs, int k, int n_expert,
                                                             int *__restrict__ off,
                                                             int *__restrict__ slot_tok,
                                                             int *__restrict__ slot_of,
                                                             int *__restrict__ act,
                                                             int *__restrict__ n_act,
                                                             MfgBatch *__restrict__ bat,
                                                             int *__restrict__ n_bat, int bw) {
    extern __shared__ int sh[];  // 2 n_expert
    __shared__ int ep[kRoute1Pairs];
    __shared__ int part[kScanThreads];
    moe_route1(ids, wts, n_pairs, k, n_expert, off, slot_tok, slot_of, act, n_act, bat, n_bat, bw,
               sh, ep, part);
}

// Workspace of launch_moe_route: hist (n_expert x blocks), rank (one per
// pair), flags (n_expert + 1).
static size_t moe_route_work_bytes(int n_pairs, int n_expert) {
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    return al((size_t)n_expert * route_blocks(n_pairs) * 4) + al((size_t)n_pairs * 4) +
           al(((size_t)n_expert + 1) * 4);
}

static hipError_t launch_moe_route(const int *ids, const float *wts, int n_pairs, int k,
                                   int n_expert, uint8_t *work, int *off, int *slot_tok,
                                   int *slot_of, int *act, int *n_act, MfgBatch *bat, int *n_bat,
                                   int bw, hipStream_t s) {
    if (n_pairs <= kRoute1Pairs && n_expert <= kRoute1Experts) {
        k_moe_route1<<<1, kScanThreads, (size_t)n_expert * 8, s>>>(
            ids, wts, n_pairs, k, n_expert, off, slot_tok, slot_of, act, n_act, bat, n_bat, bw);
        return hipGetLastError();
    }
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    const int nblk = route_blocks(n_pairs);
    int *hist = reinterpret_cast<int *>(work);
    int *rank = reinterpret_cast<int *>(work + al((size_t)n_expert * nblk * 4));
    int *flags = reinterpret_cast<int *>(work + al((size_t)n_expert * nblk * 4) +
                                         al((size_t)n_pairs * 4));
    k_moe_hist<<<(unsigned)nblk, kRouteBlock, (size_t)n_expert * 4, s>>>(ids, wts, n_pairs,
                                                                          n_expert, hist, rank);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_moe_scan<<<1, kScanThreads, 0, s>>>(hist, nblk, n_expert, off, act, n_act, bat, n_bat, bw,
                                          flags);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    k_moe_scatter<<<(unsigned)nblk, kRouteBlock, 0, s>>>(ids, wts, n_pairs, k, n_expert, hist,
                                                         rank, slot_tok, slot_of);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_moe_accumulate(float *__restrict__ out,
                                                        const float *__restrict__ yd,
                                                        const float *__restrict__ wts,
                                                        const int *__restrict__ slot_of,
                                                        int n_tok, int k, int n_embd) {
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n_tok * n_embd) return;
    const int t = (int)(i / n_embd), j = (int)(i % n_embd);
    float v = out[i];
    for (int p = 0; p < k; p++) {
        const int s = slot_of[t * k + p];
        if (s >= 0) {
            const float prod = wts[t * k + p] * yd[(size_t)s * n_embd + j];
            v = v + prod;
        }
    }
    out[i] = v;
}

__global__ __launch_bounds__(256) void k_moe_accumulate4(float *__restrict__ out,
                                                        const float *__restrict__ yd,
                                                        const float *__restrict__ wts,
                                                        const int *__restrict__ slot_of,
                                                        int n_tok, int k, int n_embd) {
#pragma clang fp contract(off)
    // four consecutive outputs per thread (n_embd a multiple of 4, out
    // 16-byte aligned); each
    // group of 8 slots' ids and weights is loaded first and their rows' loads
    // are issued together (a skipped slot reads row 0 and is not added), then
    // the products are added in i order as before
    const int n4 = n_embd >> 2;
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i4 >= (size_t)n_tok * n4) return;
    const int t = (int)(i4 / n4), j = (int)(i4 % n4) * 4;
    float4 v = reinterpret_cast<float4 *>(out)[i4];
    for (int p0 = 0; p0 < k; p0 += 8) {
        int sl[8];
        float w[8];
        float4 y[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int p = p0 + u;
            sl[u] = p < k ? slot_of[t * k + p] : -1;
            w[u] = p < k ? wts[t * k + p] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            y[u] = *reinterpret_cast<const float4 *>(yd + (size_t)(sl[u] >= 0 ? sl[u] : 0) * n_embd + j);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (sl[u] >= 0) {
                v.x = v.x + w[u] * y[u].x;
                v.y = v.y + w[u] * y[u].y;
                v.z = v.z + w[u] * y[u].z;
                v.w = v.w + w[u] * y[u].w;
            }
        }
    }
    reinterpret_cast<float4 *>(out)[i4] = v;
}

// out[t, j] += sum_i w[t, i] * yd[slot(t, i), j] in i order, without
// contraction (skipped slots add nothing).
static hipError_t launch_moe_accumulate(float *out, const float *yd, const float *wts,
                                        const int *slot_of, int n_tok, int k, int n_embd,
                                        hipStream_t s) {
    if (n_embd % 4 == 0 && ((uintptr_t)out & 15) == 0)
        k_moe_accumulate4<<<(unsigned)(((size_t)n_tok * (n_embd / 4) + 255) / 256), 256, 0, s>>>(
            out, yd, wts, slot_of, n_tok, k, n_embd);
    else
        k_moe_accumulate<<<(unsigned)(((size_t)n_tok * n_embd + 255) / 256), 256, 0, s>>>(
            out, yd, wts, slot_of, n_tok, k, n_embd);
    return hipGetLastError();
}


// ---- fused path for a few tokens (decode) -----------------------------------
// For n_tok * k <= kFusedPairs (and x, h fitting in LDS) the layer is two
// launches of k_moe_fused:
//   gate/up: every workgroup routes the (t, i) pairs in LDS, quantises x of
//            all tokens into LDS, streams gate and up rows, and writes
//            h[slot, row] = SwiGLU with the pre-activation clamp;
//   down:    routes again (same result), quantises h of all slots into LDS,
//            streams down rows, and adds w[t, i] * y[slot(t, i), row] into
//            out[t, row] in i order.
// The active experts are walked as "chunks" of at most kChunk slots of one
// expert, so each expert row is read once for all of its slots. Pairs that
// pick the same expert twice are separate slots, as in the reference.
constexpr int kFusedPairs = 32;
constexpr int kChunk = 4;

struct MoeRoute {
    int n_chunks;
    int chunk_e[kFusedPairs], chunk_s0[kFusedPairs], chunk_n[kFusedPairs];
    int slot_tok[kFusedPairs];  // token of each slot
    int slot_of[kFusedPairs];   // pair (t * k + i) -> slot, -1 if skipped
    float wt[kFusedPairs];      // pair weights
    int eid[kFusedPairs];       // pair -> expert, -1 if skipped
    int nch[kFusedPairs];       // at an expert's first pair: its chunk count, else 0
};

// Threads p < P route pair p (P = n_tok * k <= kFusedPairs). Slots sorted by
// expert, ties in pair order, as the grid-wide routing; skipped pairs (w == 0 or an
// expert id out of range) get no slot. Ends with a workgroup barrier.
__device__ __forceinline__ void moe_route_lds(MoeRoute &r, int e_p, float w_p, int P, int k,
                                              int n_expert) {
    const int p = threadIdx.x;
    const bool valid = p < P && w_p != 0.0f && e_p >= 0 && e_p < n_expert;
    if (p < P) {
        r.eid[p] = valid ? e_p : -1;
        r.wt[p] = w_p;
    }
    __syncthreads();
    int below = 0, rank = 0, cnt = 0;
    if (p < P) {
        for (int q = 0; q < P; q++) {
            const int eq = r.eid[q];
            if (!valid || eq < 0) continue;
            if (eq < e_p) below++;
            if (eq == e_p) {
                cnt++;
                if (q < p) rank++;
            }
        }
        r.nch[p] = valid && rank == 0 ? (cnt + kChunk - 1) / kChunk : 0;
    }
    __syncthreads();
    if (p < P) {
        int chunks_below = 0, chunks_all = 0;
        for (int q = 0; q < P; q++) {
            const int c = r.nch[q];
            chunks_all += c;
            if (valid && r.eid[q] < e_p) chunks_below += c;
        }
        const int slot = valid ? below + rank : -1;
        r.slot_of[p] = slot;
        if (valid) r.slot_tok[slot] = p / k;
        if (valid && rank == 0) {
            for (int c = 0; c * kChunk < cnt; c++) {
                r.chunk_e[chunks_below + c] = e_p;
                r.chunk_s0[chunks_below + c] = below + c * kChunk;
                r.chunk_n[chunks_below + c] = min(kChunk, cnt - c * kChunk);
            }
        }
        if (p == 0) r.n_chunks = chunks_all;
    }
    __syncthreads();
}

// Quantise GPT groups per thread of `rows` rows of length in_dim (row stride
// in_dim floats) into LDS in the pre-pass layout (row-major: row, column,
// field, lane). `vals` holds the values, loaded by moe_load_groups.
template <class F, int GPT>
struct MoeGroups {
    uint4 v[GPT][4];
};

template <class F, int NW, int GPT>
__device__ __forceinline__ void moe_load_groups(MoeGroups<F, GPT> &g, const float *src,
                                                int rows, int in_dim) {
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    const int nunits = F::units(in_dim), ncols = (nunits + 7) >> 3;
    const int per_row = ncols * 64 * kHalves, n_groups = rows * per_row;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)rows * (uint32_t)in_dim * 4u);
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        if (wv * 64 + i * 64 * NW >= n_groups) continue;
        const int gidx = threadIdx.x + i * 64 * NW;
        const int row = gidx / per_row, rem = gidx % per_row;
        const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        const int kk = ln & 7, unit = col * 8 + (ln >> 3);
        const bool ok = gidx < n_groups && unit < nunits && F::valid(unit, kk, in_dim);
        const int e = ok ? (half ? F::elem_hi(unit, kk) : F::elem_lo(unit, kk)) : -1;
        const uint32_t off = e >= 0 ? ((uint32_t)row * (uint32_t)in_dim + (uint32_t)e) * 4u
                                    : 0x80000000u;
#pragma unroll
        for (int q = 0; q < 4; q++) g.v[i][q] = bload16(rs, off + 16u * q, 0);
    }
}

template <class F, int NW, int GPT>
__device__ __forceinline__ void moe_store_groups(const MoeGroups<F, GPT> &g, uint4 *xl, int rows,
                                                 int in_dim) {
    constexpr int kHalves = F::kXF == 5 ? 2 : 1;
    const int nunits = F::units(in_dim), ncols = (nunits + 7) >> 3;
    const int per_row = ncols * 64 * kHalves, n_groups = rows * per_row;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        if (wv * 64 + i * 64 * NW >= n_groups) continue;
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[4 * q] = __uint_as_float(g.v[i][q].x);
            v[4 * q + 1] = __uint_as_float(g.v[i][q].y);
            v[4 * q + 2] = __uint_as_float(g.v[i][q].z);
            v[4 * q + 3] = __uint_as_float(g.v[i][q].w);
        }
        uint4 h, l;
        float sc, sum;
        quant_values(v, h, l, sc, sum);
        const int gidx = threadIdx.x + i * 64 * NW;
        const int gg = gidx < n_groups ? gidx : n_groups;  // spare column past the end
        const int row = gg / per_row, rem = gg % per_row;
        const int col = rem / (64 * kHalves), r2 = rem % (64 * kHalves);
        const int half = r2 >> 6, ln = r2 & 63;
        uint4 *b = xl + ((size_t)row * ncols + col) * F::kXF * 64 + ln;
        b[(half ? 3 : 0) * 64] = h;
        b[(half ? 4 : 1) * 64] = l;
        reinterpret_cast<float2 *>(b + 2 * 64)[half] = make_float2(sc, sum);
    }
}

// One kernel body for both halves (GU = true: gate and up; false: down).
// Workgroup b owns rows b + n_wg * l (l < nrows). Its tiles (chunk ch, row l,
// column c), chunk-major, are split into NW contiguous runs of whole (chunk,
// row) pairs, one per wavefront: within a run the expert changes only at chunk boundaries and
// consecutive tiles are consecutive bytes of one expert's matrix. PD tiles
// are in flight. When a (chunk, row) completes, the values of the chunk's
// slots go to LDS (stage[l][slot]); after the stream and a barrier the
// workgroup writes them out:
//   GU:    h[slot, row] = silu(min(g, c)) * clamp(u, -c, c)  (per slot),
//   down:  out[t, row] += w[t, i] * y[slot(t, i), row]  in i order  (per token).
template <class F, int NW, int PD, int GPT, bool GU>
__global__ __launch_bounds__(64 * NW) void k_moe_fused(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, uint32_t stride,
    const float *__restrict__ src, int src_rows, const int *__restrict__ ids,
    const float *__restrict__ wts, float *__restrict__ dst, int n_tok, int k, int n_expert,
    int in_dim, int out_dim, float clamp, int n_wg) {
#pragma clang fp contract(off)
    extern __shared__ uint4 xlds[];
    __shared__ MoeRoute rt;
    stage_format_tables<F>();
    const int lane = threadIdx.x & 63, kk = lane & 7, ks = lane >> 3;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int P = n_tok * k;
    const int nunits = F::units(in_dim), ncols = (nunits + 7) >> 3;
    const uint32_t row_fields = (uint32_t)ncols * F::kXF * 64;  // uint4 per LDS x row
    const int r0 = blockIdx.x;
    const int nrows = (out_dim - r0 + n_wg - 1) / n_wg;
    // stage[l][slot] (GU: [l][slot] holds g, [l][P + slot] u)
    float *stage = reinterpret_cast<float *>(xlds + ((size_t)src_rows * ncols + 1) * F::kXF * 64);
    constexpr int kVals = GU ? 2 : 1;

    int e_p = -1;
    float w_p = 0.f;
    if ((int)threadIdx.x < P) {
        e_p = ids[threadIdx.x];
        w_p = wts[threadIdx.x];
    }
    MoeGroups<F, GPT> xg;
    moe_load_groups<F, NW, GPT>(xg, src, src_rows, in_dim);
    moe_route_lds(rt, e_p, w_p, P, k, n_expert);

    const int n_chunks = __builtin_amdgcn_readfirstlane(rt.n_chunks);
    const int per_chunk = nrows * ncols;
    // runs are whole (chunk, row) pairs: a row's columns are summed by one
    // wavefront, which writes the row's values when its last column is done
    const int R = n_chunks * nrows;
    const int t_beg = (int)(((long long)R * wv) / NW) * ncols,
              t_end = (int)(((long long)R * (wv + 1)) / NW) * ncols;
    const int T = t_end - t_beg;
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(w0, 0);

    typename F::Slice b0[PD], b1[PD];
    // load cursor at tile t_beg
    int lch = T > 0 ? t_beg / per_chunk : 0;
    int ll = T > 0 ? (t_beg - lch * per_chunk) / ncols : 0;
    int lc = T > 0 ? t_beg - lch * per_chunk - ll * ncols : 0;
    int le = T > 0 ? __builtin_amdgcn_readfirstlane(rt.chunk_e[lch]) : 0;
    auto load_next = [&](typename F::Slice &s0_, typename F::Slice &s1_, int lt) {
        const bool ok = lt < T;
        const size_t base = (size_t)le * stride;
        const int unit = min(lc * 8 + ks, nunits - 1);
        const int row = min(r0 + n_wg * ll, out_dim - 1);
        F::load(s0_, ok ? make_rsrc(w0 + base, stride) : rnull, row, unit, kk, in_dim, out_dim);
        if (GU) F::load(s1_, ok ? make_rsrc(w1 + base, stride) : rnull, row, unit, kk, in_dim, out_dim);
        if (++lc == ncols) {
            lc = 0;
            if (++ll == nrows) {
                ll = 0;
                if (++lch < n_chunks) le = __builtin_amdgcn_readfirstlane(rt.chunk_e[lch]);
            }
        }
    };
#pragma unroll
    for (int j = 0; j < PD - 1; j++) load_next(b0[j], b1[j], j);
    __builtin_amdgcn_sched_barrier(0);
    moe_store_groups<F, NW, GPT>(xg, xlds, src_rows, in_dim);
    __syncthreads();

    // compute cursor
    int cch = lch, cl = 0, cc = 0;
    {
        const int c0 = T > 0 ? t_beg / per_chunk : 0;
        cch = c0;
        cl = T > 0 ? (t_beg - c0 * per_chunk) / ncols : 0;
        cc = T > 0 ? t_beg - c0 * per_chunk - cl * ncols : 0;
    }
    int cn = T > 0 ? __builtin_amdgcn_readfirstlane(rt.chunk_n[cch]) : 0;
    int cs0 = T > 0 ? __builtin_amdgcn_readfirstlane(rt.chunk_s0[cch]) : 0;
    float a0[kChunk], a1[kChunk];
#pragma unroll
    for (int q = 0; q < kChunk; q++) a0[q] = a1[q] = 0.f;
    for (int t0 = 0; t0 < T; t0 += PD) {
#pragma unroll
        for (int jj = 0; jj < PD; jj++) {
            const int t = t0 + jj;
            load_next(b0[(jj + PD - 1) % PD], b1[(jj + PD - 1) % PD], t + PD - 1);
            __builtin_amdgcn_sched_barrier(0);
            if (t < T) {
                const int unit = cc * 8 + ks;
                const bool okl = unit < nunits && F::valid(unit, kk, in_dim);
#pragma unroll
                for (int q = 0; q < kChunk; q++) {
                    if (q < cn) {
                        // GU: x row = the slot's token; down: x row = the slot
                        const int xr = GU ? __builtin_amdgcn_readfirstlane(rt.slot_tok[cs0 + q]) : cs0 + q;
                        const uint4 *bx = xlds + xr * row_fields + cc * F::kXF * 64 + lane;
                        XSlice xs;
                        xs.hlo = bx[0];
                        xs.llo = bx[64];
                        xs.meta = bx[128];
                        if (F::kXF == 5) {
                            xs.hhi = bx[192];
                            xs.lhi = bx[256];
                        }
                        const float d0 = F::dot(b0[jj], kk, xs);
                        a0[q] += okl ? d0 : 0.f;
                        if (GU) {
                            const float d1 = F::dot(b1[jj], kk, xs);
                            a1[q] += okl ? d1 : 0.f;
                        }
                    }
                }
                if (++cc == ncols) {
#pragma unroll
                    for (int q = 0; q < kChunk; q++) {
                        if (q < cn) {
                            const float v0 = wave_sum_dpp(a0[q]);
                            const float v1 = GU ? wave_sum_dpp(a1[q]) : 0.f;
                            if (lane == 0) {
                                stage[(size_t)cl * kVals * P + cs0 + q] = v0;
                                if (GU) stage[(size_t)cl * kVals * P + P + cs0 + q] = v1;
                            }
                        }
                        a0[q] = a1[q] = 0.f;
                    }
                    cc = 0;
                    if (++cl == nrows) {
                        cl = 0;
                        if (++cch < n_chunks) {
                            cn = __builtin_amdgcn_readfirstlane(rt.chunk_n[cch]);
                            cs0 = __builtin_amdgcn_readfirstlane(rt.chunk_s0[cch]);
                        }
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();
    if (n_chunks == 0) return;
    if (GU) {
        // h[slot, row] for the valid slots (a slot belongs to exactly one chunk)
        const int n_slots = rt.chunk_s0[n_chunks - 1] + rt.chunk_n[n_chunks - 1];
        for (int i = threadIdx.x; i < nrows * n_slots; i += 64 * NW) {
            const int l = i / n_slots, sl = i % n_slots;
            const float g = stage[(size_t)l * 2 * P + sl], u = stage[(size_t)l * 2 * P + P + sl];
            dst[(size_t)sl * out_dim + r0 + n_wg * l] = swiglu_clamped(g, u, clamp);
        }
    } else {
        for (int i = threadIdx.x; i < nrows * n_tok; i += 64 * NW) {
            const int l = i / n_tok, t = i % n_tok;
            float *o = dst + (size_t)t * out_dim + r0 + n_wg * l;
            float v = *o;
            for (int q = 0; q < k; q++) {
                const int sl = rt.slot_of[t * k + q];
                if (sl >= 0) {
                    const float prod = rt.wt[t * k + q] * stage[(size_t)l * P + sl];
                    v = v + prod;
                }
            }
            *o = v;
        }
    }
}

// LDS (dynamic part) of the two fused kernels.
template <class F>
static size_t moe_x_lds(int rows, int in_dim) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    return ((size_t)rows * ncols + 1) * F::kXF * 1024;
}
template <class F>
static int moe_gpt(int rows, int in_dim, int nw) {
    const int ncols = ((in_dim + F::kEPU - 1) / F::kEPU + 7) >> 3;
    const int groups = rows * ncols * 64 * (F::kXF == 5 ? 2 : 1);
    const int g = (groups + 64 * nw - 1) / (64 * nw);
    return g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : 0;
}
// LDS of k_moe_fused: the quantised x rows plus one spare column, then the
// stage of (rows per workgroup) x P values (x 2 for gate/up).
template <class F>
static size_t moe_fused_lds(int src_rows, int in_dim, int out_dim, int n_wg, int P, bool gu) {
    const int rows_wg = (out_dim + n_wg - 1) / n_wg;
    return moe_x_lds<F>(src_rows, in_dim) + (size_t)rows_wg * P * (gu ? 2 : 1) * 4;
}
constexpr size_t kMoeMaxLds = 152 * 1024;

template <class F, int NW, int PD, int GPT, bool GU>
static hipError_t fused_go(const uint8_t *w0, const uint8_t *w1, size_t stride, const float *src,
                           int src_rows, const int *ids, const float *wts, float *dst, int n_tok,
                           int k, int n_expert, int in_dim, int out_dim, float clamp, int n_wg,
                           hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)k_moe_fused<F, NW, PD, GPT, GU>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMoeMaxLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    n_wg = min(n_wg, out_dim);
    const size_t lds = moe_fused_lds<F>(src_rows, in_dim, out_dim, n_wg, n_tok * k, GU);
    k_moe_fused<F, NW, PD, GPT, GU><<<(unsigned)n_wg, 64 * NW, lds, s>>>(
        w0, w1, (uint32_t)stride, src, src_rows, ids, wts, dst, n_tok, k, n_expert, in_dim,
        out_dim, clamp, n_wg);
    return hipGetLastError();
}

template <class F, int NW, int PD, int GPT>
static hipError_t gu_go(const uint8_t *gate, const uint8_t *up, size_t stride, const float *x,
                        const int *ids, const float *wts, float *h, int n_tok, int k, int n_expert,
                        int n_embd, int n_ff, float clamp, int n_wg, hipStream_t s) {
    return fused_go<F, NW, PD, GPT, true>(gate, up, stride, x, n_tok, ids, wts, h, n_tok, k,
                                          n_expert, n_embd, n_ff, clamp, n_wg, s);
}

template <class F, int NW, int PD, int GPT>
static hipError_t down_go(const uint8_t *down, size_t stride, const float *h, const int *ids,
                          const float *wts, float *out, int n_tok, int k, int n_expert, int n_embd,
                          int n_ff, int n_wg, hipStream_t s) {
    return fused_go<F, NW, PD, GPT, false>(down, down, stride, h, n_tok * k, ids, wts, out, n_tok,
                                           k, n_expert, n_ff, n_embd, 0.f, n_wg, s);
}

constexpr int kMoeNW = 16, kMoePD = 2;
// Most token chunks the fused pair is run over before the multi-launch path
// takes over.
constexpr int kMaxFusedChunks = 16;

template <class F>
static bool gu_fits(int n_tok, int k, int n_embd, int n_ff) {
    return moe_fused_lds<F>(n_tok, n_embd, n_ff, min(device_cus(), n_ff), n_tok * k, true) <=
               kMoeMaxLds &&
           moe_gpt<F>(n_tok, n_embd, kMoeNW) != 0;
}
template <class F>
static bool down_fits(int P, int n_ff, int n_embd) {
    return moe_fused_lds<F>(P, n_ff, n_embd, min(device_cus(), n_embd), P, false) <= kMoeMaxLds &&
           moe_gpt<F>(P, n_ff, kMoeNW) != 0;
}

template <class F>
static hipError_t gu_launch(const uint8_t *gate, const uint8_t *up, size_t stride, const float *x,
                            const int *ids, const float *wts, float *h, int n_tok, int k,
                            int n_expert, int n_embd, int n_ff, float clamp, hipStream_t s) {
    const int n_wg = device_cus();
    switch (moe_gpt<F>(n_tok, n_embd, kMoeNW)) {
    case 1: return gu_go<F, kMoeNW, kMoePD, 1>(gate, up, stride, x, ids, wts, h, n_tok, k, n_expert, n_embd, n_ff, clamp, n_wg, s);
    case 2: return gu_go<F, kMoeNW, kMoePD, 2>(gate, up, stride, x, ids, wts, h, n_tok, k, n_expert, n_embd, n_ff, clamp, n_wg, s);
    case 4: return gu_go<F, kMoeNW, kMoePD, 4>(gate, up, stride, x, ids, wts, h, n_tok, k, n_expert, n_embd, n_ff, clamp, n_wg, s);
    default: return hipErrorInvalidValue;
    }
}

template <class F>
static hipError_t down_launch(const uint8_t *down, size_t stride, const float *h, const int *ids,
                              const float *wts, float *out, int n_tok, int k, int n_expert,
                              int n_embd, int n_ff, hipStream_t s) {
    const int n_wg = device_cus();
    switch (moe_gpt<F>(n_tok * k, n_ff, kMoeNW)) {
    case 1: return down_go<F, kMoeNW, kMoePD, 1>(down, stride, h, ids, wts, out, n_tok, k, n_expert, n_embd, n_ff, n_wg, s);
    case 2: return down_go<F, kMoeNW, kMoePD, 2>(down, stride, h, ids, wts, out, n_tok, k, n_expert, n_embd, n_ff, n_wg, s);
    case 4: return down_go<F, kMoeNW, kMoePD, 4>(down, stride, h, ids, wts, out, n_tok, k, n_expert, n_embd, n_ff, n_wg, s);
    default: return hipErrorInvalidValue;
    }
}

#define MOE_FORMATS(X)                                                                             \
    X(T_Q4_K, FQ4K) X(T_Q6_K, FQ6K) X(T_Q8_0, FQ8<false>) X(T_Q4_0, FQ8<true>) X(T_Q2_K, FQ2K)     \
    X(T_IQ2_XXS, FIQ2XXS)

static bool moe_fused_fits(uint32_t dt_gu, uint32_t dt_d, int n_tok, int k, int n_embd, int n_ff,
                           size_t gu_stride, size_t d_stride) {
    if (n_tok * k > kFusedPairs || n_tok > 64) return false;
    if (gu_stride >= ((size_t)1 << 31) || d_stride >= ((size_t)1 << 31)) return false;
    bool a = false, b = false;
#define X(T, F) if (dt_gu == T) a = gu_fits<F>(n_tok, k, n_embd, n_ff); if (dt_d == T) b = down_fits<F>(n_tok * k, n_ff, n_embd);
    MOE_FORMATS(X)
#undef X
    return a && b;
}

static hipError_t moe_fused(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                            const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                            const int *ids, const float *wts, float *out, float *h, int n_tok,
                            int k, int n_expert, int n_embd, int n_ff, float clamp, hipStream_t s) {
    hipError_t e = hipErrorInvalidValue;
#define X(T, F) if (dt_gu == T) e = gu_launch<F>(gate, up, gu_stride, x, ids, wts, h, n_tok, k, n_expert, n_embd, n_ff, clamp, s);
    MOE_FORMATS(X)
#undef X
    if (e != hipSuccess) return e;
    e = hipErrorInvalidValue;
#define X(T, F) if (dt_d == T) e = down_launch<F>(down, d_stride, h, ids, wts, out, n_tok, k, n_expert, n_embd, n_ff, s);
    MOE_FORMATS(X)
#undef X
    return e;
}

// Pairs one pass of the layer takes: longer calls (prefill) run in token
// chunks of at most this many (token, slot) pairs. Tokens are independent, so
// the result is the same as one pass; the chunk bounds the workspace (about
// 44 KB per pair at n_embd 4096, n_ff 2048) and each chunk re-reads the
// experts it routes to.
constexpr int kMoeMaxPairs = 8192;

static int moe_chunk_tokens(int n_tok, int k) {
    const int c = kMoeMaxPairs / k;
    return c < 1 ? 1 : c < n_tok ? c : n_tok;
}

// Workspace of one pass over n_tok tokens.
static size_t moe_pass_bytes(uint32_t dt_gu, uint32_t dt_d, int n_tok, int k, int n_expert,
                             int n_embd, int n_ff) {
    const size_t P = (size_t)n_tok * k;
    size_t b = 0;
    auto add = [&](size_t n) { b += (n + 255) / 256 * 256; };
    add((size_t)(n_expert + 1) * 4);                      // off
    add((size_t)(n_expert + 1) * 4);                      // act, n_act
    add(P * 4);                                           // slot_tok
    add(P * 4);                                           // slot_of
    add(moe_route_work_bytes((int)P, n_expert));          // routing
    add(gemv_scratch_bytes(dt_gu, n_tok, n_embd));        // x limbs
    add(P * n_ff * 4);                                    // hg
    add(P * n_ff * 4);                                    // hu
    add(gemv_scratch_bytes(dt_d, (int)P, n_ff));          // SwiGLU limbs
    add(P * n_embd * 4);                                  // yd
    if (moe_mfma_supported(dt_gu, dt_d, n_embd, n_ff))
        add(moe_mfma_scratch_bytes((int)P, n_expert, n_embd, n_ff));
    return b;
}

size_t moe_scratch_bytes(uint32_t dt_gu, uint32_t dt_d, int n_tok, int k, int n_expert,
                         int n_embd, int n_ff) {
    if (n_tok <= 0 || k <= 0) return 0;
    return moe_pass_bytes(dt_gu, dt_d, moe_chunk_tokens(n_tok, k), k, n_expert, n_embd, n_ff);
}

// Calls of more than kMoeFusedMfmaPairs pairs, and those the fused pair does
// not take in one go, run grouped by expert on the matrix cores (formats
// moe_mfma_supported takes): each expert's weights are streamed once per
// batch of up to 8 or 16 of its slots, where the fused pair over token
// chunks streams them once per chunk that routes to the expert. C3 (64
// experts, top-8) on MI355X, grouped against the fused pair: 66 vs 54 us at
// 1 token, 104 vs 96 us at 2, 136 vs 143 us at 3; against the fused pair's
// token chunks 158 vs 187 us at 4, 204 vs 272 us at 6, 225 vs 335 us at 7
// (one process, one box each).
constexpr int kMoeMfmaMinTok = 1;
constexpr size_t kMoeFusedMfmaPairs = 16;

// Q2_K and IQ2_XXS experts whose rows are not whole super-tiles (in_dim not
// a multiple of 2048) reach the matrix cores without staged weights
// (mf_rows), which loses to the int8-limb routes while few active experts
// hold more than one slot. DS-V4 shapes (IQ2_XXS gate/up, Q2_K down, 4096 /
// 2048, 256 experts, top-6) on mf_rows, int8-limb against matrix cores: 113
// vs 126 us at 4 tokens (24 pairs), 229 vs 228 us at 8 (48), 343 vs 305 us
// at 12 (72), 465 vs 381 us at 16 (one process, one box). So such calls take
// the grouped matrix-core route from n_expert / 5 pairs. Staged, the same
// shapes take it from the fused pair's limit: 92 vs 74 us at 3 tokens, 114
// vs 89 at 4, 229 vs 156 at 8.
static bool moe_mfma_dense_enough(uint32_t dt_gu, uint32_t dt_d, size_t n_pairs, int n_expert,
                                  int n_embd, int n_ff) {
    auto unstaged = [](uint32_t t, int in_dim) {
        return (t == T_Q2_K || t == T_IQ2_XXS) && in_dim % 2048 != 0;
    };
    return !(unstaged(dt_gu, n_embd) || unstaged(dt_d, n_ff)) || n_pairs >= (size_t)n_expert / 5;
}

// One pass over n_tok tokens (n_tok * k <= kMoeMaxPairs).
static hipError_t moe_pass(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                           const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                           const int *ids, const float *wts, float *out, uint8_t *scratch,
                           int n_tok, int k, int n_expert, int n_embd, int n_ff, float clamp,
                           hipStream_t s) {
    const size_t P = (size_t)n_tok * k;
    uint8_t *p = scratch;
    auto take = [&](size_t n) {
        uint8_t *r = p;
        p += (n + 255) / 256 * 256;
        return r;
    };
    int *off = reinterpret_cast<int *>(take((size_t)(n_expert + 1) * 4));
    int *act = reinterpret_cast<int *>(take((size_t)(n_expert + 1) * 4));
    int *n_act = act + n_expert;
    int *slot_tok = reinterpret_cast<int *>(take(P * 4));
    int *slot_of = reinterpret_cast<int *>(take(P * 4));
    uint8_t *route_work = take(moe_route_work_bytes((int)P, n_expert));
    const size_t xq1_bytes = gemv_scratch_bytes(dt_gu, n_tok, n_embd);
    uint8_t *xq1 = take(xq1_bytes);
    float *hg = reinterpret_cast<float *>(take(P * n_ff * 4));
    float *hu = reinterpret_cast<float *>(take(P * n_ff * 4));
    const size_t xq2_bytes = gemv_scratch_bytes(dt_d, (int)P, n_ff);
    uint8_t *xq2 = take(xq2_bytes);
    float *yd = reinterpret_cast<float *>(take(P * n_embd * 4));
    const bool mfma_ok = moe_mfma_supported(dt_gu, dt_d, n_embd, n_ff) &&
                         moe_mfma_fits((int)P, n_embd, n_ff) && n_tok >= kMoeMfmaMinTok &&
                         moe_mfma_dense_enough(dt_gu, dt_d, P, n_expert, n_embd, n_ff) &&
                         gu_stride <= 0xFFFFFFFFu && d_stride <= 0xFFFFFFFFu;
    const bool fused1 = (!mfma_ok || P <= kMoeFusedMfmaPairs) &&
                        moe_fused_fits(dt_gu, dt_d, n_tok, k, n_embd, n_ff, gu_stride, d_stride);
    const bool mfma = !fused1 && mfma_ok;
    if (mfma) {
        uint8_t *mscratch = take(moe_mfma_scratch_bytes((int)P, n_expert, n_embd, n_ff));
        MfgBatch *bat = reinterpret_cast<MfgBatch *>(mscratch);
        const int bw = mfg_width((int)P, n_expert);
        int *n_bat = reinterpret_cast<int *>(mscratch + mfg_batch_bytes((int)P, n_expert, bw) - 256);
        hipError_t e;
        // up to kRoute1Pairs pairs the routing runs inside the route's first
        // launch, beside the x image
        const bool route1 = P <= (size_t)kRoute1Pairs && n_expert <= kRoute1Experts;
        const MoeRoute1Args ra{ids, wts, (int)P, k, n_expert, off, slot_tok, slot_of, act, n_act};
        if (!route1 && (e = launch_moe_route(ids, wts, (int)P, k, n_expert, route_work, off,
                                             slot_tok, slot_of, act, n_act, bat, n_bat, bw, s)) !=
                           hipSuccess)
            return e;
        if ((e = launch_moe_mfma(dt_gu, dt_d, gate, up, down, gu_stride, d_stride, x, n_tok,
                                 route1 ? &ra : nullptr, off, slot_tok, bat, n_bat, (int)P,
                                 n_expert, hg, hu, yd, mscratch, n_embd, n_ff, clamp, s)) !=
            hipSuccess)
            return e;
        return launch_moe_accumulate(out, yd, wts, slot_of, n_tok, k, n_embd, s);
    }
    if (fused1)
        return moe_fused(dt_gu, dt_d, gate, up, down, gu_stride, d_stride, x, ids, wts, out, hg,
                         n_tok, k, n_expert, n_embd, n_ff, clamp, s);
    // More tokens than the fused pair takes: the fused pair over token
    // chunks when few chunks cover them (tokens are independent; each chunk
    // re-reads the experts it shares with the others).
    int tc = n_tok;
    while (tc > 1 && !moe_fused_fits(dt_gu, dt_d, tc, k, n_embd, n_ff, gu_stride, d_stride)) tc--;
    if (moe_fused_fits(dt_gu, dt_d, tc, k, n_embd, n_ff, gu_stride, d_stride) &&
        (n_tok + tc - 1) / tc <= kMaxFusedChunks) {
        for (int t0 = 0; t0 < n_tok; t0 += tc) {
            const int nt = n_tok - t0 < tc ? n_tok - t0 : tc;
            const hipError_t e =
                moe_fused(dt_gu, dt_d, gate, up, down, gu_stride, d_stride, x + (size_t)t0 * n_embd,
                          ids + (size_t)t0 * k, wts + (size_t)t0 * k, out + (size_t)t0 * n_embd,
                          hg, nt, k, n_expert, n_embd, n_ff, clamp, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // at most min(n_expert, n_tok * k) experts are active
    const int grid_experts = (int)(P < (size_t)n_expert ? P : (size_t)n_expert);
    hipError_t e = launch_moe_route(ids, wts, (int)P, k, n_expert, route_work, off, slot_tok,
                                    slot_of, act, n_act, nullptr, nullptr, 0, s);
    if (e != hipSuccess) return e;
    if ((e = launch_quantize_x(dt_gu, x, xq1, n_tok, n_embd, s)) != hipSuccess) return e;
    if ((e = launch_gemv_grouped(dt_gu, gate, up, gu_stride, xq1, xq1_bytes, off, slot_tok, act,
                                 n_act, grid_experts, hg, hu, n_embd, n_ff, s)) != hipSuccess)
        return e;
    if ((e = launch_quantize_swiglu(dt_d, hg, hu, clamp, xq2, (int)P, n_ff, off, n_expert, s)) !=
        hipSuccess)
        return e;
    if ((e = launch_gemv_grouped(dt_d, down, nullptr, d_stride, xq2, xq2_bytes, off, nullptr, act,
                                 n_act, grid_experts, yd, nullptr, n_ff, n_embd, s)) != hipSuccess)
        return e;
    return launch_moe_accumulate(out, yd, wts, slot_of, n_tok, k, n_embd, s);
}

hipError_t launch_moe(uint32_t dt_gu, uint32_t dt_d, const uint8_t *gate, const uint8_t *up,
                      const uint8_t *down, size_t gu_stride, size_t d_stride, const float *x,
                      const int *ids, const float *wts, float *out, uint8_t *scratch, int n_tok,
                      int k, int n_expert, int n_embd, int n_ff, float clamp, hipStream_t s) {
    if (n_tok <= 0 || k <= 0) return hipSuccess;
    const int ct = moe_chunk_tokens(n_tok, k);
    for (int t0 = 0; t0 < n_tok; t0 += ct) {
        const int nt = n_tok - t0 < ct ? n_tok - t0 : ct;
        const hipError_t e =
            moe_pass(dt_gu, dt_d, gate, up, down, gu_stride, d_stride, x + (size_t)t0 * n_embd,
                     ids + (size_t)t0 * k, wts + (size_t)t0 * k, out + (size_t)t0 * n_embd,
                     scratch, nt, k, n_expert, n_embd, n_ff, clamp, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---- shared expert (apply_shared_expert, moe.rs:422-455) ---------------------
// a[i] = silu(min(g[i], c)) * clamp(u[i], -c, c): apply_swiglu_clamp
// (:515-531) then scalar::swiglu, on gate and up outputs kept apart
// (k_swiglu) or side by side per token (k_swiglu_pair).
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ g,
                                                const float *__restrict__ u,
                                                float *__restrict__ a, size_t n, float c) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = swiglu_clamped(g[i], u[i], c);
}

hipError_t launch_swiglu(const float *g, const float *u, float *a, size_t n, float c,
                         hipStream_t s) {
    if (n == 0) return hipSuccess;
    k_swiglu<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(g, u, a, n, c);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_swiglu_pair(const float *__restrict__ h,
                                                     float *__restrict__ a, size_t total, int n,
                                                     float c) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const size_t t = i / (size_t)n, j = i - t * (size_t)n;
    const float *ht = h + t * 2 * (size_t)n;
    a[i] = swiglu_clamped(ht[j], ht[n + j], c);
}

hipError_t launch_swiglu_pair(const float *h, float *a, int n_tok, int n, float c, hipStream_t s) {
    const size_t total = (size_t)n_tok * (size_t)n;
    if (total == 0) return hipSuccess;
    k_swiglu_pair<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(h, a, total, n, c);
    return hipGetLastError();
}

}  // namespace rsllm_hip
