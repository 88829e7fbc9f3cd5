// One-workgroup routing of the routed-expert layer, shared by the routing
// kernel (moe.hip) and the matrix-core route's first launch (gemv_mfma.hip),
// which runs it in workgroup 0 beside the activation image's workgroups.
//
// (t, i) pairs p = t * k + i with w != 0 and an expert id in range get slots
// sorted by expert, ties in pair order (accumulate_moe_outputs,
// rsllm-models/src/dsv4/moe.rs:648-707, visits them per token; the grouping
// is this build's).
#pragma once

#include "kernels.h"

namespace rsllm_hip {

// Exclusive scan of v[0..n) in place by the whole workgroup (kScanThreads
// threads), returning the total; `part` holds kScanThreads ints of LDS (the
// first kScanThreads / 64 are used). Each thread sums a contiguous segment;
// the per-thread sums are scanned within each wavefront (six shuffle-up
// steps), the wavefront totals by every thread in turn (16 adds), so the
// scan costs two barriers plus the final one. Integer sums: the order does
// not change the result.
constexpr int kScanThreads = 1024;
__device__ inline int scan_inplace(int *__restrict__ v, size_t n, int *part) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const size_t seg = (n + kScanThreads - 1) / kScanThreads;
    const size_t lo = min(n, (size_t)tid * seg), hi = min(n, lo + seg);
    int sum = 0;
    for (size_t i = lo; i < hi; i++) sum += v[i];
    // inclusive scan of the per-thread sums within the wavefront
    int inc = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int add = __shfl_up(inc, (unsigned)d, 64);
        if (lane >= d) inc += add;
    }
    if (lane == 63) part[wv] = inc;
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; w++) {
        const int t = part[w];
        base += w < wv ? t : 0;
        total += t;
    }
    int run = base + inc - sum;  // exclusive prefix of this thread's segment
    for (size_t i = lo; i < hi; i++) {
        const int c = v[i];
        v[i] = run;
        run += c;
    }
    __syncthreads();
    return total;
}

// The whole routing in one workgroup of kScanThreads threads, for calls of
// up to kRoute1Pairs pairs and kRoute1Experts experts (decode batches):
// counts, ranks and offsets in LDS, then the scatter, the active experts
// and (bat given) the batches, written as the three-launch routing writes
// them: off[e] (n_expert + 1 entries), slot_tok[slot] = t, slot_of[p] = slot
// or -1, act / *n_act the active experts ascending, bat / *n_bat each
// active expert's slots cut into batches of up to bw. LDS: sh holds
// 2 n_expert ints, ep kRoute1Pairs, part kScanThreads.
constexpr int kRoute1Pairs = 512;
constexpr int kRoute1Experts = 4096;
__device__ inline void moe_route1(const int *__restrict__ ids, const float *__restrict__ wts,
                                  int n_pairs, int k, int n_expert, int *__restrict__ off,
                                  int *__restrict__ slot_tok, int *__restrict__ slot_of,
                                  int *__restrict__ act, int *__restrict__ n_act,
                                  MfgBatch *__restrict__ bat, int *__restrict__ n_bat, int bw,
                                  int *sh, int *ep, int *part) {
    int *base = sh, *flags = sh + n_expert;
    const int tid = threadIdx.x;
    for (int x = tid; x < n_expert; x += kScanThreads) base[x] = 0;
    int e = -1;
    if (tid < n_pairs) {
        const int id = ids[tid];
        if (wts[tid] != 0.0f && id >= 0 && id < n_expert) e = id;
    }
    if (tid < kRoute1Pairs) ep[tid] = e;
    __syncthreads();
    // rank: valid pairs of the same expert before this one (pair order)
    int r = 0;
    if (e >= 0) {
        atomicAdd(&base[e], 1);
        for (int q = 0; q < tid; q++) r += ep[q] == e ? 1 : 0;
    }
    __syncthreads();
    const int total = scan_inplace(base, (size_t)n_expert, part);
    for (int x = tid; x < n_expert; x += kScanThreads) off[x] = base[x];
    if (tid == 0) off[n_expert] = total;
    if (tid < n_pairs) {
        const int slot = e >= 0 ? base[e] + r : -1;
        if (e >= 0) slot_tok[slot] = tid / k;
        slot_of[tid] = slot;
    }
    auto count = [&](int x) { return (x + 1 < n_expert ? base[x + 1] : total) - base[x]; };
    // active experts: positions from a scan of the 0/1 flags
    for (int x = tid; x < n_expert; x += kScanThreads) flags[x] = count(x) > 0 ? 1 : 0;
    __syncthreads();
    const int na = scan_inplace(flags, (size_t)n_expert, part);
    for (int x = tid; x < n_expert; x += kScanThreads) {
        const int next = x + 1 < n_expert ? flags[x + 1] : na;
        if (next != flags[x]) act[flags[x]] = x;
    }
    if (tid == 0) *n_act = na;
    if (!bat) return;
    __syncthreads();
    // batches: positions from a scan of ceil(count / bw)
    for (int x = tid; x < n_expert; x += kScanThreads) flags[x] = (count(x) + bw - 1) / bw;
    __syncthreads();
    const int nb = scan_inplace(flags, (size_t)n_expert, part);
    for (int x = tid; x < n_expert; x += kScanThreads) {
        const int c = count(x);
        for (int f = 0, j = flags[x]; f < c; f += bw, j++)
            bat[j] = MfgBatch{base[x] + f, c - f < bw ? c - f : bw, x, 0};
    }
    if (tid == 0) *n_bat = nb;
}

// Arguments of the routing that the matrix-core route's first launch runs
// in its workgroup 0 (moe_route1's, minus the LDS).
struct MoeRoute1Args {
    const int *ids;
    const float *wts;
    int n_pairs, k, n_expert;
    int *off, *slot_tok, *slot_of, *act, *n_act;
};

}  // namespace rsllm_hip
