// C-ABI entry points: argument validation in the reference's order, process
// state (device, registered weights), per-thread streams and staging, and
// dispatch to the kernel launchers.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/rsllm_hip.h"
#include "abi_internal.h"
#include "kernels.h"

using namespace rsllm_hip;

namespace {

// ---- error state (per thread) -------------------------------------------
struct ErrState {
    rsllm_hip_error_detail d{};
    std::string msg;
};
thread_local ErrState g_err;

int set_err(int status, const char *msg, const char *what = nullptr, size_t a = 0, size_t b = 0,
            size_t src = 0, size_t exp = 0) {
    g_err.msg = msg ? msg : "";
    g_err.d.status = status;
    g_err.d.message = g_err.msg.c_str();
    g_err.d.what = what;
    g_err.d.actual = a;
    g_err.d.block = b;
    g_err.d.src_bytes = src;
    g_err.d.expected_bytes = exp;
    return status;
}

int ok() { return set_err(RSLLM_HIP_OK, ""); }

int dev_err(hipError_t e, const char *where) {
    std::string m = std::string(where) + ": " + hipGetErrorString(e);
    return set_err(RSLLM_HIP_ERR_DEVICE, m.c_str());
}

#define HIP_TRY(expr, where)                         \
    do {                                             \
        hipError_t e_ = (expr);                      \
        if (e_ != hipSuccess) return dev_err(e_, where); \
    } while (0)

// ---- process state --------------------------------------------------------
std::mutex g_mu;
int g_device = 0;
bool g_inited = false;

// Host tensors with a device copy, keyed by host address. owner 0:
// rsllm_hip_register_weights (the entry's own allocation); otherwise the id
// of the uploaded model whose arena holds dev. `keep` shares ownership of the
// device memory: a call that found the entry holds its own reference until it
// has synchronised, so a release running meanwhile frees nothing it reads.
struct Registered {
    size_t len;
    uint32_t dtype;
    size_t in_dim;
    const uint8_t *dev;
    uint64_t owner;
    std::shared_ptr<void> keep;
};
std::unordered_multimap<const uint8_t *, Registered> g_registry;

// A registered device copy held for the length of one call.
struct Lease {
    const uint8_t *dev = nullptr;
    std::shared_ptr<void> keep;
    explicit operator bool() const { return dev != nullptr; }
};

// ---- device allocations ----------------------------------------------------
std::atomic<uint64_t> g_dev_allocs{0};

// ---- per-thread state -----------------------------------------------------
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        size_t want = n < 4096 ? 4096 : n;
        hipError_t e = abi::dev_malloc(&p, want);
        if (e == hipSuccess) cap = want;
        return e;
    }
};

// Per calling thread: the stream and host<->device staging of the
// host-pointer entry points (each such call synchronises before it returns).
struct ThreadCtx {
    int device = -1;
    hipStream_t stream = nullptr;
    DevBuf w_raw, w_dev, x, y, moe_in, moe_w[3];
};
thread_local ThreadCtx t_ctx;

// Device workspace of the kernels (activation images, MoE tables and
// intermediates), one set per (device, stream). Work on one stream runs in
// order, so every call enqueued on that stream can use the same set; `mu` is
// held while a call sizes the set and enqueues, so threads that share a
// stream take turns, and calls on different streams never share a set. A
// buffer that grows is freed with hipFree, which waits for the device first.
struct Scratch {
    std::mutex mu;
    DevBuf xq, xh, moe;
    ~Scratch() {
        for (DevBuf *b : {&xq, &xh, &moe})
            if (b->p) (void)hipFree(b->p);
    }
};
std::mutex g_scratch_map_mu;
// Key of a workspace set: (device, stream handle, thread tag). The special
// handle hipStreamPerThread names a different stream in every thread, so
// its sets also carry the calling thread's tag (0 for every other handle).
using ScratchKey = std::tuple<int, hipStream_t, uint64_t>;
// never destroyed: its buffers are freed only by rsllm_hip_stream_release,
// not at process exit (when the HIP runtime may already be gone)
auto *g_scratch_map = new std::map<ScratchKey, std::shared_ptr<Scratch>>();
std::atomic<uint64_t> g_thread_tags{0};
ScratchKey scratch_key(int dev, hipStream_t st) {
    thread_local const uint64_t tag = ++g_thread_tags;
    return ScratchKey{dev, st, st == hipStreamPerThread ? tag : 0};
}

// The current device's set for stream `st`, locked for the caller.
struct ScratchLease {
    std::shared_ptr<Scratch> keep;
    std::unique_lock<std::mutex> lk;
    Scratch *operator->() const { return keep.get(); }
    Scratch &operator*() const { return *keep; }
};
ScratchLease stream_scratch(hipStream_t st) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::shared_ptr<Scratch> sc;
    {
        std::lock_guard<std::mutex> lk(g_scratch_map_mu);
        auto &p = (*g_scratch_map)[scratch_key(dev, st)];
        if (!p) p = std::make_shared<Scratch>();
        sc = p;
    }
    ScratchLease l{sc, std::unique_lock<std::mutex>(sc->mu)};
    return l;
}

int ensure_device() {
    int dev;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_inited = true;
        dev = g_device;
    }
    HIP_TRY(hipSetDevice(dev), "hipSetDevice");
    if (t_ctx.device != dev || !t_ctx.stream) {
        HIP_TRY(hipStreamCreateWithFlags(&t_ctx.stream, hipStreamNonBlocking), "hipStreamCreate");
        t_ctx.device = dev;
    }
    return RSLLM_HIP_OK;
}

bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

// ---- static workspace of the no-allocation entry point ---------------------
// One copy of `scratch` per GPU, held until the process ends. In host code the
// array's name is not a device address: the address hipGetSymbolAddress gives
// for a device (looked up once per device, with that device current) is the
// only one passed to kernels.
constexpr size_t kNoAllocScratchBytes = RSLLM_HIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// Address of `scratch` on device `dev`, which must be current.
int noalloc_scratch(int dev, uint8_t **p) {
    if (dev < 0 || dev >= kMaxDevices)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return dev_err(e, "hipGetSymbolAddress(scratch)");
        if (!ptr) return set_err(RSLLM_HIP_ERR_DEVICE, "hipGetSymbolAddress(scratch): null");
        g_scratch_ptr[dev] = static_cast<uint8_t *>(ptr);
    }
    *p = g_scratch_ptr[dev];
    return RSLLM_HIP_OK;
}

// The process's device made current, without creating a stream or touching
// any allocator.
int current_device_noalloc(int *dev_out) {
    int dev;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_inited = true;
        dev = g_device;
    }
    int cur = -1;
    HIP_TRY(hipGetDevice(&cur), "hipGetDevice");
    if (cur != dev) HIP_TRY(hipSetDevice(dev), "hipSetDevice");
    *dev_out = dev;
    return RSLLM_HIP_OK;
}

bool mul_ok(size_t a, size_t b, size_t *r) { return !__builtin_mul_overflow(a, b, r); }

// dtypes matmul_quant_f32 accepts (quant_matmul.rs:57-64), and which of
// them this backend implements.
bool matmul_dtype_known(uint32_t t) {
    return t == T_Q4_K || t == T_Q2_K || t == T_IQ2_XXS || t == T_Q4_0 || t == T_Q8_0 ||
           t == T_Q6_K;
}
bool matmul_dtype_impl(uint32_t t) {
    return t == T_Q4_K || t == T_Q8_0 || t == T_Q4_0 || t == T_Q6_K || t == T_Q2_K ||
           t == T_IQ2_XXS;
}

// Shared validation of matmul_quant_f32 (quant_matmul.rs:57-92), then the
// parallel.rs:44 row_len > 0 assertion.
int validate_matmul(size_t out_len, const void *w, size_t w_len, const void *x, size_t x_len,
                    const void *out, size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype) {
    if (!matmul_dtype_known(dtype))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_quant_f32: unsupported dtype for MoE expert matmul");
    const size_t be = block_elems_of(dtype);
    if (in_dim % be != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", in_dim, be);
    size_t need;
    if (!mul_ok(out_dim, row_bytes_of(dtype, in_dim), &need) || w_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_quant_f32: weights must be out_dim * (in_dim / block_elem * "
                       "block_bytes)");
    if (!mul_ok(n_tok, in_dim, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_quant_f32: x must be n_tok * in_dim");
    if (!mul_ok(n_tok, out_dim, &need) || out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_quant_f32: out must be n_tok * out_dim");
    if (out_dim == 0)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "for_each_row_mut: row_len must be non-zero (out_dim == 0)");
    if ((w_len && !w) || (x_len && !x) || (out_len && !out))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    if (!matmul_dtype_impl(dtype))
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED,
                       "matmul_quant_f32: dtype accepted by the reference is not implemented by "
                       "the HIP backend");
    if (!fits_int(n_tok) || !fits_int(in_dim) || !fits_int(out_dim))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_quant_f32: dimension exceeds 2^31-1");
    if (w_len > kMaxWeightBytes)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_quant_f32: weight tensors above 4 GiB are not supported");
    return RSLLM_HIP_OK;
}

const char *ggml_name(uint32_t t) {
    switch (t) {
    case 0: return "f32"; case 1: return "f16"; case 2: return "q4_0"; case 3: return "q4_1";
    case 6: return "q5_0"; case 7: return "q5_1"; case 8: return "q8_0"; case 9: return "q8_1";
    case 10: return "q2_k"; case 11: return "q3_k"; case 12: return "q4_k"; case 13: return "q5_k";
    case 14: return "q6_k"; case 15: return "q8_k"; case 16: return "iq2_xxs";
    case 30: return "bf16";
    default: return "unknown";
    }
}

// dequant_to_f32's dispatch and size rule (dequant/mod.rs:69-85,
// q4_k.rs:36-49, float.rs check_size).
int validate_dequant(uint32_t dtype, const void *src, size_t src_len, const void *dst,
                     size_t dst_len) {
    // every arm of the reference's dispatch (mod.rs:71-84)
    const bool impl = dtype == T_F32 || dtype == T_F16 || dtype == T_BF16 || dtype == T_Q4_0 ||
                      dtype == T_Q4_1 || dtype == T_Q4_K || dtype == T_Q5_K || dtype == T_Q6_K ||
                      dtype == T_Q8_0 || dtype == T_Q2_K || dtype == T_Q8_K || dtype == T_IQ2_XXS;
    if (!impl) {
        std::string m = std::string("dtype `") + ggml_name(dtype) +
                        "` is not yet supported for dequantization in this build";
        return set_err(RSLLM_HIP_ERR_UNSUPPORTED_DEQUANT, m.c_str(), ggml_name(dtype));
    }
    const size_t be = block_elems_of(dtype), bb = block_bytes_of(dtype);
    size_t expected;
    if (be > 1 && dst_len % be != 0) {
        expected = (dst_len + be - 1) / be * bb;
        return set_err(RSLLM_HIP_ERR_DEQUANT_SIZE_MISMATCH, "dequant size mismatch", nullptr, 0, 0,
                       src_len, expected);
    }
    if (!mul_ok(dst_len / be, bb, &expected) || src_len != expected)
        return set_err(RSLLM_HIP_ERR_DEQUANT_SIZE_MISMATCH, "dequant size mismatch", nullptr, 0, 0,
                       src_len, expected);
    if ((src_len && !src) || (dst_len && !dst))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    return RSLLM_HIP_OK;
}

Lease find_registered(const uint8_t *host, size_t len, uint32_t dtype, size_t in_dim) {
    std::lock_guard<std::mutex> lk(g_mu);
    const auto range = g_registry.equal_range(host);
    for (auto it = range.first; it != range.second; ++it) {
        const Registered &r = it->second;
        if (r.len == len && r.dtype == dtype && r.in_dim == in_dim) return Lease{r.dev, r.keep};
    }
    return Lease{};
}

bool needs_prepare(uint32_t dtype) { return dtype != T_Q4_K; }

// A host weight blob on the device for one call: its registered copy, else
// uploaded into `dst` (quant formats other than Q4_K converted to the device
// layout through the w_raw staging buffer). F32 blobs are uploaded as is.
int blob_on_device(const uint8_t *blob, size_t len, uint32_t dtype, size_t in_dim, DevBuf &dst,
                   Lease &lease, const uint8_t **dev) {
    ThreadCtx &c = t_ctx;
    if ((lease = find_registered(blob, len, dtype, in_dim))) {
        *dev = lease.dev;
        return RSLLM_HIP_OK;
    }
    HIP_TRY(dst.ensure(len), "hipMalloc");
    if (dtype == T_F32 || !needs_prepare(dtype) || in_dim == 0) {
        if (len)
            HIP_TRY(hipMemcpyAsync(dst.p, blob, len, hipMemcpyHostToDevice, c.stream),
                    "upload weights");
    } else {
        HIP_TRY(c.w_raw.ensure(len), "hipMalloc");
        HIP_TRY(hipMemcpyAsync(c.w_raw.p, blob, len, hipMemcpyHostToDevice, c.stream),
                "upload weights");
        HIP_TRY(launch_prepare(dtype, (const uint8_t *)c.w_raw.p, (uint8_t *)dst.p,
                               len / row_bytes_of(dtype, in_dim), in_dim, c.stream),
                "prepare weights");
    }
    *dev = (const uint8_t *)dst.p;
    return RSLLM_HIP_OK;
}


// ---- caller chain (weight.rs:113-266) --------------------------------------
// matmul_weight_f32: out, x lengths (:121-135), then the F32 arm's weight
// length (:141-146) or matmul_quant_f32 with any error of it reported as
// ShapeMismatch "matmul_weight_f32.quant" (:160-167). matmul_quant_f32's
// out_dim == 0 is a panic in the reference (not an Err) and stays
// INVALID_ARGUMENT, as do NULL pointers; UNIMPLEMENTED passes through.
int validate_weight_f32(size_t out_len, const void *w, size_t w_len, const void *x, size_t x_len,
                        const void *out, size_t n_tok, size_t in_dim, size_t out_dim,
                        uint32_t dtype) {
    size_t need;
    if (!mul_ok(n_tok, out_dim, &need) || out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_weight_f32.out: out must be n_tok * out_dim");
    if (!mul_ok(n_tok, in_dim, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_weight_f32.x: x must be n_tok * in_dim");
    if (dtype == T_F32) {
        size_t e;
        if (!mul_ok(out_dim, in_dim, &e) || !mul_ok(e, 4, &need) || w_len != need)
            return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                           "matmul_weight_f32.weight_f32: weights must be out_dim * in_dim f32");
        if ((w_len && !w) || (x_len && !x) || (out_len && !out))
            return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
        if (!fits_int(n_tok) || !fits_int(in_dim) || !fits_int(out_dim) || w_len > kMaxWeightBytes)
            return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_weight_f32: size exceeds 2^31-1");
        return RSLLM_HIP_OK;
    }
    const int rc = validate_matmul(out_len, w, w_len, x, x_len, out, n_tok, in_dim, out_dim, dtype);
    if (rc == RSLLM_HIP_ERR_SHAPE_MISMATCH || rc == RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED) {
        const std::string m = std::string("matmul_weight_f32.quant: ") + g_err.msg;
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, m.c_str());
    }
    return rc;
}

// matmul_grouped_lora_down (:209-266): x, out lengths, then per group g in
// order grouped_weight_slice (:271-323: alignment of the group's element
// count to the block, the slice's end within the blob) and
// matmul_weight_f32 on the group. The group checks are the same for every g
// except the slice end, so they reduce to: alignment, group 0's end, the
// group matmul's checks, then the last group's end. All of them are
// ShapeMismatch in the reference; n_groups == 0 is Ok.
int validate_lora_down(size_t out_len, const void *w, size_t w_len, const void *x, size_t x_len,
                       const void *out, size_t n_tok, size_t n_groups, size_t group_dim,
                       size_t rank, uint32_t dtype, size_t *stride_out) {
    size_t total_in, total_out, need;
    if (!mul_ok(n_groups, group_dim, &total_in) || !mul_ok(n_tok, total_in, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_grouped_lora_down.x: x must be n_tok * n_groups * group_dim");
    if (!mul_ok(n_groups, rank, &total_out) || !mul_ok(n_tok, total_out, &need) || out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_grouped_lora_down.out: out must be n_tok * n_groups * rank");
    *stride_out = 0;
    if (n_groups == 0) return RSLLM_HIP_OK;
    size_t epg;
    if (!mul_ok(group_dim, rank, &epg))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "grouped_weight_slice: size overflow");
    size_t stride;
    const char *end_key;
    if (dtype == T_F32) {
        if (!mul_ok(epg, 4, &stride))
            return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "grouped_weight_slice: size overflow");
        end_key = "grouped_weight_slice.f32: the group's slice ends past the blob";
    } else {
        const size_t be = block_elems_of(dtype), bb = block_bytes_of(dtype);
        if (be == 0 || !matmul_dtype_known(dtype))
            return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                           "matmul_weight_f32.quant: unsupported dtype for MoE expert matmul");
        if (epg % be != 0)
            return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                           "grouped_weight_slice.alignment: group_dim * rank is not a multiple "
                           "of the block");
        stride = epg / be * bb;
        end_key = "grouped_weight_slice.quant: the group's slice ends past the blob";
    }
    if (stride > w_len) return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, end_key);
    // group 0's matmul_weight_f32 (its out and x lengths match by construction)
    size_t o0, x0;
    if (!mul_ok(n_tok, rank, &o0) || !mul_ok(n_tok, group_dim, &x0))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_grouped_lora_down: size overflow");
    int rc = validate_weight_f32(o0, w, stride, x, x0, out, n_tok, group_dim, rank, dtype);
    if (rc) return rc;
    if (!mul_ok(n_groups, stride, &need) || need > w_len)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, end_key);
    if (need > kMaxWeightBytes)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_grouped_lora_down: stacked weights above 4 GiB are not supported");
    if (!fits_int(total_in) || !fits_int(total_out) || !mul_ok(n_tok, total_in, &need) ||
        !fits_int(need) || !mul_ok(n_tok, total_out, &need) || !fits_int(need))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_grouped_lora_down: size exceeds 2^31-1");
    *stride_out = stride;
    return RSLLM_HIP_OK;
}

// matmul_weight_f32 on device pointers (validated).
int weight_f32_compute(float *out, size_t out_len, const uint8_t *w, size_t w_len, const float *x,
                       size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype, hipStream_t s,
                       Scratch &sc) {
    if (n_tok == 0 || out_dim == 0) return ok();
    if (in_dim == 0) {  // every dot is empty
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    if (dtype == T_F32) {
        HIP_TRY(launch_gemv_f32((const float *)w, x, out, (int)n_tok, (int)in_dim, (int)out_dim,
                                (int)in_dim, (int)in_dim, (int)out_dim, (int)out_dim, s),
                "gemv_f32");
        return ok();
    }
    HIP_TRY(sc.xq.ensure(gemv_work_bytes(dtype, (int)n_tok, (int)in_dim, (int)out_dim)), "hipMalloc");
    HIP_TRY(launch_gemv(dtype, w, w_len, x, (uint8_t *)sc.xq.p, out, (int)n_tok, (int)in_dim,
                        (int)out_dim, s),
            "gemv");
    return ok();
}

// matmul_grouped_lora_down on device pointers (validated; stride = bytes of
// one group's [rank x group_dim] weights). The stacked blob is the
// [n_groups * rank x group_dim] row-major matrix, so each chunk of up to 8
// tokens is one launch for all groups (workgroups dealt per group, each with
// its group's x in LDS, row r reading x group r / rank). Only when one
// group's x is too long for LDS does each group run its own launch on
// gathered x, scattered into out.
// group_layout: each group's slice was converted to the device layout on its
// own (only the per-group launches read it that way).
int lora_down_compute(float *out, size_t out_len, const uint8_t *w, size_t stride, const float *x,
                      size_t n_tok, size_t n_groups, size_t group_dim, size_t rank,
                      uint32_t dtype, hipStream_t s, Scratch &sc, bool group_layout = false) {
    if (n_tok == 0 || n_groups == 0 || rank == 0) return ok();
    if (group_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    const int T = (int)n_tok, G = (int)n_groups, D = (int)group_dim, R = (int)rank;
    const int tin = G * D, tout = G * R;
    if (dtype == T_F32) {
        HIP_TRY(launch_gemv_f32((const float *)w, x, out, T, D, tout, tin, tin, tout, R, s),
                "gemv_f32");
        return ok();
    }
    hipError_t e = hipErrorNotSupported;
    // 9 or more tokens of the matrix-core formats: one pass over the stacked
    // matrix per 16 tokens, on the matrix cores
    if (!group_layout && lora_mfma_supported(dtype, T, D, G, R)) {
        HIP_TRY(sc.xq.ensure(lora_mfma_scratch_bytes(T, D, G)), "hipMalloc");
        e = launch_lora_mfma(dtype, w, stride * n_groups, x, tin, out, tout, (uint8_t *)sc.xq.p, T,
                             D, G, R, s);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return dev_err(e, "lora_mfma");
        (void)hipGetLastError();
    }
    if (!group_layout) {
        e = launch_gemv_rows(dtype, w, stride * n_groups, x, out, T, D, tout, tin, tin, tout, R, s);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return dev_err(e, "gemv_rows");
        (void)hipGetLastError();
    }
    // one launch per group on gathered x: group g's weights are rows
    // [g R, (g + 1) R) of the stacked matrix; in the super-tile layouts that
    // is whole super-tiles only when R * (blocks per row) is a multiple of 8
    if (!group_layout && needs_prepare(dtype) && (rank * (group_dim / block_elems_of(dtype))) % 8 != 0)
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED,
                       "matmul_grouped_lora_down: groups that do not end on a super-tile of the "
                       "device layout, with one group's x too long for LDS");
    HIP_TRY(sc.xh.ensure((size_t)T * D * 4 + (size_t)T * R * 4), "hipMalloc");
    HIP_TRY(sc.xq.ensure(gemv_work_bytes(dtype, T, D, R)), "hipMalloc");
    float *xg = (float *)sc.xh.p, *yg = xg + (size_t)T * D;
    for (int g = 0; g < G; g++) {
        const uint8_t *wg = w + (size_t)g * stride;
        HIP_TRY(hipMemcpy2DAsync(xg, (size_t)D * 4, x + (size_t)g * D, (size_t)tin * 4,
                                 (size_t)D * 4, (size_t)T, hipMemcpyDeviceToDevice, s),
                "gather x");
        HIP_TRY(launch_gemv(dtype, wg, stride, xg, (uint8_t *)sc.xq.p, yg, T, D, R, s), "gemv");
        HIP_TRY(hipMemcpy2DAsync(out + (size_t)g * R, (size_t)tout * 4, yg, (size_t)R * 4,
                                 (size_t)R * 4, (size_t)T, hipMemcpyDeviceToDevice, s),
                "scatter y");
    }
    return ok();
}

// ---- shared expert (moe.rs:422-502) ------------------------------------------
// check_moe_shapes (:557-573: x, then out), then the matmul_weight_f32
// checks of the first token's gate (n_embd -> n_ff), up and down (n_ff ->
// n_embd) calls, which are the same for every token; n_tok == 0 runs no
// matmul and is Ok.
int validate_shared(size_t out_len, const void *out, size_t x_len, const void *x,
                    const uint8_t *gate, size_t gate_len, uint32_t dt_gate, const uint8_t *up,
                    size_t up_len, uint32_t dt_up, const uint8_t *down, size_t down_len,
                    uint32_t dt_down, size_t n_tok, size_t n_embd, size_t n_ff) {
    static const float kInternal = 0.f;  // stands for the h_gate / h_up / h_act scratch
    size_t need;
    if (!mul_ok(n_tok, n_embd, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe.x: x must be n_tok * n_embd");
    if (out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe.out: out must be n_tok * n_embd");
    if (n_tok == 0) return RSLLM_HIP_OK;
    int rc = validate_weight_f32(n_ff, gate, gate_len, x, n_embd, &kInternal, 1, n_embd, n_ff,
                                 dt_gate);
    if (!rc) rc = validate_weight_f32(n_ff, up, up_len, x, n_embd, &kInternal, 1, n_embd, n_ff,
                                      dt_up);
    if (!rc) rc = validate_weight_f32(n_embd, down, down_len, &kInternal, n_ff, out, 1, n_ff,
                                      n_embd, dt_down);
    if (rc) return rc;
    if (!mul_ok(n_tok, n_ff, &need) || !fits_int(need) || !fits_int(n_tok * n_embd))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "apply_shared_expert: size exceeds 2^31-1");
    return RSLLM_HIP_OK;
}

// apply_shared_expert on device pointers (validated). Gate and up of one
// quant format run as one launch per chunk of up to 8 tokens (the two
// matrices as two row groups of one GEMV on the same x, h = [gate | up] per
// token), then the clamped SwiGLU and the down projection; other
// combinations (F32 blobs, mixed formats) run gate and up through
// matmul_weight_f32 separately.
int shared_compute(float *out, const float *x, const uint8_t *gate, size_t gate_len,
                   uint32_t dt_gate, const uint8_t *up, size_t up_len, uint32_t dt_up,
                   const uint8_t *down, size_t down_len, uint32_t dt_down, size_t n_tok,
                   size_t n_embd, size_t n_ff, float clamp, hipStream_t s, Scratch &sc) {
    if (n_tok == 0 || n_embd == 0) return ok();
    const int T = (int)n_tok, E = (int)n_embd, FF = (int)n_ff;
    // gate and up of one quant format as one paired launch per chunk of up
    // to 8 tokens; from 9 tokens the matrix-core formats run gate and up as
    // two matrix-core GEMVs instead (one pass over each matrix per 16 or 32
    // tokens, exact weights)
    const bool mfma_gu = T >= 9 && gemv_mfma_supported(dt_gate, T, E, FF) &&
                         gemv_mfma_supported(dt_up, T, E, FF);
    if (!mfma_gu && dt_gate == dt_up && dt_gate != T_F32 && gate_len == up_len && n_ff &&
        gemv_rows_fits(dt_gate, E)) {
        const size_t hb = (n_tok * n_ff * 8 + 255) / 256 * 256;
        HIP_TRY(sc.xh.ensure(hb + n_tok * n_ff * 4 + 256), "hipMalloc");
        float *h = (float *)sc.xh.p, *act = (float *)((uint8_t *)sc.xh.p + hb);
        HIP_TRY(launch_gemv_pair(dt_gate, gate, up, gate_len, x, h, T, E, FF, 2 * FF, s),
                "gemv_pair");
        HIP_TRY(launch_swiglu_pair(h, act, T, FF, clamp, s), "swiglu");
        return weight_f32_compute(out, n_tok * n_embd, down, down_len, act, n_tok, n_ff, n_embd,
                                  dt_down, s, sc);
    }
    const size_t hb = (n_tok * n_ff * 4 + 255) / 256 * 256;
    HIP_TRY(sc.xh.ensure(3 * hb + 256), "hipMalloc");
    float *hg = (float *)sc.xh.p, *hu = (float *)((uint8_t *)sc.xh.p + hb),
          *ha = (float *)((uint8_t *)sc.xh.p + 2 * hb);
    int rc = weight_f32_compute(hg, n_tok * n_ff, gate, gate_len, x, n_tok, n_embd, n_ff, dt_gate, s,
                                sc);
    if (!rc)
        rc = weight_f32_compute(hu, n_tok * n_ff, up, up_len, x, n_tok, n_embd, n_ff, dt_up, s, sc);
    if (rc) return rc;
    HIP_TRY(launch_swiglu(hg, hu, ha, n_tok * n_ff, clamp, s), "swiglu");
    return weight_f32_compute(out, n_tok * n_embd, down, down_len, ha, n_tok, n_ff, n_embd,
                              dt_down, s, sc);
}

}  // namespace

// ---- interface for the other host-side files (abi_internal.h) --------------
namespace rsllm_hip::abi {
hipError_t dev_malloc(void **p, size_t bytes) {
    const hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) g_dev_allocs.fetch_add(1, std::memory_order_relaxed);
    return e;
}
int set_error(int status, const char *msg) { return set_err(status, msg); }
int ok_status() { return ok(); }
int device_error(hipError_t e, const char *where) { return dev_err(e, where); }
int ensure_current_device() { return ensure_device(); }
void registry_add(const uint8_t *host, size_t len, uint32_t dtype, size_t in_dim, uint8_t *dev,
                  uint64_t owner, std::shared_ptr<void> keep) {
    std::lock_guard<std::mutex> lk(g_mu);
    const auto range = g_registry.equal_range(host);
    for (auto it = range.first; it != range.second; ++it) {
        const Registered &r = it->second;
        if (r.len == len && r.dtype == dtype && r.in_dim == in_dim && r.dev == dev &&
            r.owner == owner)
            return;
    }
    g_registry.emplace(host, Registered{len, dtype, in_dim, dev, owner, std::move(keep)});
}
void registry_drop_owner(uint64_t owner) {
    std::vector<std::shared_ptr<void>> drop;  // released after the lock
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (auto it = g_registry.begin(); it != g_registry.end();) {
            if (it->second.owner == owner) {
                drop.push_back(std::move(it->second.keep));
                it = g_registry.erase(it);
            } else {
                ++it;
            }
        }
    }
}
DevMem::~DevMem() {
    if (!p) return;
    int cur = -1;
    const bool other = hipGetDevice(&cur) == hipSuccess && cur != device;
    if (other) (void)hipSetDevice(device);
    (void)hipFree(p);
    if (other) (void)hipSetDevice(cur);
}
}  // namespace rsllm_hip::abi

extern "C" {

uint64_t rsllm_hip_device_allocations(void) { return g_dev_allocs.load(std::memory_order_relaxed); }

void rsllm_hip_last_error(rsllm_hip_error_detail *out) {
    if (!out) return;
    *out = g_err.d;
    out->message = g_err.msg.c_str();
}

int rsllm_hip_init(int device_ordinal) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return dev_err(e, "hipGetDeviceCount");
    if (device_ordinal < 0 || device_ordinal >= n)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "device ordinal out of range");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_device = device_ordinal;
        g_inited = true;
    }
    int rc = ensure_device();
    if (rc) return rc;
    uint8_t *ws;  // the no-allocation workspace's address on this device
    rc = noalloc_scratch(device_ordinal, &ws);
    return rc ? rc : ok();
}

void rsllm_hip_capability_get(rsllm_hip_capability *out) {
    if (!out) return;
    out->backend = "rocm";
    out->arch = "gfx950";
    out->q4k_matmul = 1;
    out->q6k_matmul = 1;
    out->q8_0_matmul = 1;
    out->q2k_matmul = 1;
    out->iq2xxs_matmul = 1;
    out->fp8_kv_cache = 0;
}

int rsllm_hip_matmul_quant_f32_dev(float *out, size_t out_len, const uint8_t *weights,
                                   size_t weights_len, const float *x, size_t x_len,
                                   size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                   rsllm_hip_stream_t stream) {
    int rc = validate_matmul(out_len, weights, weights_len, x, x_len, out, n_tok, in_dim, out_dim,
                             dtype);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch(s);
    HIP_TRY(sc->xq.ensure(gemv_work_bytes(dtype, (int)n_tok, (int)in_dim, (int)out_dim)), "hipMalloc");
    HIP_TRY(launch_gemv(dtype, weights, weights_len, x, (uint8_t *)sc->xq.p, out, (int)n_tok,
                        (int)in_dim, (int)out_dim, s),
            "gemv");
    return ok();
}

int rsllm_hip_matmul_quant_f32_dev_noalloc(float *out, size_t out_len, const uint8_t *weights,
                                           size_t weights_len, const float *x, size_t x_len,
                                           size_t n_tok, size_t in_dim, size_t out_dim,
                                           uint32_t dtype, rsllm_hip_stream_t stream) {
    int rc = validate_matmul(out_len, weights, weights_len, x, x_len, out, n_tok, in_dim, out_dim,
                             dtype);
    if (rc) return rc;
    const size_t need =
        n_tok && in_dim ? gemv_work_bytes(dtype, (int)n_tok, (int)in_dim, (int)out_dim) : 0;
    if (need > kNoAllocScratchBytes) {
        const std::string m = "matmul_quant_f32_dev_noalloc: the call needs " +
                              std::to_string(need) + " bytes of workspace, above the static " +
                              std::to_string(kNoAllocScratchBytes) + "-byte maximum";
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, m.c_str());
    }
    hipStream_t s = (hipStream_t)stream;
    if (n_tok == 0) return ok();
    int dev;
    if ((rc = current_device_noalloc(&dev))) return rc;
    if (in_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    uint8_t *ws;
    if ((rc = noalloc_scratch(dev, &ws))) return rc;
    HIP_TRY(launch_gemv(dtype, weights, weights_len, x, ws, out, (int)n_tok, (int)in_dim,
                        (int)out_dim, s),
            "gemv");
    return ok();
}

int rsllm_hip_matmul_quant_f32(float *out, size_t out_len, const uint8_t *weights,
                               size_t weights_len, const float *x, size_t x_len, size_t n_tok,
                               size_t in_dim, size_t out_dim, uint32_t dtype, uint32_t tier) {
    (void)tier;  // quant_matmul.rs:55
    int rc = validate_matmul(out_len, weights, weights_len, x, x_len, out, n_tok, in_dim, out_dim,
                             dtype);
    if (rc) return rc;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {  // every dot is empty: 0.0 (quant_matmul.rs:110-114)
        std::memset(out, 0, out_len * sizeof(float));
        return ok();
    }
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    const Lease reg = find_registered(weights, weights_len, dtype, in_dim);
    const uint8_t *dw = reg.dev;
    if (!dw) {
        HIP_TRY(c.w_raw.ensure(weights_len), "hipMalloc");
        HIP_TRY(hipMemcpyAsync(c.w_raw.p, weights, weights_len, hipMemcpyHostToDevice, c.stream),
                "upload weights");
        dw = (const uint8_t *)c.w_raw.p;
        if (needs_prepare(dtype)) {
            HIP_TRY(c.w_dev.ensure(weights_len), "hipMalloc");
            HIP_TRY(launch_prepare(dtype, dw, (uint8_t *)c.w_dev.p, out_dim, in_dim, c.stream),
                    "prepare weights");
            dw = (const uint8_t *)c.w_dev.p;
        }
    }
    HIP_TRY(c.x.ensure(x_len * sizeof(float)), "hipMalloc");
    HIP_TRY(c.y.ensure(out_len * sizeof(float)), "hipMalloc");
    HIP_TRY(hipMemcpyAsync(c.x.p, x, x_len * sizeof(float), hipMemcpyHostToDevice, c.stream),
            "upload x");
    ScratchLease sc = stream_scratch(c.stream);
    HIP_TRY(sc->xq.ensure(gemv_work_bytes(dtype, (int)n_tok, (int)in_dim, (int)out_dim)), "hipMalloc");
    HIP_TRY(launch_gemv(dtype, dw, weights_len, (const float *)c.x.p, (uint8_t *)sc->xq.p,
                        (float *)c.y.p, (int)n_tok, (int)in_dim, (int)out_dim, c.stream),
            "gemv");
    HIP_TRY(hipMemcpyAsync(out, c.y.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

size_t rsllm_hip_xq_bytes(uint32_t dtype, size_t n_tok, size_t in_dim) {
    if (!matmul_dtype_impl(dtype) || !fits_int(n_tok) || !fits_int(in_dim)) return 0;
    return gemv_scratch_bytes(dtype, (int)n_tok, (int)in_dim);
}

int rsllm_hip_quantize_x_dev(uint32_t dtype, const float *x, size_t x_len, size_t n_tok,
                             size_t in_dim, uint8_t *xq, size_t xq_len, rsllm_hip_stream_t stream) {
    if (!matmul_dtype_impl(dtype))
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED, "quantize_x: dtype not implemented");
    const size_t be = block_elems_of(dtype);
    if (in_dim % be != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", in_dim, be);
    size_t need;
    if (!mul_ok(n_tok, in_dim, &need) || x_len != need || !fits_int(n_tok) || !fits_int(in_dim))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "quantize_x: x must be n_tok * in_dim");
    if (xq_len != rsllm_hip_xq_bytes(dtype, n_tok, in_dim))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "quantize_x: xq must be rsllm_hip_xq_bytes");
    if ((x_len && !x) || (xq_len && !xq))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    HIP_TRY(launch_quantize_x(dtype, x, xq, (int)n_tok, (int)in_dim, (hipStream_t)stream),
            "quantize_x");
    return ok();
}

int rsllm_hip_matmul_prequant_dev(float *out, size_t out_len, const uint8_t *weights,
                                  size_t weights_len, const uint8_t *xq, size_t xq_len,
                                  size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                  rsllm_hip_stream_t stream) {
    // Same validation as matmul_quant_f32 with the x length check replaced.
    size_t x_len_equiv;
    if (!mul_ok(n_tok, in_dim, &x_len_equiv)) x_len_equiv = 0;
    int rc = validate_matmul(out_len, weights, weights_len, xq, x_len_equiv, out, n_tok, in_dim,
                             out_dim, dtype);
    if (rc) return rc;
    if (xq_len != rsllm_hip_xq_bytes(dtype, n_tok, in_dim) || (xq_len && !xq))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_prequant: xq must be rsllm_hip_xq_bytes");
    hipStream_t s = (hipStream_t)stream;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    HIP_TRY(launch_gemv_prequant(dtype, weights, weights_len, xq, out, (int)n_tok, (int)in_dim,
                                 (int)out_dim, s),
            "gemv");
    return ok();
}

int rsllm_hip_matmul_q4k_bf16_dev(float *out, size_t out_len, const uint8_t *weights,
                                  size_t weights_len, const uint16_t *x_bf16, size_t x_len,
                                  size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                  rsllm_hip_stream_t stream) {
    int rc = validate_matmul(out_len, weights, weights_len, x_bf16, x_len, out, n_tok, in_dim,
                             out_dim, dtype);
    if (rc) return rc;
    if (dtype != T_Q4_K)
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED,
                       "matmul_q4k_bf16: only Q4_K weights have a prefill GEMM");
    if (x_len > (size_t)INT_MAX)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_q4k_bf16: n_tok * in_dim exceeds 2^31-1");
    if (((uintptr_t)weights | (uintptr_t)x_bf16) & 15)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "matmul_q4k_bf16: weights and x must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch(s);
    HIP_TRY(sc->xh.ensure(prefill_scratch_bytes((int)n_tok, (int)in_dim, (int)out_dim)), "hipMalloc");
    HIP_TRY(launch_prefill_q4k(weights, weights_len, x_bf16, (uint8_t *)sc->xh.p, out,
                               (int)n_tok, (int)in_dim, (int)out_dim, s),
            "prefill_q4k");
    return ok();
}

// Shared validation of the routed-expert entry points, in the order of the
// reference's own checks for the matmuls involved.
static int validate_moe(size_t out_len, size_t x_len, size_t gate_up_len, size_t down_len,
                        size_t ids_len, size_t n_tok, size_t n_embd, size_t n_ff,
                        size_t n_expert, size_t k, uint32_t dt_gu, uint32_t dt_d,
                        const void *out, const void *x, const void *gate, const void *up,
                        const void *down, const void *ids, const void *weights) {
    if (!matmul_dtype_known(dt_gu) || !matmul_dtype_known(dt_d))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "moe_routed: unsupported dtype for MoE expert matmul");
    const size_t be_gu = block_elems_of(dt_gu), be_d = block_elems_of(dt_d);
    if (n_embd % be_gu != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", n_embd, be_gu);
    if (n_ff % be_d != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", n_ff, be_d);
    size_t need, per;
    if (!mul_ok(n_ff, row_bytes_of(dt_gu, n_embd), &per) || !mul_ok(per, n_expert, &need) ||
        gate_up_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "moe_routed: gate/up blobs must be n_expert * n_ff rows of n_embd");
    if (!mul_ok(n_embd, row_bytes_of(dt_d, n_ff), &per) || !mul_ok(per, n_expert, &need) ||
        down_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "moe_routed: down blob must be n_expert * n_embd rows of n_ff");
    if (!mul_ok(n_tok, n_embd, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe_routed: x must be n_tok * n_embd");
    if (out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe_routed: out must be n_tok * n_embd");
    if (!mul_ok(n_tok, k, &need) || ids_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe_routed: ids/weights must be n_tok * k");
    if (n_embd == 0 || n_ff == 0 || n_expert == 0)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "for_each_row_mut: row_len must be non-zero (n_embd, n_ff, n_expert)");
    if ((out_len && (!out || !x)) || (gate_up_len && (!gate || !up)) || (down_len && !down) ||
        (ids_len && (!ids || !weights)))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    if (!matmul_dtype_impl(dt_gu) || !matmul_dtype_impl(dt_d))
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED,
                       "moe_routed: dtype accepted by the reference is not implemented by the "
                       "HIP backend");
    if (n_expert > 16384)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "moe_routed: n_expert above 16384 is not supported");
    if (!fits_int(n_tok) || !fits_int(n_embd) || !fits_int(n_ff) || !fits_int(n_expert) ||
        !fits_int(k) || gate_up_len / n_expert > kMaxWeightBytes ||
        down_len / n_expert > kMaxWeightBytes)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "moe_routed: dimension out of range");
    // the device layout of non-Q4_K formats groups 8 blocks: every expert
    // must start on a group boundary
    if ((dt_gu != T_Q4_K && ((n_ff * (n_embd / be_gu)) % 8 != 0)) ||
        (dt_d != T_Q4_K && ((n_embd * (n_ff / be_d)) % 8 != 0)))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "moe_routed: blocks per expert must be a multiple of 8 for this dtype");
    return RSLLM_HIP_OK;
}

int rsllm_hip_moe_routed_dev(float *out, size_t out_len, const float *x, size_t x_len,
                             const uint8_t *gate, const uint8_t *up, size_t gate_up_len,
                             const uint8_t *down, size_t down_len, const int32_t *ids,
                             const float *weights, size_t ids_len, size_t n_tok, size_t n_embd,
                             size_t n_ff, size_t n_expert, size_t k, uint32_t dtype_gate_up,
                             uint32_t dtype_down, float clamp, rsllm_hip_stream_t stream) {
    int rc = validate_moe(out_len, x_len, gate_up_len, down_len, ids_len, n_tok, n_embd, n_ff,
                          n_expert, k, dtype_gate_up, dtype_down, out, x, gate, up, down, ids,
                          weights);
    if (rc) return rc;
    if (n_tok == 0 || k == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch((hipStream_t)stream);
    HIP_TRY(sc->moe.ensure(moe_scratch_bytes(dtype_gate_up, dtype_down, (int)n_tok, (int)k,
                                             (int)n_expert, (int)n_embd, (int)n_ff)),
            "hipMalloc");
    HIP_TRY(launch_moe(dtype_gate_up, dtype_down, gate, up, down, gate_up_len / n_expert,
                       down_len / n_expert, x, ids, weights, out, (uint8_t *)sc->moe.p,
                       (int)n_tok, (int)k, (int)n_expert, (int)n_embd, (int)n_ff, clamp,
                       (hipStream_t)stream),
            "moe");
    return ok();
}

int rsllm_hip_moe_routed(float *out, size_t out_len, const float *x, size_t x_len,
                         const uint8_t *gate, const uint8_t *up, size_t gate_up_len,
                         const uint8_t *down, size_t down_len, const int32_t *ids,
                         const float *weights, size_t ids_len, size_t n_tok, size_t n_embd,
                         size_t n_ff, size_t n_expert, size_t k, uint32_t dtype_gate_up,
                         uint32_t dtype_down, float clamp) {
    int rc = validate_moe(out_len, x_len, gate_up_len, down_len, ids_len, n_tok, n_embd, n_ff,
                          n_expert, k, dtype_gate_up, dtype_down, out, x, gate, up, down, ids,
                          weights);
    if (rc) return rc;
    for (size_t p = 0; p < ids_len; p++)
        if (weights[p] != 0.0f && (ids[p] < 0 || (size_t)ids[p] >= n_expert))
            return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                           "StackedExperts::expert: expert index out of range");
    if (n_tok == 0 || k == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    // expert blobs: registered device copies, else uploaded (and converted to
    // the device layout) for this call
    const uint8_t *blob[3] = {gate, up, down};
    const size_t blen[3] = {gate_up_len, gate_up_len, down_len};
    const uint32_t bdt[3] = {dtype_gate_up, dtype_gate_up, dtype_down};
    const size_t bin[3] = {n_embd, n_embd, n_ff};
    const uint8_t *dev[3];
    Lease reg[3];
    for (int i = 0; i < 3; i++)
        if ((rc = blob_on_device(blob[i], blen[i], bdt[i], bin[i], c.moe_w[i], reg[i], &dev[i])))
            return rc;
    // inputs: x | out | ids | weights, 256-byte aligned pieces
    const size_t a_x = (x_len * 4 + 255) / 256 * 256, a_o = (out_len * 4 + 255) / 256 * 256;
    const size_t a_i = (ids_len * 4 + 255) / 256 * 256;
    HIP_TRY(c.moe_in.ensure(a_x + a_o + 2 * a_i), "hipMalloc");
    uint8_t *base = (uint8_t *)c.moe_in.p;
    float *d_x = (float *)base, *d_out = (float *)(base + a_x);
    int32_t *d_ids = (int32_t *)(base + a_x + a_o);
    float *d_w = (float *)(base + a_x + a_o + a_i);
    HIP_TRY(hipMemcpyAsync(d_x, x, x_len * 4, hipMemcpyHostToDevice, c.stream), "upload x");
    HIP_TRY(hipMemcpyAsync(d_out, out, out_len * 4, hipMemcpyHostToDevice, c.stream), "upload out");
    HIP_TRY(hipMemcpyAsync(d_ids, ids, ids_len * 4, hipMemcpyHostToDevice, c.stream), "upload ids");
    HIP_TRY(hipMemcpyAsync(d_w, weights, ids_len * 4, hipMemcpyHostToDevice, c.stream),
            "upload weights");
    ScratchLease sc = stream_scratch(c.stream);
    HIP_TRY(sc->moe.ensure(moe_scratch_bytes(dtype_gate_up, dtype_down, (int)n_tok, (int)k,
                                             (int)n_expert, (int)n_embd, (int)n_ff)),
            "hipMalloc");
    HIP_TRY(launch_moe(dtype_gate_up, dtype_down, dev[0], dev[1], dev[2], gate_up_len / n_expert,
                       down_len / n_expert, d_x, d_ids, d_w, d_out, (uint8_t *)sc->moe.p,
                       (int)n_tok, (int)k, (int)n_expert, (int)n_embd, (int)n_ff, clamp, c.stream),
            "moe");
    HIP_TRY(hipMemcpyAsync(out, d_out, out_len * 4, hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

// quantize_q8_0_batch's checks (q8_0.rs:101-118), then the panic of
// par_chunks_mut(0) for in_dim == 0.
static int validate_q8_quantize(const void *x, size_t x_len, const void *xq, size_t xq_len,
                                const void *scale, size_t scale_len, size_t n_tok,
                                size_t in_dim) {
    const size_t blocks = (in_dim + 31) / 32;
    size_t need, nb;
    if (!mul_ok(n_tok, in_dim, &need) || x_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "quantize_q8_0_batch: x must be n_tok*in_dim");
    if (!mul_ok(n_tok, blocks, &nb) || !mul_ok(nb, 32, &need) || xq_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "quantize_q8_0_batch: xq must be n_tok*blocks*32");
    if (scale_len != nb)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "quantize_q8_0_batch: scale must be n_tok*blocks");
    if (in_dim == 0)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "par_chunks_mut: chunk size must be non-zero");
    if ((x_len && !x) || (xq_len && (!xq || !scale)))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    if (!fits_int(xq_len))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "quantize_q8_0_batch: xq exceeds 2^31-1");
    return RSLLM_HIP_OK;
}

// matmul_q8_0_batch's checks (q8_0.rs:229-252), then for_each_row_mut's
// row_len assertion (parallel.rs:44).
static int validate_q8_matmul(const void *out, size_t out_len, const void *w, size_t w_len,
                              const void *xq, size_t xq_len, const void *xscale,
                              size_t xscale_len, size_t n_tok, size_t in_dim, size_t out_dim) {
    const size_t blocks = (in_dim + 31) / 32;
    size_t need, nb;
    if (!mul_ok(out_dim, blocks, &nb) || !mul_ok(nb, 34, &need) || w_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_q8_0_batch: weights must be out_dim*blocks*34");
    if (!mul_ok(n_tok, blocks, &nb) || !mul_ok(nb, 32, &need) || xq_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_q8_0_batch: xq must be n_tok*blocks*32");
    if (xscale_len != nb)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "matmul_q8_0_batch: xscale must be n_tok*blocks");
    if (!mul_ok(n_tok, out_dim, &need) || out_len != need)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_q8_0_batch: out must be n_tok*out_dim");
    if (out_dim == 0)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "for_each_row_mut: row_len must be non-zero (out_dim == 0)");
    if ((w_len && !w) || (xq_len && (!xq || !xscale)) || (out_len && !out))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    if (!fits_int(n_tok) || !fits_int(in_dim) || !fits_int(out_dim) || w_len > kMaxWeightBytes)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH, "matmul_q8_0_batch: dimension out of range");
    return RSLLM_HIP_OK;
}

int rsllm_hip_quantize_q8_0_batch_dev(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                                      float *scale, size_t scale_len, size_t n_tok,
                                      size_t in_dim, int32_t *status, rsllm_hip_stream_t stream) {
    int rc = validate_q8_quantize(x, x_len, xq, xq_len, scale, scale_len, n_tok, in_dim);
    if (rc) return rc;
    if ((((uintptr_t)x | (uintptr_t)scale | (uintptr_t)status) & 3) || ((uintptr_t)xq & 15))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "quantize_q8_0_batch: xq must be 16-byte aligned, x/scale/status 4-byte");
    hipStream_t s = (hipStream_t)stream;
    if (status) HIP_TRY(launch_fill_zero(reinterpret_cast<float *>(status), 1, s), "fill_zero");
    if (n_tok == 0) return ok();
    HIP_TRY(launch_q8_quantize(x, xq, scale, (int)n_tok, (int)in_dim, status, s), "q8_quantize");
    return ok();
}

int rsllm_hip_quantize_q8_0_batch(const float *x, size_t x_len, int8_t *xq, size_t xq_len,
                                  float *scale, size_t scale_len, size_t n_tok, size_t in_dim) {
    int rc = validate_q8_quantize(x, x_len, xq, xq_len, scale, scale_len, n_tok, in_dim);
    if (rc) return rc;
    if (n_tok == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    const size_t a_x = (x_len * 4 + 255) / 256 * 256, a_q = (xq_len + 255) / 256 * 256;
    const size_t a_s = (scale_len * 4 + 255) / 256 * 256;
    HIP_TRY(c.x.ensure(a_x + a_q + a_s + 256), "hipMalloc");
    uint8_t *base = (uint8_t *)c.x.p;
    float *d_x = (float *)base;
    int8_t *d_q = (int8_t *)(base + a_x);
    float *d_s = (float *)(base + a_x + a_q);
    int32_t *d_st = (int32_t *)(base + a_x + a_q + a_s);
    HIP_TRY(hipMemcpyAsync(d_x, x, x_len * 4, hipMemcpyHostToDevice, c.stream), "upload x");
    HIP_TRY(launch_fill_zero(reinterpret_cast<float *>(d_st), 1, c.stream), "fill_zero");
    HIP_TRY(launch_q8_quantize(d_x, d_q, d_s, (int)n_tok, (int)in_dim, d_st, c.stream),
            "q8_quantize");
    int32_t st = 0;
    HIP_TRY(hipMemcpyAsync(xq, d_q, xq_len, hipMemcpyDeviceToHost, c.stream), "download xq");
    HIP_TRY(hipMemcpyAsync(scale, d_s, scale_len * 4, hipMemcpyDeviceToHost, c.stream),
            "download scale");
    HIP_TRY(hipMemcpyAsync(&st, d_st, 4, hipMemcpyDeviceToHost, c.stream), "download status");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    if (st)
        return set_err(RSLLM_HIP_ERR_NON_FINITE_INPUT, "quantize_q8_0: activation");
    return ok();
}

int rsllm_hip_matmul_q8_0_batch_dev(float *out, size_t out_len, const uint8_t *weights,
                                    size_t weights_len, const int8_t *xq, size_t xq_len,
                                    const float *xscale, size_t xscale_len, size_t n_tok,
                                    size_t in_dim, size_t out_dim, rsllm_hip_stream_t stream) {
    int rc = validate_q8_matmul(out, out_len, weights, weights_len, xq, xq_len, xscale,
                                xscale_len, n_tok, in_dim, out_dim);
    if (rc) return rc;
    if ((((uintptr_t)weights | (uintptr_t)xq) & 15) || (((uintptr_t)xscale | (uintptr_t)out) & 3))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                       "matmul_q8_0_batch: weights and xq must be 16-byte aligned, xscale and out "
                       "4-byte");
    hipStream_t s = (hipStream_t)stream;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {
        HIP_TRY(launch_fill_zero(out, out_len, s), "fill_zero");
        return ok();
    }
    HIP_TRY(launch_q8_int8_matmul(weights, weights_len, xq, xscale, out, (int)n_tok, (int)in_dim,
                                  (int)out_dim, s),
            "q8_matmul");
    return ok();
}

int rsllm_hip_matmul_q8_0_batch(float *out, size_t out_len, const uint8_t *weights,
                                size_t weights_len, const int8_t *xq, size_t xq_len,
                                const float *xscale, size_t xscale_len, size_t n_tok,
                                size_t in_dim, size_t out_dim, uint32_t tier) {
    (void)tier;  // every tier returns the scalar tier's result (q8_0.rs:271-296)
    int rc = validate_q8_matmul(out, out_len, weights, weights_len, xq, xq_len, xscale,
                                xscale_len, n_tok, in_dim, out_dim);
    if (rc) return rc;
    if (n_tok == 0) return ok();
    if (in_dim == 0) {  // zero blocks: every dot is 0.0
        std::memset(out, 0, out_len * sizeof(float));
        return ok();
    }
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    // device layout: a registered copy (Q8_0 with this in_dim), else the rows
    // uploaded and regrouped for this call
    const Lease reg = find_registered(weights, weights_len, T_Q8_0, in_dim);
    const uint8_t *dw = reg.dev;
    if (!dw) {
        HIP_TRY(c.w_raw.ensure(weights_len), "hipMalloc");
        HIP_TRY(c.w_dev.ensure(weights_len), "hipMalloc");
        HIP_TRY(hipMemcpyAsync(c.w_raw.p, weights, weights_len, hipMemcpyHostToDevice, c.stream),
                "upload weights");
        HIP_TRY(launch_prepare(T_Q8_0, (const uint8_t *)c.w_raw.p, (uint8_t *)c.w_dev.p, out_dim,
                               (in_dim + 31) / 32 * 32, c.stream),
                "prepare weights");
        dw = (const uint8_t *)c.w_dev.p;
    }
    const size_t a_q = (xq_len + 255) / 256 * 256;
    HIP_TRY(c.x.ensure(a_q + xscale_len * 4), "hipMalloc");
    int8_t *d_q = (int8_t *)c.x.p;
    float *d_s = (float *)((uint8_t *)c.x.p + a_q);
    HIP_TRY(hipMemcpyAsync(d_q, xq, xq_len, hipMemcpyHostToDevice, c.stream), "upload xq");
    HIP_TRY(hipMemcpyAsync(d_s, xscale, xscale_len * 4, hipMemcpyHostToDevice, c.stream),
            "upload xscale");
    HIP_TRY(c.y.ensure(out_len * sizeof(float)), "hipMalloc");
    HIP_TRY(launch_q8_int8_matmul(dw, weights_len, d_q, d_s,
                                  (float *)c.y.p, (int)n_tok, (int)in_dim, (int)out_dim,
                                  c.stream),
            "q8_matmul");
    HIP_TRY(hipMemcpyAsync(out, c.y.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

int rsllm_hip_register_weights(const uint8_t *weights, size_t weights_len, uint32_t dtype,
                               size_t in_dim) {
    if (!matmul_dtype_impl(dtype))
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED, "register_weights: dtype not implemented");
    const size_t be = block_elems_of(dtype);
    if (in_dim == 0 || in_dim % be != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", in_dim, be);
    const size_t rb = row_bytes_of(dtype, in_dim);
    if (weights_len % rb != 0 || (weights_len && !weights))
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "register_weights: length is not a whole number of rows");
    if (find_registered(weights, weights_len, dtype, in_dim)) return ok();
    int rc = ensure_device();
    if (rc) return rc;
    auto mem = std::make_shared<abi::DevMem>();
    HIP_TRY(hipGetDevice(&mem->device), "hipGetDevice");
    HIP_TRY(abi::dev_malloc((void **)&mem->p, weights_len ? weights_len : 1), "hipMalloc");
    hipError_t e;
    if (!needs_prepare(dtype)) {
        e = hipMemcpy(mem->p, weights, weights_len, hipMemcpyHostToDevice);
    } else {
        uint8_t *raw = nullptr;
        e = abi::dev_malloc((void **)&raw, weights_len ? weights_len : 1);
        if (e == hipSuccess) e = hipMemcpy(raw, weights, weights_len, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = launch_prepare(dtype, raw, mem->p, weights_len / rb, in_dim, t_ctx.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(t_ctx.stream);
        if (raw) (void)hipFree(raw);
    }
    if (e != hipSuccess) return dev_err(e, "register_weights");
    // a thread that registered the same tensor meanwhile wins; this copy is
    // then dropped (freed) when `mem` goes out of scope
    if (find_registered(weights, weights_len, dtype, in_dim)) return ok();
    uint8_t *dev = mem->p;
    abi::registry_add(weights, weights_len, dtype, in_dim, dev, 0, std::move(mem));
    return ok();
}

int rsllm_hip_release_weights(void) {
    // the entries' references are dropped after the lock: an allocation no
    // call holds is freed here (hipFree waits for the device first); one a
    // call in flight still holds is freed when that call drops it
    int rc = ensure_device();
    if (rc) return rc;
    abi::registry_drop_owner(0);
    return ok();
}

int rsllm_hip_stream_release(rsllm_hip_stream_t stream) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    std::shared_ptr<Scratch> gone;
    {
        std::lock_guard<std::mutex> lk(g_scratch_map_mu);
        auto it = g_scratch_map->find(scratch_key(dev, (hipStream_t)stream));
        if (it != g_scratch_map->end()) {
            gone = std::move(it->second);
            g_scratch_map->erase(it);
        }
    }
    // freed here, or by the last call still holding the set
    gone.reset();
    return ok();
}

int rsllm_hip_prepare_weights_dev(uint8_t *dst, const uint8_t *src, size_t len, uint32_t dtype,
                                  size_t in_dim, rsllm_hip_stream_t stream) {
    if (!matmul_dtype_impl(dtype))
        return set_err(RSLLM_HIP_ERR_UNIMPLEMENTED, "prepare_weights: dtype not implemented");
    const size_t be = block_elems_of(dtype);
    if (in_dim == 0 || in_dim % be != 0)
        return set_err(RSLLM_HIP_ERR_NOT_BLOCK_ALIGNED, "`in_dim` is not a multiple of the block",
                       "in_dim", in_dim, be);
    const size_t rb = row_bytes_of(dtype, in_dim);
    if (len % rb != 0)
        return set_err(RSLLM_HIP_ERR_SHAPE_MISMATCH,
                       "prepare_weights: length is not a whole number of rows");
    if (len && (!dst || !src))
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "NULL pointer with a nonzero length");
    if (dtype != T_Q4_K && len && dst < src + len && src < dst + len)
        return set_err(RSLLM_HIP_ERR_INVALID_ARGUMENT, "prepare_weights: dst overlaps src");
    HIP_TRY(launch_prepare(dtype, src, dst, len / rb, in_dim, (hipStream_t)stream), "prepare");
    return ok();
}

int rsllm_hip_dequant_to_f32_dev(uint32_t dtype, const uint8_t *src, size_t src_len, float *dst,
                                 size_t dst_len, rsllm_hip_stream_t stream) {
    int rc = validate_dequant(dtype, src, src_len, dst, dst_len);
    if (rc) return rc;
    HIP_TRY(launch_dequant(dtype, src, dst, dst_len, (hipStream_t)stream), "dequant");
    return ok();
}

int rsllm_hip_dequant_to_f32(uint32_t dtype, const uint8_t *src, size_t src_len, float *dst,
                             size_t dst_len) {
    int rc = validate_dequant(dtype, src, src_len, dst, dst_len);
    if (rc) return rc;
    if (dst_len == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    HIP_TRY(c.w_raw.ensure(src_len), "hipMalloc");
    HIP_TRY(c.y.ensure(dst_len * sizeof(float)), "hipMalloc");
    HIP_TRY(hipMemcpyAsync(c.w_raw.p, src, src_len, hipMemcpyHostToDevice, c.stream), "upload");
    HIP_TRY(launch_dequant(dtype, (const uint8_t *)c.w_raw.p, (float *)c.y.p, dst_len, c.stream),
            "dequant");
    HIP_TRY(hipMemcpyAsync(dst, c.y.p, dst_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}


// ---- caller chain -------------------------------------------------------------
int rsllm_hip_matmul_weight_f32_dev(float *out, size_t out_len, const uint8_t *weights,
                                    size_t weights_len, const float *x, size_t x_len,
                                    size_t n_tok, size_t in_dim, size_t out_dim, uint32_t dtype,
                                    rsllm_hip_stream_t stream) {
    int rc = validate_weight_f32(out_len, weights, weights_len, x, x_len, out, n_tok, in_dim,
                                 out_dim, dtype);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch((hipStream_t)stream);
    return weight_f32_compute(out, out_len, weights, weights_len, x, n_tok, in_dim, out_dim, dtype,
                              (hipStream_t)stream, *sc);
}

int rsllm_hip_matmul_weight_f32(float *out, size_t out_len, const uint8_t *weights,
                                size_t weights_len, const float *x, size_t x_len, size_t n_tok,
                                size_t in_dim, size_t out_dim, uint32_t dtype) {
    int rc = validate_weight_f32(out_len, weights, weights_len, x, x_len, out, n_tok, in_dim,
                                 out_dim, dtype);
    if (rc) return rc;
    if (n_tok == 0 || out_dim == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    const Lease reg = find_registered(weights, weights_len, dtype, in_dim);
    const uint8_t *dw = reg.dev;
    if (!dw && weights_len) {
        HIP_TRY(c.w_raw.ensure(weights_len), "hipMalloc");
        HIP_TRY(hipMemcpyAsync(c.w_raw.p, weights, weights_len, hipMemcpyHostToDevice, c.stream),
                "upload weights");
        dw = (const uint8_t *)c.w_raw.p;
        if (dtype != T_F32 && needs_prepare(dtype) && in_dim) {
            HIP_TRY(c.w_dev.ensure(weights_len), "hipMalloc");
            HIP_TRY(launch_prepare(dtype, dw, (uint8_t *)c.w_dev.p, out_dim, in_dim, c.stream),
                    "prepare weights");
            dw = (const uint8_t *)c.w_dev.p;
        }
    }
    HIP_TRY(c.x.ensure(x_len * sizeof(float) + 16), "hipMalloc");
    HIP_TRY(c.y.ensure(out_len * sizeof(float)), "hipMalloc");
    if (x_len)
        HIP_TRY(hipMemcpyAsync(c.x.p, x, x_len * sizeof(float), hipMemcpyHostToDevice, c.stream),
                "upload x");
    ScratchLease sc = stream_scratch(c.stream);
    rc = weight_f32_compute((float *)c.y.p, out_len, dw, weights_len, (const float *)c.x.p, n_tok,
                            in_dim, out_dim, dtype, c.stream, *sc);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(out, c.y.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

int rsllm_hip_matmul_grouped_lora_down_dev(float *out, size_t out_len, const uint8_t *weights,
                                           size_t weights_len, const float *x, size_t x_len,
                                           size_t n_tok, size_t n_groups, size_t group_dim,
                                           size_t rank, uint32_t dtype,
                                           rsllm_hip_stream_t stream) {
    size_t stride;
    int rc = validate_lora_down(out_len, weights, weights_len, x, x_len, out, n_tok, n_groups,
                                group_dim, rank, dtype, &stride);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch((hipStream_t)stream);
    return lora_down_compute(out, out_len, weights, stride, x, n_tok, n_groups, group_dim, rank,
                             dtype, (hipStream_t)stream, *sc);
}

int rsllm_hip_matmul_grouped_lora_down(float *out, size_t out_len, const uint8_t *weights,
                                       size_t weights_len, const float *x, size_t x_len,
                                       size_t n_tok, size_t n_groups, size_t group_dim,
                                       size_t rank, uint32_t dtype) {
    size_t stride;
    int rc = validate_lora_down(out_len, weights, weights_len, x, x_len, out, n_tok, n_groups,
                                group_dim, rank, dtype, &stride);
    if (rc) return rc;
    if (n_tok == 0 || n_groups == 0 || rank == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    // The blob may be longer; the groups use this much. The device layout
    // packs 8 blocks per super-tile with a shorter last one, so a group's
    // slice of the whole matrix's layout is the group's own layout only when
    // the group is whole super-tiles. Groups that are not, and that need the
    // per-group launches (one group's x too long for LDS), are converted one
    // by one. A
    // registered copy (the whole blob's layout) is used only when it is
    // exactly the groups' rows and is not converted per group.
    const size_t used = stride * n_groups;
    const bool prep = dtype != T_F32 && needs_prepare(dtype) && group_dim;
    const bool per_group = prep && (rank * (group_dim / block_elems_of(dtype))) % 8 != 0 &&
                           !gemv_rows_fits(dtype, (int)group_dim);
    const Lease reg = used != weights_len || per_group
                          ? Lease{}
                          : find_registered(weights, weights_len, dtype, group_dim);
    const uint8_t *dw = reg.dev;
    if (!dw) {
        HIP_TRY(c.w_raw.ensure(used), "hipMalloc");
        HIP_TRY(hipMemcpyAsync(c.w_raw.p, weights, used, hipMemcpyHostToDevice, c.stream),
                "upload weights");
        dw = (const uint8_t *)c.w_raw.p;
        if (prep) {
            HIP_TRY(c.w_dev.ensure(used), "hipMalloc");
            uint8_t *wd = (uint8_t *)c.w_dev.p;
            if (!per_group) {
                HIP_TRY(launch_prepare(dtype, dw, wd, n_groups * rank, group_dim, c.stream),
                        "prepare weights");
            } else {
                for (size_t g = 0; g < n_groups; g++)
                    HIP_TRY(launch_prepare(dtype, dw + g * stride, wd + g * stride, rank,
                                           group_dim, c.stream),
                            "prepare weights");
            }
            dw = wd;
        }
    }
    HIP_TRY(c.x.ensure(x_len * sizeof(float) + 16), "hipMalloc");
    HIP_TRY(c.y.ensure(out_len * sizeof(float)), "hipMalloc");
    if (x_len)
        HIP_TRY(hipMemcpyAsync(c.x.p, x, x_len * sizeof(float), hipMemcpyHostToDevice, c.stream),
                "upload x");
    ScratchLease sc = stream_scratch(c.stream);
    rc = lora_down_compute((float *)c.y.p, out_len, dw, stride, (const float *)c.x.p, n_tok,
                           n_groups, group_dim, rank, dtype, c.stream, *sc, per_group);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(out, c.y.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

// ---- shared expert --------------------------------------------------------------
int rsllm_hip_apply_shared_expert_dev(float *out, size_t out_len, const float *x, size_t x_len,
                                      const uint8_t *gate, size_t gate_len, uint32_t dtype_gate,
                                      const uint8_t *up, size_t up_len, uint32_t dtype_up,
                                      const uint8_t *down, size_t down_len, uint32_t dtype_down,
                                      size_t n_tok, size_t n_embd, size_t n_ff, float clamp,
                                      rsllm_hip_stream_t stream) {
    int rc = validate_shared(out_len, out, x_len, x, gate, gate_len, dtype_gate, up, up_len,
                             dtype_up, down, down_len, dtype_down, n_tok, n_embd, n_ff);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    ScratchLease sc = stream_scratch((hipStream_t)stream);
    return shared_compute(out, x, gate, gate_len, dtype_gate, up, up_len, dtype_up, down,
                          down_len, dtype_down, n_tok, n_embd, n_ff, clamp, (hipStream_t)stream,
                          *sc);
}

int rsllm_hip_apply_shared_expert(float *out, size_t out_len, const float *x, size_t x_len,
                                  const uint8_t *gate, size_t gate_len, uint32_t dtype_gate,
                                  const uint8_t *up, size_t up_len, uint32_t dtype_up,
                                  const uint8_t *down, size_t down_len, uint32_t dtype_down,
                                  size_t n_tok, size_t n_embd, size_t n_ff, float clamp) {
    int rc = validate_shared(out_len, out, x_len, x, gate, gate_len, dtype_gate, up, up_len,
                             dtype_up, down, down_len, dtype_down, n_tok, n_embd, n_ff);
    if (rc) return rc;
    if (n_tok == 0 || n_embd == 0) return ok();
    if ((rc = ensure_device())) return rc;
    ThreadCtx &c = t_ctx;
    const uint8_t *blob[3] = {gate, up, down};
    const size_t blen[3] = {gate_len, up_len, down_len};
    const uint32_t bdt[3] = {dtype_gate, dtype_up, dtype_down};
    const size_t bin[3] = {n_embd, n_embd, n_ff};
    const uint8_t *dev[3];
    Lease reg[3];
    for (int i = 0; i < 3; i++)
        if ((rc = blob_on_device(blob[i], blen[i], bdt[i], bin[i], c.moe_w[i], reg[i], &dev[i])))
            return rc;
    HIP_TRY(c.x.ensure(x_len * sizeof(float) + 16), "hipMalloc");
    HIP_TRY(c.y.ensure(out_len * sizeof(float)), "hipMalloc");
    HIP_TRY(hipMemcpyAsync(c.x.p, x, x_len * sizeof(float), hipMemcpyHostToDevice, c.stream),
            "upload x");
    ScratchLease sc = stream_scratch(c.stream);
    rc = shared_compute((float *)c.y.p, (const float *)c.x.p, dev[0], gate_len, dtype_gate, dev[1],
                        up_len, dtype_up, dev[2], down_len, dtype_down, n_tok, n_embd, n_ff, clamp,
                        c.stream, *sc);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(out, c.y.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c.stream),
            "download out");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return ok();
}

}  // extern "C"
