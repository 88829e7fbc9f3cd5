// Whole-model weight residency: every tensor of a GGUF checkpoint uploaded
// once into one device arena, in this backend's device layout.
//
// The reference borrows tensor payloads from the GGUF mmap for the life of
// the GgufFile (rsllm-gguf/src/file.rs:81-97 open, :181-187 tensor_bytes;
// rsllm-models/src/dsv4/loader.rs:199-216 resolve_blob) and runs every matmul
// on those host bytes. Here the caller hands over the same (name, bytes,
// dtype, row length) list once:
//   - one hipMalloc arena holds all tensors in list order, each 256-byte
//     aligned, so a stacked expert tensor stays one contiguous range;
//   - bytes travel through two pinned staging buffers: host threads copy
//     chunk k + 1 out of the mapping while chunk k is in flight to the
//     device, and formats with a converted layout go through a device
//     staging buffer and launch_prepare_blocks into the arena (chunks start
//     on 8-block super-tile boundaries, so the result is byte-identical to
//     converting the whole tensor);
//   - every matmul-format tensor is added to the registry under its host
//     range, so the host-pointer entry points use the resident copy;
//   - a model is keyed by the GGUF fingerprint (file.rs:175-177, which
//     hashes names, types and shapes only), the tensor table and a hash of
//     every payload byte, taken by the copy threads as they stage the bytes.
//     An upload whose fingerprint, table and sampled-window digest match a
//     live model hashes its whole payload (a read pass, no device work) and
//     reuses that model (reference count, new host ranges registered) only
//     when the full hashes agree.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/rsllm_hip.h"
#include "abi_internal.h"
#include "kernels.h"

using namespace rsllm_hip;

namespace {

constexpr size_t kStage = 64u << 20;  // bytes per staging buffer
constexpr size_t kAlign = 256;
constexpr int kCopyThreads = 8;

struct Tensor {
    std::string name;
    uint32_t dtype;
    size_t len, in_dim, off;
    bool matmul;  // registered for the matmul entry points
};

struct Model {
    uint64_t id;
    uint8_t fp[32];
    uint64_t digest;  // table + sampled windows: the cheap pre-filter
    uint64_t full;    // table + every payload byte
    int device;
    std::vector<Tensor> t;
    // the arena; registry entries of the model share it, so it is freed when
    // the model is released and no call in flight still reads it
    std::shared_ptr<abi::DevMem> mem;
    uint8_t *arena = nullptr;
    size_t arena_bytes = 0;
    uint32_t refs = 0;
    uint64_t uploaded = 0;
    double seconds = 0;
};

std::mutex m_mu;  // guards g_models and g_next (uploads are serialised by it)
std::vector<std::unique_ptr<Model>> g_models;
uint64_t g_next = 1;

int dev_err(hipError_t e, const char *where) { return abi::device_error(e, where); }

#define HIP_TRY(expr, where)                                 \
    do {                                                     \
        hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) return dev_err(e_, where);     \
    } while (0)

bool is_matmul_dtype(uint32_t t) {
    return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0 || t == T_Q4_0 || t == T_Q2_K ||
           t == T_IQ2_XXS || t == T_F32;
}

// FNV-1a, 64-bit.
struct Fnv {
    uint64_t h = 1469598103934665603ull;
    void add(const void *p, size_t n) {
        const uint8_t *b = static_cast<const uint8_t *>(p);
        for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
    }
    template <class T> void put(T v) { add(&v, sizeof v); }
};

// The tensor table plus 16 windows of 256 bytes spread over each payload
// (the whole payload when it is at most 4 KiB).
uint64_t model_digest(const rsllm_hip_tensor_desc *d, size_t n) {
    Fnv f;
    f.put((uint64_t)n);
    for (size_t i = 0; i < n; i++) {
        f.add(d[i].name, strlen(d[i].name) + 1);
        f.put(d[i].dtype);
        f.put((uint64_t)d[i].len);
        f.put((uint64_t)d[i].in_dim);
        const size_t L = d[i].len;
        if (L <= 4096) {
            f.add(d[i].data, L);
        } else {
            for (int w = 0; w < 16; w++) f.add(d[i].data + (L - 256) / 15 * w, 256);
        }
    }
    return f.h;
}

// Checks of one tensor. Matmul formats need whole rows of a block-aligned
// row length, as their matmul entry points do.
int validate_tensor(const rsllm_hip_tensor_desc &d) {
    if (!d.name) return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_upload: NULL name");
    if (d.len && !d.data) {
        const std::string m = std::string("model_upload: ") + d.name + ": NULL data";
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, m.c_str());
    }
    if (is_matmul_dtype(d.dtype) && d.in_dim) {
        const size_t be = block_elems_of(d.dtype);
        const size_t rb = row_bytes_of(d.dtype, d.in_dim);
        if (d.in_dim % be != 0 || rb == 0 || d.len % rb != 0) {
            const std::string m = std::string("model_upload: ") + d.name +
                                  ": length is not a whole number of rows of in_dim";
            return abi::set_error(RSLLM_HIP_ERR_SHAPE_MISMATCH, m.c_str());
        }
    }
    return RSLLM_HIP_OK;
}

// Payload hash: 64-bit words folded into four independent lanes (multiply,
// rotate, multiply by odd constants), the lanes and the length mixed at the
// end; the tail bytes go through FNV-1a. Not cryptographic: it tells apart
// payloads that differ anywhere, which the sampled digest cannot.
constexpr size_t kHashBlock = 1u << 20;  // bytes per block hash
inline uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
uint64_t hash_bytes(const uint8_t *p, size_t n) {
    constexpr uint64_t K1 = 0x9E3779B97F4A7C15ull, K2 = 0xC2B2AE3D27D4EB4Full;
    uint64_t a[4] = {K1, K2, K1 ^ K2, ~K1};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int l = 0; l < 4; l++) {
            uint64_t w;
            memcpy(&w, p + i + 8 * l, 8);
            a[l] = rotl64(a[l] + w * K2, 31) * K1;
        }
    Fnv f;
    f.put((uint64_t)n);
    for (int l = 0; l < 4; l++) f.put(a[l]);
    f.add(p + i, n - i);
    return f.h;
}

// hash_bytes of [src, src + n) while copying it to dst, in one pass over
// the source.
uint64_t copy_hash_bytes(uint8_t *dst, const uint8_t *src, size_t n) {
    constexpr uint64_t K1 = 0x9E3779B97F4A7C15ull, K2 = 0xC2B2AE3D27D4EB4Full;
    uint64_t a[4] = {K1, K2, K1 ^ K2, ~K1};
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        uint64_t w[4];
        memcpy(w, src + i, 32);
        memcpy(dst + i, w, 32);
        for (int l = 0; l < 4; l++) a[l] = rotl64(a[l] + w[l] * K2, 31) * K1;
    }
    memcpy(dst + i, src + i, n - i);
    Fnv f;
    f.put((uint64_t)n);
    for (int l = 0; l < 4; l++) f.put(a[l]);
    f.add(src + i, n - i);
    return f.h;
}

// Hashes of the kHashBlock blocks of [p, p + n) into h[0..] (copying them
// to dst when dst is not NULL).
void hash_blocks(uint8_t *dst, const uint8_t *p, size_t n, uint64_t *h) {
    const size_t nblk = (n + kHashBlock - 1) / kHashBlock;
    for (size_t k = 0; k < nblk; k++) {
        const size_t o = k * kHashBlock, m = std::min(kHashBlock, n - o);
        h[k] = dst ? copy_hash_bytes(dst + o, p + o, m) : hash_bytes(p + o, m);
    }
}

// Block hashes of [src, src + n) into h, in parallel (the source is usually
// a file mapping being paged in), copying the bytes to dst on the way when
// dst is not NULL (the upload's staging copy). Threads take whole
// kHashBlock blocks; pieces no thread could be started for are handled by
// the caller.
void copy_parallel(uint8_t *dst, const uint8_t *src, size_t n, uint64_t *h) {
    if (n < (8u << 20)) {
        hash_blocks(dst, src, n, h);
        return;
    }
    const size_t nblk = (n + kHashBlock - 1) / kHashBlock;
    const size_t per = (nblk + kCopyThreads - 1) / kCopyThreads * kHashBlock;
    std::vector<std::thread> th;
    for (size_t o = 0; o < n; o += per) {
        const size_t m = std::min(per, n - o);
        auto work = [=] { hash_blocks(dst ? dst + o : nullptr, src + o, m, h + o / kHashBlock); };
        try {
            th.emplace_back(work);
        } catch (...) {
            work();
        }
    }
    for (auto &t : th) t.join();
}

// Bytes per staging chunk of a tensor: converted formats move whole 8-block
// super-tiles.
size_t chunk_bytes(uint32_t dtype, size_t in_dim) {
    const bool conv = layout_converted(dtype) && in_dim;
    const size_t unit = conv ? 8 * block_bytes_of(dtype) : 1;
    return kStage / unit * unit;
}

// Folds the tensor table, then every chunk's block hashes in upload order.
struct FullHash {
    Fnv f;
    explicit FullHash(const rsllm_hip_tensor_desc *d, size_t n) {
        f.put((uint64_t)n);
        for (size_t i = 0; i < n; i++) {
            f.add(d[i].name, strlen(d[i].name) + 1);
            f.put(d[i].dtype);
            f.put((uint64_t)d[i].len);
            f.put((uint64_t)d[i].in_dim);
        }
    }
    void add_chunk(const uint64_t *h, size_t nb) {
        for (size_t k = 0; k < (nb + kHashBlock - 1) / kHashBlock; k++) f.put(h[k]);
    }
};

// The full hash of a payload list, by a read pass (no device work).
uint64_t payload_hash(const rsllm_hip_tensor_desc *d, size_t n) {
    FullHash fh(d, n);
    std::vector<uint64_t> h(kStage / kHashBlock + 1);
    for (size_t i = 0; i < n; i++) {
        const size_t chunk = chunk_bytes(d[i].dtype, d[i].in_dim);
        for (size_t o = 0; o < d[i].len; o += chunk) {
            const size_t nb = std::min(chunk, d[i].len - o);
            copy_parallel(nullptr, d[i].data + o, nb, h.data());
            fh.add_chunk(h.data(), nb);
        }
    }
    return fh.f.h;
}

struct Staging {
    uint8_t *host[2] = {nullptr, nullptr};
    uint8_t *dev[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t s = nullptr;
    ~Staging() {
        // work still queued (an upload that failed part way) ends first
        if (s) (void)hipStreamSynchronize(s);
        for (int b = 0; b < 2; b++) {
            if (done[b]) (void)hipEventDestroy(done[b]);
            if (host[b]) (void)hipHostFree(host[b]);
            if (dev[b]) (void)hipFree(dev[b]);
        }
        if (s) (void)hipStreamDestroy(s);
    }
};

// Upload every tensor of `m` (offsets set) from the descriptors.
int upload(Model &m, const rsllm_hip_tensor_desc *d, size_t n) {
    Staging st;
    HIP_TRY(hipStreamCreateWithFlags(&st.s, hipStreamNonBlocking), "hipStreamCreate");
    bool any_conv = false;
    for (size_t i = 0; i < n; i++) any_conv |= layout_converted(d[i].dtype) && d[i].in_dim;
    for (int b = 0; b < 2; b++) {
        HIP_TRY(hipHostMalloc((void **)&st.host[b], kStage, hipHostMallocDefault), "hipHostMalloc");
        HIP_TRY(hipEventCreateWithFlags(&st.done[b], hipEventDisableTiming), "hipEventCreate");
        if (any_conv) HIP_TRY(hipMalloc((void **)&st.dev[b], kStage), "hipMalloc");
    }
    FullHash fh(d, n);
    std::vector<uint64_t> h(kStage / kHashBlock + 1);
    int k = 0;  // chunk counter (staging buffer k & 1)
    for (size_t i = 0; i < n; i++) {
        const Tensor &t = m.t[i];
        const bool conv = layout_converted(t.dtype) && t.in_dim;
        const size_t chunk = chunk_bytes(t.dtype, t.in_dim);
        for (size_t o = 0; o < t.len; o += chunk, k++) {
            const size_t nb = std::min(chunk, t.len - o);
            const int b = k & 1;
            if (k >= 2) HIP_TRY(hipEventSynchronize(st.done[b]), "hipEventSynchronize");
            copy_parallel(st.host[b], d[i].data + o, nb, h.data());
            fh.add_chunk(h.data(), nb);
            uint8_t *dst = m.arena + t.off + o;
            if (conv) {
                HIP_TRY(hipMemcpyAsync(st.dev[b], st.host[b], nb, hipMemcpyHostToDevice, st.s),
                        "upload");
                HIP_TRY(launch_prepare_blocks(t.dtype, st.dev[b], dst,
                                              nb / block_bytes_of(t.dtype), st.s),
                        "prepare");
            } else {
                HIP_TRY(hipMemcpyAsync(dst, st.host[b], nb, hipMemcpyHostToDevice, st.s),
                        "upload");
            }
            HIP_TRY(hipEventRecord(st.done[b], st.s), "hipEventRecord");
            m.uploaded += nb;
        }
    }
    HIP_TRY(hipStreamSynchronize(st.s), "hipStreamSynchronize");
    m.full = fh.f.h;
    return RSLLM_HIP_OK;
}

void register_host_ranges(const Model &m, const rsllm_hip_tensor_desc *d) {
    for (size_t i = 0; i < m.t.size(); i++)
        if (m.t[i].matmul)
            abi::registry_add(d[i].data, d[i].len, d[i].dtype, d[i].in_dim, m.arena + m.t[i].off,
                              m.id, m.mem);
}

Model *find_model(uint64_t id) {
    for (auto &p : g_models)
        if (p->id == id) return p.get();
    return nullptr;
}

}  // namespace

extern "C" {

int rsllm_hip_model_upload(const uint8_t *fingerprint, const rsllm_hip_tensor_desc *tensors,
                           size_t n_tensors, uint64_t *model) {
    if (!fingerprint || !model || (n_tensors && !tensors))
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_upload: NULL argument");
    for (size_t i = 0; i < n_tensors; i++) {
        const int rc = validate_tensor(tensors[i]);
        if (rc) return rc;
        for (size_t j = 0; j < i; j++)
            if (!strcmp(tensors[i].name, tensors[j].name)) {
                const std::string m =
                    std::string("model_upload: duplicate tensor name ") + tensors[i].name;
                return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, m.c_str());
            }
    }
    int rc = abi::ensure_current_device();
    if (rc) return rc;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    const uint64_t digest = model_digest(tensors, n_tensors);
    std::lock_guard<std::mutex> lk(m_mu);
    // a candidate passes the sampled digest; reuse needs the full hash too
    // (taken once, over the new payload, for all candidates)
    bool have_full = false;
    uint64_t full = 0;
    for (auto &p : g_models) {
        if (p->device == dev && p->digest == digest && !memcmp(p->fp, fingerprint, 32) &&
            p->t.size() == n_tensors) {
            if (!have_full) {
                full = payload_hash(tensors, n_tensors);
                have_full = true;
            }
            if (p->full != full) continue;
            p->refs++;
            register_host_ranges(*p, tensors);
            *model = p->id;
            return abi::ok_status();
        }
    }
    auto m = std::make_unique<Model>();
    m->id = g_next++;
    memcpy(m->fp, fingerprint, 32);
    m->digest = digest;
    m->device = dev;
    size_t off = 0;
    for (size_t i = 0; i < n_tensors; i++) {
        const rsllm_hip_tensor_desc &d = tensors[i];
        m->t.push_back({d.name, d.dtype, d.len, d.in_dim, off,
                        is_matmul_dtype(d.dtype) && d.in_dim != 0 && d.len != 0});
        off += (d.len + kAlign - 1) / kAlign * kAlign;
    }
    m->arena_bytes = off;
    const auto t0 = std::chrono::steady_clock::now();
    m->mem = std::make_shared<abi::DevMem>();
    m->mem->device = dev;
    if (off) HIP_TRY(abi::dev_malloc((void **)&m->mem->p, off), "hipMalloc arena");
    m->arena = m->mem->p;
    rc = upload(*m, tensors, n_tensors);
    if (rc) return rc;  // m (and its arena) is dropped
    m->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    m->refs = 1;
    register_host_ranges(*m, tensors);
    *model = m->id;
    g_models.push_back(std::move(m));
    return abi::ok_status();
}

int rsllm_hip_model_tensor(uint64_t model, const char *name, const uint8_t **dev, size_t *len) {
    if (!name || !dev || !len)
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_tensor: NULL argument");
    std::lock_guard<std::mutex> lk(m_mu);
    const Model *m = find_model(model);
    if (!m) return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_tensor: unknown model");
    for (const Tensor &t : m->t)
        if (t.name == name) {
            *dev = m->arena + t.off;
            *len = t.len;
            return abi::ok_status();
        }
    const std::string msg = std::string("model_tensor: no tensor named ") + name;
    return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, msg.c_str());
}

int rsllm_hip_model_info_get(uint64_t model, rsllm_hip_model_info *out) {
    if (!out) return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_info: NULL argument");
    std::lock_guard<std::mutex> lk(m_mu);
    const Model *m = find_model(model);
    if (!m) return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_info: unknown model");
    out->device_bytes = m->arena_bytes;
    out->uploaded_bytes = m->uploaded;
    out->upload_seconds = m->seconds;
    out->refs = m->refs;
    out->n_tensors = (uint32_t)m->t.size();
    return abi::ok_status();
}

int rsllm_hip_model_release(uint64_t model) {
    std::unique_ptr<Model> gone;
    {
        std::lock_guard<std::mutex> lk(m_mu);
        for (size_t i = 0; i < g_models.size(); i++) {
            if (g_models[i]->id != model) continue;
            if (--g_models[i]->refs == 0) {
                gone = std::move(g_models[i]);
                g_models.erase(g_models.begin() + (long)i);
            }
            break;
        }
        if (!gone && !find_model(model))
            return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT, "model_release: unknown model");
    }
    if (gone) {
        // the registry's references go first; the arena is freed when the
        // model's own reference below and every call in flight that found
        // one of its tensors have let go (hipFree waits for the device)
        abi::registry_drop_owner(gone->id);
        gone.reset();
    }
    return abi::ok_status();
}

}  // extern "C"
