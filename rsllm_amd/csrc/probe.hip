// Measurement aid: a pure streaming read of device memory, the ceiling any
// HBM-bound kernel of this library is compared with (same bytes, no
// arithmetic). Not part of the reference's interface.
//
// k_stream_read<U>: n_wg workgroups of `threads` threads. In the contiguous
// mode workgroup b reads bytes [b * chunk, (b + 1) * chunk) (chunk = the
// buffer split evenly in 16-byte units), the order in which the GEMVs stream
// a row range; in the strided mode the whole grid walks the buffer with a
// grid-wide stride. Each lane issues U 16-byte buffer loads before it
// consumes any of them. The loaded words are folded into one xor per lane,
// written only when it equals a value the data would have to be built for,
// so the loads cannot be removed and nothing is stored in practice.
#include <hip/hip_runtime.h>

#include "../../include/rsllm_hip.h"
#include "abi_internal.h"
#include "kernels.h"

namespace rsllm_hip {

template <int U>
__global__ __launch_bounds__(1024) void k_stream_read(const uint8_t *__restrict__ p, uint32_t n16,
                                                      uint32_t *__restrict__ sink, int contiguous) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(p, n16 * 16u);
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    uint32_t beg, end, stride, i;
    if (contiguous) {
        const uint32_t per = (n16 + gridDim.x - 1) / gridDim.x;
        beg = blockIdx.x * per;
        end = min(beg + per, n16);
        stride = nt;
        i = beg + tid;
    } else {
        beg = 0;
        end = n16;
        stride = gridDim.x * nt;
        i = blockIdx.x * nt + tid;
    }
    uint32_t acc = 0;
    for (; i < end; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t j = i + (uint32_t)u * stride;
            // past `end`: an offset past the resource, which reads zeros
            v[u] = bload16(r, j < end ? j * 16u : 0xFFFFFFF0u, 0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x * nt + tid] = acc;
    (void)beg;
}

static hipError_t stream_read(const uint8_t *p, size_t bytes, uint32_t *sink, int n_wg, int threads,
                              int unroll, int contiguous, hipStream_t s) {
    const uint32_t n16 = (uint32_t)(bytes / 16);
    switch (unroll) {
#define U(N)                                                                                      \
    case N:                                                                                       \
        k_stream_read<N><<<(unsigned)n_wg, (unsigned)threads, 0, s>>>(p, n16, sink, contiguous); \
        break;
        U(1) U(2) U(4) U(8) U(16)
#undef U
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rsllm_hip

extern "C" int rsllm_hip_stream_read_dev(const uint8_t *p, size_t bytes, uint32_t *sink,
                                         size_t sink_len, int n_wg, int threads, int unroll,
                                         int contiguous, rsllm_hip_stream_t stream) {
    using namespace rsllm_hip;
    if (bytes % 16 != 0 || bytes > kMaxWeightBytes || ((uintptr_t)p & 15))
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                              "stream_read: bytes must be a multiple of 16 below 4 GiB and p "
                              "16-byte aligned");
    if (n_wg <= 0 || threads <= 0 || threads > 1024 || threads % 64 != 0)
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                              "stream_read: n_wg > 0 and threads a multiple of 64 up to 1024");
    if (!sink || sink_len < (size_t)n_wg * (size_t)threads || (bytes && !p))
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                              "stream_read: sink must hold n_wg * threads words");
    const hipError_t e =
        stream_read(p, bytes, sink, n_wg, threads, unroll, contiguous, (hipStream_t)stream);
    if (e == hipErrorInvalidValue)
        return abi::set_error(RSLLM_HIP_ERR_INVALID_ARGUMENT,
                              "stream_read: unroll must be 1, 2, 4, 8 or 16");
    if (e != hipSuccess) return abi::device_error(e, "stream_read");
    return abi::ok_status();
}
