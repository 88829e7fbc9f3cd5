// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rsllm_hip {

// GgmlType ids (rsllm-gguf/src/tensor.rs:26-85).
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q2_K = 10,
    T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15, T_IQ2_XXS = 16, T_BF16 = 30
};

constexpr int kQ4kBytes = 144;
constexpr int kQ6kBytes = 210;
constexpr int kQ8Bytes = 34;

// Exact f16 -> f32 widening of a 16-bit pattern (v_cvt_f32_f16 keeps f16
// subnormals: the f16 denormal mode is "preserve" on gfx9).
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Raw buffer loads: offsets are bytes from the base, and an access past
// num_records (checked per access) returns zeros instead of faulting.
typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
    return make_uint2((uint32_t)v.x, (uint32_t)v.y);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    // word 3 = 0x00020000: the raw-buffer configuration of the gfx9 family
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}

// Packed f16 vectors of the MFMA paths.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight 4-bit codes (the low nibbles of two dwords, or the high nibbles when
// `hi`) -> 8 f16 values q * dsc - dm. v_cvt_scalef32_pk_f16_fp8 reads each
// byte 0..15 as an e4m3 value q * 2^-9 (exact) and applies a power-of-two
// scale, so a scale of 2^9 yields the integer q in f16 exactly, two per
// instruction; one packed FMA then applies the block scales (one rounding).
__device__ __forceinline__ f16x8 dequant_q4x8_f16(uint32_t d0, uint32_t d1, bool hi, f16x2 dsc,
                                                  f16x2 dm) {
    if (hi) {
        d0 >>= 4;
        d1 >>= 4;
    }
    d0 &= 0x0F0F0F0Fu;
    d1 &= 0x0F0F0F0Fu;
    const f16x2 q0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 512.0f, false);  // bytes 0, 1
    const f16x2 q1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 512.0f, true);   // bytes 2, 3
    const f16x2 q2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 512.0f, false);
    const f16x2 q3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 512.0f, true);
    const f16x2 w0 = q0 * dsc - dm, w1 = q1 * dsc - dm, w2 = q2 * dsc - dm, w3 = q3 * dsc - dm;
    f16x8 r;
    r[0] = w0[0]; r[1] = w0[1]; r[2] = w1[0]; r[3] = w1[1];
    r[4] = w2[0]; r[5] = w2[1]; r[6] = w3[0]; r[7] = w3[1];
    return r;
}

// Sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Byte b (0..3) of a dword as float: one v_cvt_f32_ubyte{b}.
__device__ __forceinline__ float ubyte_f(uint32_t v, int b) {
    return (float)((v >> (8 * b)) & 0xFFu);
}

// Dword i (0..3) of a uint4 without indexing a local array (a runtime index
// into an array would be placed in scratch memory).
__device__ __forceinline__ uint32_t sel4(const uint4 &v, int i) {
    const uint32_t a = (i & 1) ? v.y : v.x;
    const uint32_t b = (i & 1) ? v.w : v.z;
    return (i & 2) ? b : a;
}

// Signed byte i (0..15) of a uint4.
__device__ __forceinline__ int sbyte16(const uint4 &v, int i) {
    return (int)(int8_t)(sel4(v, i >> 2) >> (8 * (i & 3)));
}

// (sc, m) of Q4_K sub-block j from the three scale dwords s0 = bytes 0-3,
// s1 = bytes 4-7, s2 = bytes 8-11 (q4_k_scale_min, dequant/mod.rs:48-58).
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int q = 8 * (j - 4);
        sc = ((s2 >> q) & 15u) | (((s0 >> (q + 6)) & 3u) << 4);
        m = ((s2 >> (q + 4)) & 15u) | (((s1 >> (q + 6)) & 3u) << 4);
    }
}

}  // namespace rsllm_hip
