// Device-side helpers shared by the gfx950 kernels: wave64 reductions and
// scans, bf16 conversion, error plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/cbq_hip.h"

#define CBQ_WAVE 64

// Launch-error check shared by every C entry point.
static inline int cbq_launch_status(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "[cbq_hip] %s: %s\n", what, hipGetErrorString(e));
        return CK_ERR_HIP;
    }
    return CK_SUCCESS;
}

// Number of compute units of the current device (cached per device id).
int cbq_num_cus();

__device__ __forceinline__ float bf16_to_f32(uint16_t h)
{
    return __uint_as_float((uint32_t)h << 16);
}

// Round-to-nearest-even float -> bf16 bit pattern; NaN stays quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <typename XT> __device__ __forceinline__ float to_f32(XT v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename OT> __device__ __forceinline__ OT from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

// Butterfly sum over aligned groups of `width` lanes (power of two <= 64);
// every lane of a group ends with the group total.
__device__ __forceinline__ float group_sum(float v, int width)
{
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, CBQ_WAVE);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum(v, CBQ_WAVE); }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    for (int o = 1; o < CBQ_WAVE; o <<= 1) {
        uint32_t u = __shfl_up(v, o, CBQ_WAVE);
        if (lane >= o) v += u;
    }
    return v;
}

// Workgroup barrier for LDS hand-off only: waits for this wave's LDS
// operations, then s_barrier.  Unlike __syncthreads() it does not wait for
// outstanding global loads, so prefetched weight data stays in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// b-bit field starting at bit `s` of the little-endian pair (hi:lo).
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s)
{
    return __builtin_amdgcn_alignbit(hi, lo, s);
}
