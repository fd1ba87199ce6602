/*
 * iris_dev.h - device-side helpers shared by the gfx950 kernels.
 *
 * Storage type for bf16 is uint16_t everywhere; MFMA operands are reinterpreted
 * as __bf16 vectors. Wave size is 64 (CDNA).
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define IRIS_WAVE 64

__device__ __forceinline__ float bf2f(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

/* round-to-nearest-even f32 -> bf16 (NaN stays NaN) */
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

/* Sum over each 16-lane row of the wave; every lane gets its row's total.
 * DPP moves (no LDS round trip) whose pairings give the same sums, bit for
 * bit, as the xor butterfly 1, 2, 4, 8: after the two quad steps a quad holds
 * one value, so mirroring within 8 and then within 16 lanes adds the same
 * partner values as xor 4 and xor 8. */
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));  /* quad_perm 1,0,3,2 */
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));  /* quad_perm 2,3,0,1 */
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)); /* row_half_mirror */
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)); /* row_mirror */
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* Sum over a block of `nwaves` waves; `red` is LDS scratch of >= nwaves floats.
 * Every thread returns the total. */
template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    int w = threadIdx.x / IRIS_WAVE, l = threadIdx.x % IRIS_WAVE;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NWAVES; i++) t += red[i];
    return t;
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

/* SiLU with the hardware reciprocal (~1 ulp) instead of an IEEE division;
 * for results rounded to bf16 next */
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

/* hardware round-to-nearest-even f32 -> bf16 (v_cvt_pk_bf16_f32; NaN stays NaN) */
__device__ __forceinline__ uint16_t f2bf_hw(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

/* Streaming (nontemporal) 16- and 8-byte accesses for data a kernel touches
 * once and that nothing reads again soon (row inputs of the normalisations,
 * split-K partials): they keep the caches for the operands that are reused.
 * A 1 GiB device copy runs at 6.0 TB/s with them against 5.5 TB/s with plain
 * accesses. */
__device__ __forceinline__ float4 ld_stream(const float4 *p) {
    const f32x4 v = __builtin_nontemporal_load((const f32x4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(float4 *p, float4 v) {
    __builtin_nontemporal_store((f32x4){v.x, v.y, v.z, v.w}, (f32x4 *)p);
}
__device__ __forceinline__ void st_stream(u16x4 *p, u16x4 v) { __builtin_nontemporal_store(v, p); }
