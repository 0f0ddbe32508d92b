// Shared device/host helpers of the MI355X engine (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

// ---- library-wide launch stream and error buffer (support.hip) ----------
extern "C" char *hd_cuda_errbuf(void);
hipStream_t hd_stream(void);
// Records a launch failure (if any) of the previous kernel under `what`.
void hd_check_launch(const char *what);

// ---- bf16 <-> fp32 ------------------------------------------------------
// bf16 payloads are uint16_t. fp32 -> bf16 uses gfx950's v_cvt_pk_bf16_f32,
// IEEE round-to-nearest-even: for finite values the same bits as the
// reference's integer rule (support.cu:21-28); NaN payloads are not produced
// on this path.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf2f(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}
// Two floats -> packed bf16x2 (low half = a), one instruction.
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
    bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float bfround(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// ---- MFMA operand types -------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define HD_LDS __attribute__((address_space(3)))

static inline unsigned hd_cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }
