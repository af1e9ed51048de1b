// Shared device definitions for the gfx950 (CDNA4, wave64) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dhx {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kHidden = 384;
constexpr int kHeads = 6;
constexpr int kHeadDim = 64;
constexpr int kPrefix = 5;
constexpr int kFF = 1536;
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// v_mfma_f32_32x32x16_f16. Operand a: lane l holds row (l % 32), k-slice
// 8*(l / 32) .. +7; operand b: lane l holds column (l % 32), the same
// k-slice. The 16 results of lane l are rows 8*(r/4) + 4*(l/32) + r%4,
// column l % 32. Any permutation of k inside the instruction applies to both
// operands alike, so only the row/column placement matters to callers.
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// silu(g) = g / (1 + e^-g), with e^-g evaluated as 2^(-g * log2 e) on v_exp_f32.
__device__ __forceinline__ float silu(float g) { return g * fast_rcp(1.0f + fast_exp2(-g * kLog2e)); }

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Remap the hardware id so that consecutive logical ids share an XCD:
// logical tiles [k*per, (k+1)*per) land on XCD k. Ids past the last full
// group of 8 keep their identity.
__device__ __forceinline__ int xcd_remap(int hw_id, int total) {
    const int full = total & ~7;
    if (hw_id >= full) return hw_id;
    const int per = full >> 3;
    return (hw_id & 7) * per + (hw_id >> 3);
}

}  // namespace dhx
