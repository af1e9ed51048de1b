// Row LayerNorm (replaces kernels/layernorm_rowwave_f16.loom and
// layernorm_rowwave_f32out.loom) and the split-K slab reduce (replaces
// kernels/splitk_reduce_f16.loom). Both are HBM-bound streaming kernels.
#include "launch.hpp"

namespace dhx {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

// One wave per 384-channel row: lanes 0..47 each load one 16-byte piece
// (the whole 768-byte row in one coalesced load), lanes 48..63 hold zeros.
// Mean and variance are two passes over registers in fp32 (the reference
// uses E[x^2] - E[x]^2, layernorm_rowwave_f16.loom:86-93); eps 1e-5.
__global__ __launch_bounds__(kThreads) void layernorm_kernel(LayerNormArgs p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // the whole wave leaves together
    const bool active = lane < kHidden / 8;
    float v[8];
    if (active) {
        const half8_t h = *(const half8_t*)(p.x + (size_t)row * kHidden + lane * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[e];
    const float mean = wave_sum(s) * (1.0f / kHidden);
    float d = 0.f;
    if (active) {
#pragma unroll
        for (int e = 0; e < 8; ++e) d += (v[e] - mean) * (v[e] - mean);
    }
    const float rstd = rsqrtf(wave_sum(d) * (1.0f / kHidden) + 1e-5f);
    if (!active) return;
    const int c = lane * 8;
    const float4_t g0 = *(const float4_t*)(p.gamma + c), g1 = *(const float4_t*)(p.gamma + c + 4);
    const float4_t b0 = *(const float4_t*)(p.beta + c), b1 = *(const float4_t*)(p.beta + c + 4);
    float y[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        y[e] = (v[e] - mean) * rstd * g0[e] + b0[e];
        y[e + 4] = (v[e + 4] - mean) * rstd * g1[e] + b1[e];
    }
    if (p.f32_out) {
        float* o = (float*)p.out + (size_t)row * kHidden + c;
        *(float4_t*)o = float4_t{y[0], y[1], y[2], y[3]};
        *(float4_t*)(o + 4) = float4_t{y[4], y[5], y[6], y[7]};
    } else {
        half8_t h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (half_t)y[e];
        *(half8_t*)((half_t*)p.out + (size_t)row * kHidden + c) = h;
    }
}

// x += ls * (sum_s partials[s] + b): one wave per row, lanes 0..47 own 8
// channels each (8 lanes per 64-column statistics slot). With STATS, the
// slot partials (mean, M2) of the updated f16 row are written as well.
template <bool STATS>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(ReduceArgs p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // the whole wave leaves together
    const bool active = lane < kHidden / 8;
    const size_t total = (size_t)p.rows * kHidden;
    const int c = (active ? lane : 0) * 8;
    const size_t i = (size_t)row * kHidden + c;
    float y[8];
    float4_t a0 = *(const float4_t*)(p.partials + i), a1 = *(const float4_t*)(p.partials + i + 4);
    for (int s = 1; s < p.splits; ++s) {
        a0 += *(const float4_t*)(p.partials + (size_t)s * total + i);
        a1 += *(const float4_t*)(p.partials + (size_t)s * total + i + 4);
    }
    a0 = (a0 + *(const float4_t*)(p.bias + c)) * *(const float4_t*)(p.ls + c);
    a1 = (a1 + *(const float4_t*)(p.bias + c + 4)) * *(const float4_t*)(p.ls + c + 4);
    const half8_t x = *(const half8_t*)(p.x + i);
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = (half_t)((float)x[e] + (e < 4 ? a0[e] : a1[e - 4]));
        y[e] = (float)h[e];
    }
    if (active) *(half8_t*)(p.x + i) = h;
    if constexpr (STATS) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += y[e];
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) s += __shfl_xor(s, o, kWave);
        const float mean = s * (1.0f / 64.0f);
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) q += (y[e] - mean) * (y[e] - mean);
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) q += __shfl_xor(q, o, kWave);
        if (active && (lane & 7) == 0)
            *(float2_t*)(p.stats + (size_t)row * kStatFloats + (lane >> 3) * 2) = float2_t{mean, q};
    }
}

}  // namespace

hipError_t launch_layernorm(const LayerNormArgs& a, hipStream_t s) {
    const int blocks = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(layernorm_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s) {
    const int blocks = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (a.stats) hipLaunchKernelGGL(splitk_reduce_kernel<true>, dim3(blocks), dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(splitk_reduce_kernel<false>, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dhx
