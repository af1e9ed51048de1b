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

// x += ls * (sum_s partials[s] + b), four channels per thread.
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(ReduceArgs p) {
    const size_t total = (size_t)p.rows * kHidden;
    const size_t i = ((size_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i >= total) return;
    const int n = (int)(i % kHidden);
    float4_t acc = *(const float4_t*)(p.partials + i);
    for (int s = 1; s < p.splits; ++s) acc += *(const float4_t*)(p.partials + (size_t)s * total + i);
    acc = (acc + *(const float4_t*)(p.bias + n)) * *(const float4_t*)(p.ls + n);
    half4_t x = *(const half4_t*)(p.x + i);
    half4_t y = {(half_t)((float)x[0] + acc[0]), (half_t)((float)x[1] + acc[1]),
                 (half_t)((float)x[2] + acc[2]), (half_t)((float)x[3] + acc[3])};
    *(half4_t*)(p.x + i) = y;
}

}  // namespace

hipError_t launch_layernorm(const LayerNormArgs& a, hipStream_t s) {
    const int blocks = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(layernorm_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s) {
    const size_t quads = (size_t)a.rows * kHidden / 4;
    const int blocks = (int)((quads + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dhx
