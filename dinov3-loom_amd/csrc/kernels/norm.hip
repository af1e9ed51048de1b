// Row LayerNorm (replaces kernels/layernorm_rowwave_f16.loom and
// layernorm_rowwave_f32out.loom) and the split-K slab reduce (replaces
// kernels/splitk_reduce_f16.loom). Both are HBM-bound streaming kernels.
#include "launch.hpp"

namespace dhx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kKs = kHidden / 16;       // 16-column blocks per row
constexpr int kLnKs = kKs / kWaves;     // blocks per wave in the LayerNorm

// One workgroup per 32-row block of x (fragment order); wave w holds the
// 16-column blocks 6w .. 6w+5 of the 32 rows, loaded as whole fragments (1 KB
// contiguous per wave access) and kept as f16: lane (l, hi) holds row l's
// half hi of each. The row statistics are two passes over them in fp32, each
// combined with the partner lane l ^ 32 and then across the four waves
// through LDS (the reference uses E[x^2] - E[x]^2,
// layernorm_rowwave_f16.loom:86-93); eps 1e-5. The f16 output (h) is written
// in fragment order; the f32 output (the final tokens, row-major) goes
// through LDS so that each wave writes 384-byte row runs.
constexpr int kOutPitch = kLnKs * 16 + 4;  // floats per staged row of a wave

__global__ __launch_bounds__(kThreads) void layernorm_kernel(LayerNormArgs p) {
    __shared__ float part[2][kWaves][32];
    __shared__ __attribute__((aligned(16))) float stage[kWaves][32 * kOutPitch];
    const int lane = threadIdx.x & 63, l32 = lane & 31, hi = lane >> 5, w = threadIdx.x >> 6;
    const int mb = blockIdx.x, row = mb * 32 + l32, ks0 = w * kLnKs;
    const half_t* xb = p.x + ((size_t)mb * kKs + ks0) * 512 + lane * 8;
    half8_t v[kLnKs];
#pragma unroll
    for (int ks = 0; ks < kLnKs; ++ks) v[ks] = *(const half8_t*)(xb + ks * 512);
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < kLnKs; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += (float)v[ks][e];
    s = half_pair_sum(s);
    if (hi == 0) part[0][w][l32] = s;
    __syncthreads();
    // correctly rounded: a constant row's mean is exact
    const float mean = ((part[0][0][l32] + part[0][1][l32]) + (part[0][2][l32] + part[0][3][l32])) / kHidden;
    float d = 0.f;
#pragma unroll
    for (int ks = 0; ks < kLnKs; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) d += ((float)v[ks][e] - mean) * ((float)v[ks][e] - mean);
    d = half_pair_sum(d);
    if (hi == 0) part[1][w][l32] = d;
    __syncthreads();
    d = (part[1][0][l32] + part[1][1][l32]) + (part[1][2][l32] + part[1][3][l32]);
    const float rstd = rsqrtf(d / kHidden + 1e-5f);
    float* const st = stage[w];
#pragma unroll
    for (int i = 0; i < kLnKs; ++i) {
        const int ks = ks0 + i, c = ks * 16 + hi * 8;
        const float4_t g0 = *(const float4_t*)(p.gamma + c), g1 = *(const float4_t*)(p.gamma + c + 4);
        const float4_t b0 = *(const float4_t*)(p.beta + c), b1 = *(const float4_t*)(p.beta + c + 4);
        float y[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            y[e] = ((float)v[i][e] - mean) * rstd * g0[e] + b0[e];
            y[e + 4] = ((float)v[i][e + 4] - mean) * rstd * g1[e] + b1[e];
        }
        if (p.f32_out) {
            float* const o = st + l32 * kOutPitch + i * 16 + hi * 8;
            *(float4_t*)o = float4_t{y[0], y[1], y[2], y[3]};
            *(float4_t*)(o + 4) = float4_t{y[4], y[5], y[6], y[7]};
        } else if (row < p.rows) {
            half8_t h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (half_t)y[e];
            const WtOut out((half_t*)p.out + (size_t)mb * kKs * 512, kKs * 1024);
            out.store((ks * 512 + lane * 8) * 2, h);
        }
    }
    if (!p.f32_out) return;
    wave_lds_sync();
    // The wave's 32 rows x 96 columns: 24 float4 per row, 12 per lane.
    constexpr int Q = kLnKs * 4;  // float4 per row
    const WtOut out((float*)p.out + (size_t)mb * 32 * kHidden, 32 * kHidden * 4);
#pragma unroll
    for (int it = 0; it < 32 * Q / 64; ++it) {
        const int idx = it * 64 + lane, r = idx / Q, q = idx % Q, m = mb * 32 + r;
        if (m < p.rows) out.store((r * kHidden + ks0 * 16 + q * 4) * 4, *(const float4_t*)(st + r * kOutPitch + q * 4));
    }
}

// x += ls * (sum_s partials[s] + b) on x in fragment order: one wave per
// (32-row block, 64-column slot), lane (l, hi) owning row l's half hi of each
// of the slot's four 16-column blocks; the f32 slabs are row-major. With
// STATS, the slot partials (mean, M2) of the updated f16 rows are written as
// well (combined with the partner lane l ^ 32).
template <bool STATS>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(ReduceArgs p) {
    const int lane = threadIdx.x & 63, l32 = lane & 31, hi = lane >> 5;
    const int wid = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int mb = wid / kStatSlots, slot = wid % kStatSlots;
    if (mb * 32 >= p.rows) return;  // the whole wave leaves together
    const int row = mb * 32 + l32;
    const bool valid = row < p.rows;
    const int rr = valid ? row : p.rows - 1;  // padding rows read a real row, write nothing
    const size_t total = (size_t)p.rows * kHidden;
    float y[32];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int ks = slot * 4 + kk, c = ks * 16 + hi * 8;
        const size_t i = (size_t)rr * kHidden + c;
        float4_t a0 = *(const float4_t*)(p.partials + i), a1 = *(const float4_t*)(p.partials + i + 4);
        for (int sp = 1; sp < p.splits; ++sp) {
            a0 += *(const float4_t*)(p.partials + (size_t)sp * total + i);
            a1 += *(const float4_t*)(p.partials + (size_t)sp * total + i + 4);
        }
        a0 = (a0 + *(const float4_t*)(p.bias + c)) * *(const float4_t*)(p.ls + c);
        a1 = (a1 + *(const float4_t*)(p.bias + c + 4)) * *(const float4_t*)(p.ls + c + 4);
        half_t* const xp = p.x + ((size_t)mb * kKs + ks) * 512 + lane * 8;
        const half8_t x = *(const half8_t*)xp;
        half8_t h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[e] = (half_t)((float)x[e] + (e < 4 ? a0[e] : a1[e - 4]));
            y[kk * 8 + e] = (float)h[e];
        }
        if (valid) *(half8_t*)xp = h;
    }
    if constexpr (STATS) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) s += y[e];
        s = half_pair_sum(s);
        const float mean = s * (1.0f / 64.0f);
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) q += (y[e] - mean) * (y[e] - mean);
        q = half_pair_sum(q);
        if (valid && hi == 0) *(float2_t*)(p.stats + (size_t)row * kStatFloats + slot * 2) = float2_t{mean, q};
    }
}

// One thread per 16-byte piece of a padding row (8 per 64-channel row) of
// each (tensor, image, head).
__global__ __launch_bounds__(kThreads) void zero_pad_rows_kernel(PadRowsArgs p) {
    const int pad = p.tpad - p.tokens;
    const size_t per_tensor = (size_t)p.images * kHeads * pad * 8;
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= 3 * per_tensor) return;
    const int t = (int)(i / per_tensor);
    const size_t j = i - t * per_tensor;
    const size_t ih = j / ((size_t)pad * 8);  // image * heads + head
    const int row = p.tokens + (int)(j / 8 % pad), piece = (int)(j % 8);
    half_t* const base = t == 0 ? p.q : t == 1 ? p.k : p.v;
    *(half8_t*)(base + ih * p.tpad * kHeadDim + frag_piece(row, piece * 8, kHeadDim)) = half8_t{};
}

}  // namespace

hipError_t launch_zero_pad_rows(const PadRowsArgs& a, hipStream_t s) {
    const size_t n = 3ull * a.images * kHeads * (a.tpad - a.tokens) * 8;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(zero_pad_rows_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_layernorm(const LayerNormArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(layernorm_kernel, dim3((a.rows + 31) / 32), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s) {
    const int waves = (a.rows + 31) / 32 * kStatSlots;
    const int blocks = (waves + kWaves - 1) / kWaves;
    if (a.stats) hipLaunchKernelGGL(splitk_reduce_kernel<true>, dim3(blocks), dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(splitk_reduce_kernel<false>, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dhx
