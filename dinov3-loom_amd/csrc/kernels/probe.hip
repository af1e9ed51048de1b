// Machine-ceiling probes for the roofline (dhx_probe in dinov3_probe.h, built
// into the measurement library libdinov3_probe.so, not the forward's): what
// one CU of this GPU sustains while 32x32x16 f16 MFMAs run, measured with the
// wave's own cycle counter (s_memtime). Every probe runs one workgroup of four
// waves per CU (one wave per SIMD, the whole register file each) on 256
// workgroups, so the numbers are per SIMD with no other wave to hide behind.
//   - the MFMA loop alone, on random or on all-zero operands: cycles per MFMA,
//     TFLOP/s over the whole GPU and the clock those imply (under random
//     operands the chip lowers its clock to stay within its power budget);
//   - the MFMA loop with N VALU FMAs or N exp2 after each MFMA: how much
//     vector work a wave issues under its own MFMAs;
//   - the MFMA loop with N 16-byte buffer loads per 8 MFMAs from footprints
//     that stay in L1, in L2, or stream from HBM, each load consumed three
//     iterations later (latency hidden): the per-CU load rate that still
//     leaves the MFMAs unslowed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "dinov3_probe.h"

namespace dhx {
namespace {

constexpr int kBlocks = 256, kThreads = 256;
constexpr int kOperands = 8;  // half8 operand registers per lane (4 A, 2 B, 2 spare)

struct ProbeOut {
    long long cycles;  // s_memtime cycles of the timed loop, per workgroup (wave 0)
};

// Operands: per lane kOperands random (or zero) half8 values.
__device__ __forceinline__ void load_operands(const half8_t* src, half8_t (&a)[4], half8_t (&b)[2]) {
    const size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = src[t * kOperands + i];
#pragma unroll
    for (int i = 0; i < 2; ++i) b[i] = src[t * kOperands + 4 + i];
}

__device__ __forceinline__ float reduce_acc(const float16_t (&acc)[8]) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][15];
    return s;
}

// 8 independent accumulators; VALU = 0: MFMAs only; VALU > 0 (TRANS false):
// VALU FMAs after each MFMA; TRANS: VALU exp2 (+ a multiply) after each.
template <int VALU, bool TRANS>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(1, 1))) void
mfma_valu_kernel(const half8_t* src, float* sink, int iters, ProbeOut* out) {
    half8_t a[4], b[2];
    load_operands(src, a, b);
    float16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = float16_t{};
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = threadIdx.x * 0.001f + i;
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[j] = mfma32x32x16(a[j % 4], b[j / 4], acc[j]);
#pragma unroll
            for (int v = 0; v < VALU; ++v) {
                float& t = x[(j * VALU + v) % 16];
                t = TRANS ? fast_exp2(t) * 0.5f : t * 1.0001f + 0.5f;
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, TRANS ? 2 * VALU : VALU, 0);
        }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    float s = reduce_acc(acc);
#pragma unroll
    for (int i = 0; i < 16; ++i) s += x[i];
    sink[(size_t)blockIdx.x * kThreads + threadIdx.x] = s;
    if (threadIdx.x == 0) out[blockIdx.x].cycles = t1 - t0;
}

// 8 MFMAs per iteration on CHAINS independent accumulators (MFMA j adds into
// accumulator j % CHAINS): with fewer chains each MFMA depends on the one
// CHAINS positions before it, as in a GEMM wave tile of CHAINS 32x32 blocks
// (the residual GEMMs' 32 x 64 wave tiles are two chains).
template <int CHAINS>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(1, 1))) void
mfma_chain_kernel(const half8_t* src, float* sink, int iters, ProbeOut* out) {
    half8_t a[4], b[2];
    load_operands(src, a, b);
    float16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = float16_t{};
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[j % CHAINS] = mfma32x32x16(a[j % 4], b[j / 4], acc[j % CHAINS]);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    sink[(size_t)blockIdx.x * kThreads + threadIdx.x] = reduce_acc(acc);
    if (threadIdx.x == 0) out[blockIdx.x].cycles = t1 - t0;
}

// LOADS 16-byte buffer loads per 8 MFMAs, each lane 16 B per load, the wave
// cycling through FOOT KB of its own (a compile-time power of two, so the
// block index costs one mask); the loaded fragments feed the MFMAs three
// iterations later (a ring of 4 operand sets).
template <int LOADS, int FOOT>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(1, 1))) void
mfma_load_kernel(const half8_t* src, const half_t* pool, uint64_t pool_bytes, float* sink, int iters,
                 ProbeOut* out) {
    static_assert((FOOT & (FOOT - 1)) == 0, "power of two");
    half8_t a[4], b[2];
    load_operands(src, a, b);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(pool), 0, (int)pool_bytes, kBufferRsrcWord3);
    const int base = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + wave) * FOOT * 1024);
    float16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = float16_t{};
    half8_t ring[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) ring[q][j] = b[j & 1];
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; it += 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[j] = mfma32x32x16(a[j % 4], ring[(q + 1) & 3][j], acc[j]);
                if (j < LOADS) {
                    const int blk = ((it + q) * 8 + j) & (FOOT - 1);  // 1 KB per load instruction
                    ring[q][j] = __builtin_bit_cast(
                        half8_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane * 16, base + blk * 1024, 0));
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (j < LOADS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    sink[(size_t)blockIdx.x * kThreads + threadIdx.x] = reduce_acc(acc);
    if (threadIdx.x == 0) out[blockIdx.x].cycles = t1 - t0;
}

#define PROBE_CHECK(x)                   \
    do {                                 \
        if ((x) != hipSuccess) return 1; \
    } while (0)

}  // namespace
}  // namespace dhx

using namespace dhx;

extern "C" int dhx_probe(int32_t device, int32_t kind, int32_t param, double* results) {
    // results: [0] cycles per 8 MFMAs of one wave, [1] TFLOP/s over the GPU,
    // [2] clock implied (GHz) = cycles / elapsed time. Kinds: 0 MFMAs on
    // random operands, 1 on zeros, 2 with param VALU FMAs per MFMA, 3 with
    // param exp2 per MFMA, 4/5/6 with param buffer loads per 8 MFMAs from an
    // 8 KB (L1) / 16 KB (L2) / 512 KB (HBM) footprint per wave, 7 on param
    // independent accumulator chains.
    if (!results) return 1;
    static const int kValu[] = {0, 2, 4, 6, 8};
    static const int kTrans[] = {1, 2};
    static const int kLoads[] = {0, 2, 3, 4, 6};
    static const int kFoot[] = {8, 16, 512};  // KB per wave: L1, L2, HBM
    static const int kChains[] = {1, 2, 4, 8};
    auto in = [](int v, const int* set, int n) {
        for (int i = 0; i < n; ++i)
            if (set[i] == v) return true;
        return false;
    };
    if (kind < 0 || kind > 7) return 2;
    if ((kind == 1 || kind == 0) && param != 0) return 2;
    if (kind == 2 && !in(param, kValu, 5)) return 2;
    if (kind == 3 && !in(param, kTrans, 2)) return 2;
    if (kind >= 4 && kind <= 6 && !in(param, kLoads, 5)) return 2;
    if (kind == 7 && !in(param, kChains, 4)) return 2;
    PROBE_CHECK(hipSetDevice(device));
    const size_t lanes = (size_t)kBlocks * kThreads;
    std::vector<half_t> host(lanes * kOperands * 8);
    uint32_t x = 12345u;
    for (auto& h : host) {
        x = x * 1664525u + 1013904223u;
        h = kind == 1 ? (half_t)0.f : (half_t)(((x >> 8) / 16777216.f - 0.5f) * 4.f);
    }
    const int foot = kind >= 4 && kind <= 6 ? kFoot[kind - 4] : 0;  // 4: L1 (8 KB), 5: L2 (16 KB), 6: HBM (512 KB)
    half8_t* src = nullptr;
    half_t* pool = nullptr;
    float* sink = nullptr;
    ProbeOut* out = nullptr;
    const uint64_t pool_bytes = (uint64_t)kBlocks * 4 * foot * 1024;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 1;
    do {
        if (hipMalloc(&src, host.size() * 2) != hipSuccess) break;
        if (hipMemcpy(src, host.data(), host.size() * 2, hipMemcpyHostToDevice) != hipSuccess) break;
        if (hipMalloc(&sink, lanes * 4) != hipSuccess || hipMalloc(&out, kBlocks * sizeof(ProbeOut)) != hipSuccess) break;
        if (pool_bytes) {  // random f16 throughout (operand data changes the power drawn)
            if (hipMalloc(&pool, pool_bytes) != hipSuccess) break;
            const uint64_t chunk = host.size() * 2;
            bool ok = true;
            for (uint64_t off = 0; ok && off < pool_bytes; off += chunk)
                ok = hipMemcpy((char*)pool + off, host.data(), std::min(chunk, pool_bytes - off), hipMemcpyHostToDevice) ==
                     hipSuccess;
            if (!ok) break;
        }
        if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) break;
        const int iters = 4000;
        auto launch = [&]() -> hipError_t {
            const dim3 g(kBlocks), t(kThreads);
            switch (kind) {
            case 0:
            case 1: hipLaunchKernelGGL((mfma_valu_kernel<0, false>), g, t, 0, 0, src, sink, iters, out); break;
            case 2:
                switch (param) {
                case 0: hipLaunchKernelGGL((mfma_valu_kernel<0, false>), g, t, 0, 0, src, sink, iters, out); break;
                case 2: hipLaunchKernelGGL((mfma_valu_kernel<2, false>), g, t, 0, 0, src, sink, iters, out); break;
                case 4: hipLaunchKernelGGL((mfma_valu_kernel<4, false>), g, t, 0, 0, src, sink, iters, out); break;
                case 6: hipLaunchKernelGGL((mfma_valu_kernel<6, false>), g, t, 0, 0, src, sink, iters, out); break;
                default: hipLaunchKernelGGL((mfma_valu_kernel<8, false>), g, t, 0, 0, src, sink, iters, out); break;
                }
                break;
            case 3:
                if (param == 1) hipLaunchKernelGGL((mfma_valu_kernel<1, true>), g, t, 0, 0, src, sink, iters, out);
                else hipLaunchKernelGGL((mfma_valu_kernel<2, true>), g, t, 0, 0, src, sink, iters, out);
                break;
            case 7:
                switch (param) {
                case 1: hipLaunchKernelGGL((mfma_chain_kernel<1>), g, t, 0, 0, src, sink, iters, out); break;
                case 2: hipLaunchKernelGGL((mfma_chain_kernel<2>), g, t, 0, 0, src, sink, iters, out); break;
                case 4: hipLaunchKernelGGL((mfma_chain_kernel<4>), g, t, 0, 0, src, sink, iters, out); break;
                default: hipLaunchKernelGGL((mfma_chain_kernel<8>), g, t, 0, 0, src, sink, iters, out); break;
                }
                break;
            default: {
                const uint64_t pb = pool_bytes;
                // (LOADS, FOOT) instantiations: LOADS in kLoads, FOOT in kFoot.
                auto go = [&](auto L, auto F) {
                    hipLaunchKernelGGL((mfma_load_kernel<decltype(L)::value, decltype(F)::value>), g, t, 0, 0, src,
                                       pool, pb, sink, iters, out);
                };
                auto by_foot = [&](auto L) {
                    if (foot == 8) go(L, std::integral_constant<int, 8>{});
                    else if (foot == 16) go(L, std::integral_constant<int, 16>{});
                    else go(L, std::integral_constant<int, 512>{});
                };
                switch (param) {
                case 0: by_foot(std::integral_constant<int, 0>{}); break;
                case 2: by_foot(std::integral_constant<int, 2>{}); break;
                case 3: by_foot(std::integral_constant<int, 3>{}); break;
                case 4: by_foot(std::integral_constant<int, 4>{}); break;
                default: by_foot(std::integral_constant<int, 6>{}); break;
                }
            }
            }
            return hipGetLastError();
        };
        if (launch() != hipSuccess || hipDeviceSynchronize() != hipSuccess) break;  // warm-up
        if (hipEventRecord(e0) != hipSuccess || launch() != hipSuccess || hipEventRecord(e1) != hipSuccess ||
            hipEventSynchronize(e1) != hipSuccess)
            break;
        float ms = 0.f;
        std::vector<ProbeOut> cyc(kBlocks);
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess ||
            hipMemcpy(cyc.data(), out, kBlocks * sizeof(ProbeOut), hipMemcpyDeviceToHost) != hipSuccess)
            break;
        double mean = 0.0;
        for (const auto& c : cyc) mean += (double)c.cycles;
        mean /= kBlocks;
        results[0] = mean / iters;
        results[1] = (double)kBlocks * 4 * iters * 8 * 32768.0 / (ms * 1e-3) / 1e12;
        results[2] = mean / (ms * 1e-3) / 1e9;
        rc = 0;
    } while (false);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(src);
    (void)hipFree(pool);
    (void)hipFree(sink);
    (void)hipFree(out);
    return rc;
}
