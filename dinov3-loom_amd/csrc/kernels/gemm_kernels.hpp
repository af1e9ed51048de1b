// The GEMM variants of the forward pass, as kernels templated on the tile
// shape (gemm.hip instantiates the shapes used in production). Replaces the
// reference's Loom GEMMs: kernels/matmul_bias_f16_wmma.loom (patch embed,
// with the embed scatter of kernels/embed_scatter_f32.loom fused in),
// matmul_qkv_rope_f16_wmma.loom, matmul_resid_f16_wmma.loom,
// matmul_swiglu_f16_wmma.loom and matmul_splitk_f16_wmma.loom.
#pragma once
#include "gemm_core.hpp"
#include "launch.hpp"

namespace dhx {
namespace gemm {

// A operand of the patch embedding, gathered from NCHW f32 pixels (the im2col
// of lib.rs:265-280): row m = image*P + gy*G + gx, column k = c*256 + dy*16 +
// dx. A 64-wide stage covers one channel and four pixel rows of the patch;
// consecutive lanes read consecutive 16-byte pieces of a pixel row, and the
// patches of one grid row are adjacent in memory. Pixels are narrowed to f16
// on the way to LDS.
template <class T>
struct PatchRows {
    static constexpr int CHUNKS = T::BM * BK / 4 / T::THREADS;
    static_assert(T::BM * BK / 4 % T::THREADS == 0, "patch tile splits evenly");
    const float* px;
    int M, G, P, S;
    float4_t r[CHUNKS];
    __device__ __forceinline__ void load(int m0, int /*n0*/, int kt, int tid) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * T::THREADS;
            const int dxq = c & 3, row = (c >> 2) % T::BM, dyl = c / (4 * T::BM);
            const int m = min(m0 + row, M - 1);  // rows past M feed unstored outputs
            const int img = m / P, p = m - img * P, gy = p / G, gx = p - gy * G;
            const int ch = kt >> 2, dy = (kt & 3) * 4 + dyl;
            r[i] = *(const float4_t*)(px + (((size_t)img * 3 + ch) * S + gy * 16 + dy) * S + gx * 16 + dxq * 4);
        }
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * T::THREADS;
            const int dxq = c & 3, row = (c >> 2) % T::BM, dyl = c / (4 * T::BM);
            *(half4_t*)(s + row * LDK + dyl * 16 + dxq * 4) = to_half4(r[i]);
        }
    }
};

// Writes this wave's (mean, M2) partial of row m over its 64 columns: the
// lane holds 32 of them (v, already rounded to the f16 values stored in x),
// its partner lane l ^ 32 the other 32. Both partners must call this.
__device__ __forceinline__ void slot_stats(float* stats, size_t m, int slot, const float4_t (&v)[2][4], int hi) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) s += (v[i][g][0] + v[i][g][1]) + (v[i][g][2] + v[i][g][3]);
    s += __shfl_xor(s, 32, 64);
    const float mean = s * (1.0f / 64.0f);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) q += (v[i][g][e] - mean) * (v[i][g][e] - mean);
    q += __shfl_xor(q, 32, 64);
    if (hi == 0) *(float2_t*)(stats + m * kStatFloats + slot * 2) = float2_t{mean, q};
}

__device__ __forceinline__ float4_t widen(half4_t h) { return float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]}; }

// Patch embedding + CLS/register scatter into the f16 residual stream x
// (with STATS, also the LayerNorm row statistics of x).
template <class T, bool STATS>
__global__ __launch_bounds__(T::THREADS) void patch_embed_kernel(PatchEmbedArgs p) {
    static_assert(!STATS || T::TN == 64, "one statistics slot per wave");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * P;
    constexpr int NT = kHidden / T::BN;
    const int S = 16 * p.grid;
    PatchRows<T> al[2] = {{p.pixels, M, p.grid, P, S}, {p.pixels, M, p.grid, P, S}};
    WeightRows<T> wl[2] = {{{}, p.w, 768, 0}, {{}, p.w, 768, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((M + T::BM - 1) / T::BM), 768 / BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = f.row(j);
            if (m >= M) continue;
            const int img = m / P, patch = m - img * P;
            const size_t row = (size_t)img * Tok + kPrefix + patch;
            half_t* dst = p.x + row * kHidden;
            float4_t v[T::FN][4];
#pragma unroll
            for (int i = 0; i < T::FN; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = f.col(i, g);
                    const half4_t h = to_half4(group4(acc.v[i][j], g) + ld4(p.bias + n));
                    *(half4_t*)(dst + n) = h;
                    v[i][g] = widen(h);
                }
            if constexpr (STATS) slot_stats(p.stats, row, f.n_base / 64, v, f.hi);
        }
        // CLS + registers of every image whose first patch row lies in this tile.
        const int m_end = min(m0 + T::BM, M);
        for (int img = (m0 + P - 1) / P; img * P < m_end; ++img) {
            for (int idx = threadIdx.x; idx < kPrefix * T::BN; idx += T::THREADS) {
                const int row = idx / T::BN, col = n0 + idx % T::BN;
                p.x[((size_t)img * Tok + row) * kHidden + col] = (half_t)p.prefix[row * kHidden + col];
            }
            if constexpr (STATS) {
                constexpr int slots = T::BN / 64;
                for (int idx = threadIdx.x; idx < kPrefix * slots * 2; idx += T::THREADS) {
                    const int row = idx / (slots * 2), e = idx % (slots * 2);
                    const int off = (n0 / 64) * 2 + e;
                    p.stats[((size_t)img * Tok + row) * kStatFloats + off] = p.prefix_stats[row * kStatFloats + off];
                }
            }
        }
    });
}

// QKV + bias + 2D RoPE. A wave's 64 columns are exactly one head of q, k or
// v, so channel c and its rotation partner c+32 are acc.v[0] / acc.v[1] of
// the same lane. q, k are written head-major, v transposed.
template <class T, bool LN>
__global__ __launch_bounds__(T::THREADS) void qkv_rope_kernel(QkvArgs p) {
    static_assert(T::TN == kHeadDim, "one head per wave");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * Tok;
    constexpr int NT = 3 * kHidden / T::BN;
    ActRows<T> al[2] = {{{}, p.h, kHidden, M, 0}, {{}, p.h, kHidden, M, 0}};
    WeightRows<T> wl[2] = {{{}, p.w, kHidden, 0}, {{}, p.w, kHidden, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((M + T::BM - 1) / T::BM), kHidden / BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int part = f.n_base / kHidden, head = (f.n_base % kHidden) / kHeadDim;
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = f.row(j);
            if (m >= M) continue;
            const int img = m / Tok, tok = m - img * Tok;
            const size_t bh = (size_t)img * kHeads + head;
            const bool rotate = part < 2 && tok >= kPrefix;
            RowNorm rn{0.f, 1.f};
            if constexpr (LN) rn = row_norm(p.stats, m);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = g * 8 + f.hi * 4;  // channel in the head (0..31); partner c + 32
                float4_t lo = group4(acc.v[0][j], g), up = group4(acc.v[1][j], g);
                if constexpr (LN) {
                    lo = (lo - rn.mean * ld4(p.wsum + f.n_base + c)) * rn.rstd;
                    up = (up - rn.mean * ld4(p.wsum + f.n_base + 32 + c)) * rn.rstd;
                }
                lo += ld4(p.bias + f.n_base + c);
                up += ld4(p.bias + f.n_base + 32 + c);
                if (rotate) {
                    const float* cs = p.cos + (tok - kPrefix) * kHeadDim;
                    const float* sn = p.sin + (tok - kPrefix) * kHeadDim;
                    const float4_t nlo = lo * ld4(cs + c) - up * ld4(sn + c);            // x[c]cos - x[c+32]sin
                    const float4_t nup = up * ld4(cs + 32 + c) + lo * ld4(sn + 32 + c);  // x[c+32]cos + x[c]sin
                    lo = nlo;
                    up = nup;
                }
                if (part < 2) {
                    half_t* dst = (part == 0 ? p.q : p.k) + (bh * p.tpad + tok) * kHeadDim;
                    *(half4_t*)(dst + c) = to_half4(lo);
                    *(half4_t*)(dst + 32 + c) = to_half4(up);
                } else {
                    half_t* dst = p.vt + bh * kHeadDim * p.tpad + tok;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dst[(size_t)(c + e) * p.tpad] = (half_t)lo[e];
                        dst[(size_t)(c + 32 + e) * p.tpad] = (half_t)up[e];
                    }
                }
            }
        }
    });
}

// Residual GEMM: x += ls * (A W^T + b), in place on the f16 residual stream
// (with STATS, also the LayerNorm row statistics of the updated x).
template <class T, bool STATS>
__global__ __launch_bounds__(T::THREADS) void resid_kernel(ResidArgs p) {
    static_assert(!STATS || T::TN == 64, "one statistics slot per wave");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    constexpr int NT = kHidden / T::BN;
    ActRows<T> al[2] = {{{}, p.a, p.k, p.rows, 0}, {{}, p.a, p.k, p.rows, 0}};
    WeightRows<T> wl[2] = {{{}, p.w, p.k, 0}, {{}, p.w, p.k, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((p.rows + T::BM - 1) / T::BM), p.k / BK, lds,
                       [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = f.row(j);
            if (m >= p.rows) continue;
            half_t* xr = p.x + (size_t)m * kHidden;
            float4_t v[T::FN][4];
#pragma unroll
            for (int i = 0; i < T::FN; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = f.col(i, g);
                    const float4_t upd = (group4(acc.v[i][j], g) + ld4(p.bias + n)) * ld4(p.ls + n);
                    const half4_t h = to_half4(widen(*(const half4_t*)(xr + n)) + upd);
                    *(half4_t*)(xr + n) = h;
                    v[i][g] = widen(h);
                }
            if constexpr (STATS) slot_stats(p.stats, m, f.n_base / 64, v, f.hi);
        }
    });
}

// SwiGLU dual GEMM. W rows are packed as blocks of 32 gate rows followed by
// the 32 matching up rows, so a wave's 64 columns are 32 gate and 32 up
// columns of the same 32 outputs.
template <class T, bool LN>
__global__ __launch_bounds__(T::THREADS) void swiglu_kernel(SwigluArgs p) {
    static_assert(T::TN == 64, "gate/up pair per wave");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    constexpr int NT = 2 * kFF / T::BN;
    ActRows<T> al[2] = {{{}, p.h, kHidden, p.rows, 0}, {{}, p.h, kHidden, p.rows, 0}};
    WeightRows<T> wl[2] = {{{}, p.w, kHidden, 0}, {{}, p.w, kHidden, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((p.rows + T::BM - 1) / T::BM), kHidden / BK, lds,
                       [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int out_base = f.n_base / 2;
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = f.row(j);
            if (m >= p.rows) continue;
            half_t* dst = p.act + (size_t)m * kFF + out_base;
            RowNorm rn{0.f, 1.f};
            if constexpr (LN) rn = row_norm(p.stats, m);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = g * 8 + f.hi * 4;
                float4_t gate = group4(acc.v[0][j], g), up = group4(acc.v[1][j], g);
                if constexpr (LN) {
                    gate = (gate - rn.mean * ld4(p.wsum + f.n_base + c)) * rn.rstd;
                    up = (up - rn.mean * ld4(p.wsum + f.n_base + 32 + c)) * rn.rstd;
                }
                gate += ld4(p.bias + f.n_base + c);
                up += ld4(p.bias + f.n_base + 32 + c);
                const float4_t y = float4_t{silu(gate[0]), silu(gate[1]), silu(gate[2]), silu(gate[3])} * up;
                *(half4_t*)(dst + c) = to_half4(y);
            }
        }
    });
}

// Split-K GEMM into f32 slabs [split][rows][384]; no atomics, so results do
// not depend on scheduling. The tile space is (split, m tile) x n tile: a
// tile's m origin runs over splits * padded rows, and both loaders decode the
// split (their K offset) from it.
template <class T>
struct SplitDecode {
    int mt, kc;
    __device__ __forceinline__ int split(int m0) const { return m0 / T::BM / mt; }
    __device__ __forceinline__ int row0(int m0) const { return m0 - split(m0) * mt * T::BM; }
};

template <class T>
struct SplitActRows {
    ActRows<T> a;
    SplitDecode<T> d;
    __device__ __forceinline__ void load(int m0, int n0, int kt, int tid) {
        a.k_off = d.split(m0) * d.kc;
        a.load(d.row0(m0), n0, kt, tid);
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const { a.store(s, tid); }
};

template <class T>
struct SplitWeightRows {
    WeightRows<T> w;
    SplitDecode<T> d;
    __device__ __forceinline__ void load(int m0, int n0, int kt, int tid) {
        w.k_off = d.split(m0) * d.kc;
        w.load(m0, n0, kt, tid);
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const { w.store(s, tid); }
};

template <class T>
__global__ __launch_bounds__(T::THREADS) void splitk_kernel(SplitKArgs p) {
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    constexpr int NT = kHidden / T::BN;
    const int MT = (p.rows + T::BM - 1) / T::BM;
    const SplitDecode<T> d{MT, p.k / p.splits};
    SplitActRows<T> al[2] = {{{{}, p.a, p.k, p.rows, 0}, d}, {{{}, p.a, p.k, p.rows, 0}, d}};
    SplitWeightRows<T> wl[2] = {{{{}, p.w, p.k, 0}, d}, {{{}, p.w, p.k, 0}, d}};
    gemm_tile<T>(al, wl, NT, NT * MT * p.splits, d.kc / BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(d.row0(m0), n0);
        float* slab = p.partials + (size_t)d.split(m0) * p.rows * kHidden;
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = f.row(j);
            if (m >= p.rows) continue;
#pragma unroll
            for (int i = 0; i < T::FN; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *(float4_t*)(slab + (size_t)m * kHidden + f.col(i, g)) = group4(acc.v[i][j], g);
        }
    });
}

}  // namespace gemm
}  // namespace dhx
