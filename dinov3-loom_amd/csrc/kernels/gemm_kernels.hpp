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
    static_assert(T::BK == 64, "a stage is one channel x four pixel rows");
    static constexpr int CHUNKS = T::BM * T::BK / 4 / T::THREADS;
    static_assert(T::BM * T::BK / 4 % T::THREADS == 0, "patch tile splits evenly");
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
            *(half4_t*)(s + row * T::LDK + dyl * 16 + dxq * 4) = to_half4(r[i]);
        }
    }
};

// Writes the (mean, M2) partial of row m over the 64 columns of one
// statistics slot, whose values are spread over 8 consecutive lanes (8 each,
// already rounded to the f16 values stored in x). All 8 lanes must call this.
__device__ __forceinline__ void slot_stats(float* stats, size_t m, int slot, const float (&v)[8], int lane8) {
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    const float mean = s * (1.0f / 64.0f);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) q += (v[e] - mean) * (v[e] - mean);
    q += __shfl_xor(q, 1, 64);
    q += __shfl_xor(q, 2, 64);
    q += __shfl_xor(q, 4, 64);
    if (lane8 == 0) *(float2_t*)(stats + m * kStatFloats + slot * 2) = float2_t{mean, q};
}

__device__ __forceinline__ float4_t widen(half4_t h) { return float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]}; }

// Patch embedding + CLS/register scatter into the f16 residual stream x
// (with STATS, also the LayerNorm row statistics of x). Each wave rounds its
// 32 x 64 block to f16 into LDS, then writes it as 128-byte row pieces
// (8 lanes per row), which is also the layout the row statistics need.
template <class T, bool STATS>
__global__ __launch_bounds__(T::THREADS) void patch_embed_kernel(PatchEmbedArgs p) {
    static_assert(T::TN == 64, "one statistics slot per wave");
    constexpr int SP = T::TN + 8;  // staging pitch in halfs
    static_assert(T::WAVES * T::TM * SP <= T::LDS_HALFS, "staging fits the stage buffers");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * P;
    constexpr int NT = kHidden / T::BN;
    const int S = 16 * p.grid;
    PatchRows<T> al[2] = {{p.pixels, M, p.grid, P, S}, {p.pixels, M, p.grid, P, S}};
    WeightRows<T> wl[2] = {{{}, p.w, 768, 0}, {{}, p.w, 768, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((M + T::BM - 1) / T::BM), 768 / T::BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        half_t* const st = lds + (threadIdx.x >> 6) * (T::TM * SP);
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = f.col(i, g);
                const float4_t b = ld4(p.bias + n);
#pragma unroll
                for (int j = 0; j < T::FM; ++j)
                    *(half4_t*)(st + (j * 32 + f.l32) * SP + (n - f.n_base)) = to_half4(group4(acc.v[i][j], g) + b);
            }
        wave_lds_sync();
        const int lane = threadIdx.x & 63, r0 = lane >> 3, c8 = (lane & 7) * 8;
#pragma unroll
        for (int it = 0; it < T::TM / 8; ++it) {
            const int r = it * 8 + r0, m = f.m_base + r;
            if (m >= M) continue;  // uniform over the 8 lanes of a row
            const size_t row = (size_t)m + (size_t)(m / P + 1) * kPrefix;  // image*Tok + kPrefix + patch
            const half8_t h = *(const half8_t*)(st + r * SP + c8);
            *(half8_t*)(p.x + row * kHidden + f.n_base + c8) = h;
            if constexpr (STATS) {
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
                slot_stats(p.stats, row, f.n_base / 64, v, lane & 7);
            }
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
// the same lane, and both use angle column c of the RoPE tables (DINOv3's
// tables repeat columns 0..31 in 32..63; only the first half is read).
// Results are rounded to f16 into a per-wave LDS block, then each wave
// writes its rows as whole 128-byte head rows: q, k and v are all
// head-major [image][head][tpad][64], and the rows of one image are
// contiguous there.
template <class T, bool LN>
__global__ __launch_bounds__(T::THREADS) void qkv_rope_kernel(QkvArgs p) {
    static_assert(T::TN == kHeadDim, "one head per wave");
    constexpr int SP = kHeadDim + 8;  // staging pitch in halfs
    static_assert(T::WAVES * T::TM * SP <= T::LDS_HALFS, "staging fits the stage buffers");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * Tok;
    constexpr int NT = 3 * kHidden / T::BN;
    ActRows<T> al[2] = {{{}, p.h, kHidden, M, 0}, {{}, p.h, kHidden, M, 0}};
    WeightRows<T> wl[2] = {{{}, p.w, kHidden, 0}, {{}, p.w, kHidden, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((M + T::BM - 1) / T::BM), kHidden / T::BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int lane = threadIdx.x & 63;
        half_t* const st = lds + (threadIdx.x >> 6) * (T::TM * SP);
        const int part = f.n_base / kHidden, head = (f.n_base % kHidden) / kHeadDim;
        float4_t bias[2][4], wsum[2][4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = g * 8 + f.hi * 4;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                bias[i][g] = ld4(p.bias + f.n_base + 32 * i + c);
                if constexpr (LN) wsum[i][g] = ld4(p.wsum + f.n_base + 32 * i + c);
            }
        }
        const bool rope_part = part < 2;  // uniform per wave
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int m = min(f.row(j), M - 1);  // rows past M are computed but never written out
            const int tok = m % Tok;
            // RoPE angles of this row, loaded together before any use (lanes
            // hold different rows, so each load is a gather; one round trip
            // per row instead of one per register group). Prefix rows and v
            // columns rotate by cos 1, sin 0.
            const size_t angle_row = (size_t)max(tok - kPrefix, 0) * kHeadDim;
            float4_t co[4], si[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                co[g] = float4_t{1.f, 1.f, 1.f, 1.f};
                si[g] = float4_t{};
                if (rope_part) {
                    co[g] = ld4(p.cos + angle_row + g * 8 + f.hi * 4);
                    si[g] = ld4(p.sin + angle_row + g * 8 + f.hi * 4);
                }
            }
            if (tok < kPrefix) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    co[g] = float4_t{1.f, 1.f, 1.f, 1.f};
                    si[g] = float4_t{};
                }
            }
            RowNorm rn{0.f, 1.f};
            if constexpr (LN) rn = row_norm(p.stats, m);
            half_t* const row = st + (j * 32 + f.l32) * SP;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = g * 8 + f.hi * 4;  // channel in the head (0..31); partner c + 32
                float4_t lo = group4(acc.v[0][j], g), up = group4(acc.v[1][j], g);
                if constexpr (LN) {
                    lo = (lo - rn.mean * wsum[0][g]) * rn.rstd;
                    up = (up - rn.mean * wsum[1][g]) * rn.rstd;
                }
                lo += bias[0][g];
                up += bias[1][g];
                const float4_t nlo = lo * co[g] - up * si[g];  // x[c] cos - x[c+32] sin
                const float4_t nup = up * co[g] + lo * si[g];  // x[c+32] cos + x[c] sin
                *(half4_t*)(row + c) = to_half4(nlo);
                *(half4_t*)(row + 32 + c) = to_half4(nup);
            }
        }
        wave_lds_sync();
        // Copy-out: 8 lanes per 128-byte row, 8 rows per pass.
        half_t* const out = part == 0 ? p.q : part == 1 ? p.k : p.v;
        const int r0 = lane >> 3, ch = (lane & 7) * 8;
        int m = f.m_base + r0;
        int img = m / Tok, tok = m - img * Tok;
#pragma unroll
        for (int it = 0; it < T::TM / 8; ++it) {
            if (m < M)
                *(half8_t*)(out + (((size_t)img * kHeads + head) * p.tpad + tok) * kHeadDim + ch) =
                    *(const half8_t*)(st + (it * 8 + r0) * SP + ch);
            m += 8;
            tok += 8;
            while (tok >= Tok) {
                tok -= Tok;
                ++img;
            }
        }
    });
}

// Residual GEMM: x += ls * (A W^T + b), in place on the f16 residual stream
// (with STATS, also the LayerNorm row statistics of the updated x); P
// register sets in the K loop (a third set measured no faster, even for the
// K = 1536 down projection). Each wave
// stages its f32 update (32 x 64) in LDS, then reads and writes x as
// 128-byte row pieces, 8 lanes per row.
template <class T, bool STATS, int P>
__global__ __launch_bounds__(T::THREADS) void resid_kernel(ResidArgs p) {
    static_assert(T::TN == 64, "one statistics slot per wave");
    constexpr int SPF = T::TN + 4;  // staging pitch in floats
    static_assert(T::WAVES * T::TM * SPF * 4 <= T::LDS_BYTES, "staging fits the stage buffers");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    constexpr int NT = kHidden / T::BN;
    ActRows<T> al[P];
    WeightRows<T> wl[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        al[i] = ActRows<T>{{}, p.a, p.k, p.rows, 0};
        wl[i] = WeightRows<T>{{}, p.w, p.k, 0};
    }
    gemm_tile<T>(al, wl, NT, NT * ((p.rows + T::BM - 1) / T::BM), p.k / T::BK, lds,
                       [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        float* const st = reinterpret_cast<float*>(lds) + (threadIdx.x >> 6) * (T::TM * SPF);
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = f.col(i, g);
                const float4_t b = ld4(p.bias + n), l = ld4(p.ls + n);
#pragma unroll
                for (int j = 0; j < T::FM; ++j)
                    *(float4_t*)(st + (j * 32 + f.l32) * SPF + (n - f.n_base)) = (group4(acc.v[i][j], g) + b) * l;
            }
        wave_lds_sync();
        const int lane = threadIdx.x & 63, r0 = lane >> 3, c8 = (lane & 7) * 8;
#pragma unroll
        for (int it = 0; it < T::TM / 8; ++it) {
            const int r = it * 8 + r0, m = f.m_base + r;
            if (m >= p.rows) continue;  // uniform over the 8 lanes of a row
            half_t* const xr = p.x + (size_t)m * kHidden + f.n_base + c8;
            const half8_t old = *(const half8_t*)xr;
            const float4_t u0 = *(const float4_t*)(st + r * SPF + c8), u1 = *(const float4_t*)(st + r * SPF + c8 + 4);
            half8_t h;
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[e] = (half_t)((float)old[e] + u0[e]);
                h[e + 4] = (half_t)((float)old[e + 4] + u1[e]);
            }
            *(half8_t*)xr = h;
            if constexpr (STATS) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
                slot_stats(p.stats, m, f.n_base / 64, v, lane & 7);
            }
        }
    });
}

// SwiGLU dual GEMM. W rows are packed as blocks of 32 gate rows followed by
// the 32 matching up rows, so a wave's 64 columns are 32 gate and 32 up
// columns of the same 32 outputs. The workgroup's BM x BN/2 block of act is
// staged in LDS and written as whole row pieces of BN bytes.
template <class T, bool LN>
__global__ __launch_bounds__(T::THREADS) void swiglu_kernel(SwigluArgs p) {
    static_assert(T::TN % 64 == 0, "whole gate/up pairs per wave");
    constexpr int OW = T::BN / 2;   // act columns per workgroup
    constexpr int SP = OW + 8;      // staging pitch in halfs
    constexpr int LPR = OW / 8;     // lanes per row in the copy-out
    static_assert(T::BM * SP <= T::LDS_HALFS && T::THREADS % LPR == 0, "staging fits the stage buffers");
    __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALFS];
    constexpr int NT = 2 * kFF / T::BN;
    ActRows<T> al[2] = {{{}, p.h, kHidden, p.rows, 0}, {{}, p.h, kHidden, p.rows, 0}};
    WeightRows<T> wl[2] = {{{}, p.w, kHidden, 0}, {{}, p.w, kHidden, 0}};
    gemm_tile<T>(al, wl, NT, NT * ((p.rows + T::BM - 1) / T::BM), kHidden / T::BK, lds,
                       [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int wave = threadIdx.x >> 6;
        half_t* const st = lds + (wave % T::WGM) * T::TM * SP + (wave / T::WGM) * (T::TN / 2);
        RowNorm rn[T::FM];
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            rn[j] = RowNorm{0.f, 1.f};
            if constexpr (LN) rn[j] = row_norm(p.stats, min(f.row(j), p.rows - 1));
        }
        // Pair q of the wave: gate = acc.v[2q], up = acc.v[2q + 1], outputs
        // 32q .. 32q+31 of the wave's TN/2. Column constants are loaded per
        // register group to keep the register footprint small next to acc.
#pragma unroll
        for (int q = 0; q < T::FN / 2; ++q)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = g * 8 + f.hi * 4, n = f.n_base + 64 * q + c;
                const float4_t bg = ld4(p.bias + n), bu = ld4(p.bias + n + 32);
                float4_t wg{}, wu{};
                if constexpr (LN) {
                    wg = ld4(p.wsum + n);
                    wu = ld4(p.wsum + n + 32);
                }
#pragma unroll
                for (int j = 0; j < T::FM; ++j) {
                    float4_t gate = group4(acc.v[2 * q][j], g), up = group4(acc.v[2 * q + 1][j], g);
                    if constexpr (LN) {
                        gate = (gate - rn[j].mean * wg) * rn[j].rstd;
                        up = (up - rn[j].mean * wu) * rn[j].rstd;
                    }
                    gate += bg;
                    up += bu;
                    const float4_t y = float4_t{silu(gate[0]), silu(gate[1]), silu(gate[2]), silu(gate[3])} * up;
                    *(half4_t*)(st + (j * 32 + f.l32) * SP + 32 * q + c) = to_half4(y);
                }
            }
        lds_barrier();
        const int r0 = threadIdx.x / LPR, c8 = (threadIdx.x % LPR) * 8;
#pragma unroll
        for (int it = 0; it < T::BM * LPR / T::THREADS; ++it) {
            const int r = it * (T::THREADS / LPR) + r0, m = m0 + r;
            if (m < p.rows) *(half8_t*)(p.act + (size_t)m * kFF + n0 / 2 + c8) = *(const half8_t*)(lds + r * SP + c8);
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
    gemm_tile<T>(al, wl, NT, NT * MT * p.splits, d.kc / T::BK, lds, [&](const Acc<T>& acc, int m0, int n0) {
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
