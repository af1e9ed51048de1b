// The GEMM variants of the forward pass, as kernels templated on the tile
// shape (gemm.hip instantiates the shapes used in production). Replaces the
// reference's Loom GEMMs: kernels/matmul_bias_f16_wmma.loom (patch embed,
// with the embed scatter of kernels/embed_scatter_f32.loom fused in),
// matmul_qkv_rope_f16_wmma.loom, matmul_resid_f16_wmma.loom,
// matmul_swiglu_f16_wmma.loom and matmul_splitk_f16_wmma.loom.
//
// Activations (x, h, attn, act) are kept in fragment order (common.hpp):
// every GEMM except the patch embedding loads its activation operand
// straight into registers (ActFrags) and stages only the weights in LDS,
// with the workgroup's waves stacked along M (32 x 128 per wave).
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
    static constexpr bool kInRegs = false;
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

// (mean, M2) partial of one row over a 64-column statistics slot whose
// values are split between this lane (32 of them, already rounded to the f16
// values stored in x) and its partner lane l ^ 32. Both partners call this;
// the lane with hi == 0 writes.
__device__ __forceinline__ void pair_stats(float* stats, size_t m, int slot, const float (&v)[32], int hi, bool store) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) s += v[e];
    s = half_pair_sum(s);
    const float mean = s * (1.0f / 64.0f);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) q += (v[e] - mean) * (v[e] - mean);
    q = half_pair_sum(q);
    if (store && hi == 0) *(float2_t*)(stats + m * kStatFloats + slot * 2) = float2_t{mean, q};
}

// Patch embedding + CLS/register scatter into the f16 residual stream x
// (fragment order; with STATS, also the LayerNorm row statistics of x). Each
// wave rounds its 32 x 64 block to f16 into LDS, then writes it as fragment
// pieces, lane (l, hi) taking row l and the half hi of each 16-column block.
template <class T, bool STATS>
__global__ __launch_bounds__(T::THREADS) void patch_embed_kernel(PatchEmbedArgs p) {
    static_assert(T::TN == 64 && T::TM == 32, "one 32-row block and one statistics slot per wave");
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
                *(half4_t*)(st + f.l32 * SP + (n - f.n_base)) = to_half4(group4(acc.v[i][0], g) + b);
            }
        wave_lds_sync();
        const int m = f.m_base + f.l32;
        const bool valid = m < M;
        const size_t row = valid ? (size_t)m + (size_t)(m / P + 1) * kPrefix : 0;  // image*Tok + kPrefix + patch
        // The wave's 32 patch rows land in x rows row(m_base) .. at most
        // 32 + 5 * (32 / P + 1) rows further: within 8 row blocks.
        const size_t rb0 = ((size_t)f.m_base + (size_t)(f.m_base / P + 1) * kPrefix) / 32;
        const WtOut xo(p.x + rb0 * (kHidden / 16) * 512, 8 * (kHidden / 16) * 1024);
        float v[32];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const half8_t h = *(const half8_t*)(st + f.l32 * SP + ks * 16 + f.hi * 8);
            if (valid)
                xo.store((uint32_t)(frag_piece((int)row, f.n_base + ks * 16 + f.hi * 8, kHidden) - rb0 * (kHidden / 16) * 512) * 2, h);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[ks * 8 + e] = (float)h[e];
        }
        if constexpr (STATS) pair_stats(p.stats, row, f.n_base / 64, v, f.hi, valid);
        // CLS + registers of every image whose first patch row lies in this tile.
        const int m_end = min(m0 + T::BM, M);
        for (int img = (m0 + P - 1) / P; img * P < m_end; ++img) {
            for (int idx = threadIdx.x; idx < kPrefix * T::BN; idx += T::THREADS) {
                const int r = idx / T::BN, col = n0 + idx % T::BN;
                p.x[frag_piece(img * Tok + r, col & ~7, kHidden) + (col & 7)] = (half_t)p.prefix[r * kHidden + col];
            }
            if constexpr (STATS) {
                constexpr int slots = T::BN / 64;
                for (int idx = threadIdx.x; idx < kPrefix * slots * 2; idx += T::THREADS) {
                    const int r = idx / (slots * 2), e = idx % (slots * 2);
                    const int off = (n0 / 64) * 2 + e;
                    p.stats[((size_t)img * Tok + r) * kStatFloats + off] = p.prefix_stats[r * kStatFloats + off];
                }
            }
        }
    });
}

template <class T>
__device__ __forceinline__ void init_frags(ActFrags<T> (&al)[2], const half_t* a, int rows, int k, int ks_off = 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        al[i].a = a;
        al[i].ksteps = k / 16;
        al[i].mblocks = (rows + 31) / 32;
        al[i].ks_off = ks_off;
    }
}

// RoPE angles in LDS. DINOv3's tables are separable (weights.rs:127-144):
// the angle of channel c < 16 of patch (gy, gx) depends on gy only, that of
// channel 16 <= c < 32 on gx only, and channels 32..63 repeat 0..31. Four
// [R][16] float tables (R = the grid side rounded up to 16) hold every angle
// the QKV epilogue needs: cos and sin of the row part (table row gy, from
// patch (gy, 0) of the full [P][64] tables) and of the column part (table
// row gx, from patch (0, gx)), the same float values the full tables hold.
__host__ __device__ constexpr int rope_table_rows(int grid) { return (grid + 15) / 16 * 16; }
__host__ __device__ constexpr int rope_lds_bytes(int grid) { return 4 * rope_table_rows(grid) * 16 * 4; }

// Wave w (0..3) fills table w (cos row part, sin row part, cos column part,
// sin column part) with DMA loads of 16 table rows each: lane i moves 16
// bytes, channels 4(i % 4) .. +3 of table row 16q + i / 4, to LDS byte
// 16i of the load's 1 KB. Rows past the grid read beyond the source table's
// bounds, which the buffer descriptor turns into zeros, or other patches'
// angles (grids under 16), and are never read back.
__device__ __forceinline__ void rope_table_dma(const float* cos, const float* sin, int grid, float* lds, int tid) {
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int rows = rope_table_rows(grid);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(wave & 1 ? sin : cos), 0, grid * grid * kHeadDim * 4, kBufferRsrcWord3);
    float* const table = lds + wave * rows * 16;
    for (int q = 0; q < rows / 16; ++q) {  // uniform, 1..4
        const int row = q * 16 + (lane >> 2);
        const int src = (wave < 2 ? row * grid * kHeadDim : row * kHeadDim + 16) + (lane & 3) * 4;  // floats
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(table + q * 256), 16,
                                                 src * 4, 0, 0, 0);
    }
}

// QKV + bias + 2D RoPE. A wave's 64 or 128 columns are one or two heads of
// q, k or v (a tile never straddles two of them); channel c and its rotation
// partner c+32 of a head are acc.v[2h] / acc.v[2h+1] of the same lane, and
// both use angle column c of the RoPE tables (DINOv3's tables repeat columns
// 0..31 in 32..63; only the first half is read, from the LDS tables of
// rope_table_dma). Results are rounded to f16 and regrouped in registers
// (frag_swap) so each lane holds 8 consecutive channels of its row. q, k
// and v are [image][head] matrices of tpad rows x 64 channels, each in
// fragment order: a lane's 8 channels are one 16-byte piece of a fragment,
// so the 64 lanes of a store cover one or two runs of whole rows' pieces per
// half-fragment (a row-major head row would take 32 separate 32-byte writes
// per store instead). Launched with rope_lds_bytes(grid) of dynamic LDS.
template <class T, bool LN>
__global__ __launch_bounds__(T::THREADS, T::FM == 1 ? (T::BK == 32 ? 4 : 3) : 2) void qkv_rope_kernel(QkvArgs p) {
    static_assert(T::TN % kHeadDim == 0 && kHidden % T::BN == 0 && T::WGN == 1,
                  "whole heads per wave and tile, whole rows per wave");
    static_assert(T::WAVES == 4, "four waves fill the four RoPE tables");
    __shared__ __attribute__((aligned(16))) half_t wb0[T::WF_HALFS], wb1[T::WF_HALFS], wb2[T::WF_HALFS];
    __shared__ __attribute__((aligned(16))) float cst[2][T::BN];  // bias, wsum of the tile's columns
    __shared__ float2_t rows_norm[T::BM];                          // (mean, rstd) of the tile's rows
    extern __shared__ __attribute__((aligned(16))) float rope_lds[];  // rope_table_dma's four tables
    static_assert(T::BN <= T::THREADS, "one thread per column constant");
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * Tok;
    constexpr int NT = 3 * kHidden / T::BN;
    const int tid = threadIdx.x;
    ActFrags<T> al[2];
    init_frags(al, p.h, M, kHidden);
    WeightDma<T> wd(p.w, 3 * kHidden, kHidden);
    // The epilogue's own operands are loaded ahead of the K loop: the RoPE
    // tables (DMA, first: they are the oldest loads every later wait covers),
    // the tile's column constants and its rows' LayerNorm (mean, rstd), all
    // of which wait in LDS.
    float4_t raw[T::FM][3];
    float cb = 0.f, cw = 0.f;
    gemm_tile_dma<T, 1, kHidden / T::BK>(
        al, wd, wb0, wb1, wb2, NT, NT * ((M + T::BM - 1) / T::BM), kHidden / T::BK,
        [&](int m0, int n0) {
            rope_table_dma(p.cos, p.sin, p.grid, rope_lds, tid);
            const Frag<T> f(m0, n0);
            if constexpr (LN) {
#pragma unroll
                for (int j = 0; j < T::FM; ++j) {
                    const float4_t* sp = (const float4_t*)(p.stats + (size_t)min(f.row(j), M - 1) * kStatFloats);
                    raw[j][0] = sp[0];
                    raw[j][1] = sp[1];
                    raw[j][2] = sp[2];
                }
            }
            if (tid < T::BN) {
                cb = p.bias[n0 + tid];
                if constexpr (LN) cw = p.wsum[n0 + tid];
            }
        },
        [&] {
            if (tid < T::BN) {
                cst[0][tid] = cb;
                cst[1][tid] = cw;
            }
            if constexpr (LN) {
                const int lane = tid & 63, r0 = (tid >> 6) % T::WGM * T::TM;
#pragma unroll
                for (int j = 0; j < T::FM; ++j) {
                    const RowNorm rn = row_norm(raw[j][0], raw[j][1], raw[j][2]);
                    if (lane < 32) rows_norm[r0 + j * 32 + lane] = float2_t{rn.mean, rn.rstd};
                }
            }
        },
        [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int part = f.n_base / kHidden, head0 = (f.n_base % kHidden) / kHeadDim;
        half_t* const out = part == 0 ? p.q : part == 1 ? p.k : p.v;
        const size_t head_elems = (size_t)p.tpad * kHeadDim;
        const int rows16 = rope_table_rows(p.grid);
        // The tile's rows lie in images img0 .. img0 + BM / Tok + 1 (img0
        // from the tile origin, so it is uniform); the descriptor covers
        // those.
        const int img0 = min(m0, M - 1) / Tok;
        const int span = min(p.images - img0, T::BM / Tok + 2);
        const WtOut wo(out + (size_t)img0 * kHeads * head_elems, (uint32_t)(span * kHeads * head_elems * 2));
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int mr = f.row(j);
            const int m = min(mr, M - 1);  // rows past M are computed but never written out
            const int img = m / Tok, tok = m - img * Tok;
            // This row's angles (cos, sin of channels 8g + 4hi .. +3, g =
            // 0..3); v tiles and prefix rows rotate by cos 1, sin 0.
            const bool rot = part < 2 && tok >= kPrefix;
            const int pt = max(tok - kPrefix, 0), gy = pt / p.grid, gx = pt - gy * p.grid;
            float4_t co[4], si[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int at = (g < 2 ? gy * 16 : 2 * rows16 * 16 + gx * 16) + (g & 1) * 8 + f.hi * 4;
                const float4_t c4 = *(const float4_t*)&rope_lds[at], s4 = *(const float4_t*)&rope_lds[at + rows16 * 16];
                co[g] = rot ? c4 : float4_t{1.f, 1.f, 1.f, 1.f};
                si[g] = rot ? s4 : float4_t{};
            }
            RowNorm rn{0.f, 1.f};
            if constexpr (LN) {
                const float2_t v = rows_norm[f.m_base - m0 + j * 32 + f.l32];
                rn = RowNorm{v[0], v[1]};
            }
#pragma unroll
            for (int h2 = 0; h2 < T::TN / kHeadDim; ++h2) {
                half4_t lo_h[4], up_h[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = g * 8 + f.hi * 4;  // channel in the head (0..31); partner c + 32
                    const int nl = f.n_base - n0 + h2 * kHeadDim + c;  // column in the tile
                    float4_t lo = group4(acc.v[2 * h2][j], g), up = group4(acc.v[2 * h2 + 1][j], g);
                    if constexpr (LN) {
                        lo = (lo - rn.mean * *(const float4_t*)&cst[1][nl]) * rn.rstd;
                        up = (up - rn.mean * *(const float4_t*)&cst[1][nl + 32]) * rn.rstd;
                    }
                    lo += *(const float4_t*)&cst[0][nl];
                    up += *(const float4_t*)&cst[0][nl + 32];
                    lo_h[g] = to_half4(lo * co[g] - up * si[g]);  // x[c] cos - x[c+32] sin
                    up_h[g] = to_half4(up * co[g] + lo * si[g]);  // x[c+32] cos + x[c] sin
                }
                // Channels 16kk + 8hi .. +7 of the head for kk = 0..3.
                const half8_t c0 = frag_swap(lo_h[0], lo_h[1]), c1 = frag_swap(lo_h[2], lo_h[3]);
                const half8_t c2 = frag_swap(up_h[0], up_h[1]), c3 = frag_swap(up_h[2], up_h[3]);
                const uint32_t hm = (uint32_t)(((img - img0) * kHeads + head0 + h2) * head_elems) * 2;
                if (mr < M) {
                    wo.store(hm + (uint32_t)frag_piece(tok, f.hi * 8, kHeadDim) * 2, c0);
                    wo.store(hm + (uint32_t)frag_piece(tok, 16 + f.hi * 8, kHeadDim) * 2, c1);
                    wo.store(hm + (uint32_t)frag_piece(tok, 32 + f.hi * 8, kHeadDim) * 2, c2);
                    wo.store(hm + (uint32_t)frag_piece(tok, 48 + f.hi * 8, kHeadDim) * 2, c3);
                }
            }
        }
    });
}

// Residual GEMM: x += ls * (A W^T + b), in place on the f16 residual stream
// in fragment order (with STATS, also the LayerNorm row statistics of the
// updated x). The epilogue turns each 16-column half of an MFMA result into a
// fragment in registers (frag_swap) and reads and writes x fragment by
// fragment (1 KB contiguous per wave access); LDS holds only the weight
// stages and the column constants.
template <class T, bool STATS, int KT = 0>
__global__ __launch_bounds__(T::THREADS, T::BK == 128 ? 3 : 4) void resid_kernel(ResidArgs p) {
    static_assert(T::TN % 64 == 0 && T::TM == 32, "whole statistics slots, one 32-row block per wave");
    static_assert(T::BN <= T::THREADS, "one thread per column constant");
    constexpr int XF = T::TN / 16;  // x fragments per wave
    __shared__ __attribute__((aligned(16))) half_t wb0[T::WF_HALFS], wb1[T::WF_HALFS], wb2[T::WF_HALFS];
    __shared__ __attribute__((aligned(16))) float cst[2][T::BN];  // bias * ls, ls of the tile's columns
    constexpr int NT = kHidden / T::BN;
    const int tid = threadIdx.x, lane = tid & 63, mblocks = (p.rows + 31) / 32;
    ActFrags<T> al[2];
    init_frags(al, p.a, p.rows, p.k);
    WeightDma<T> wd(p.w, kHidden, p.k);
    // The epilogue's own operands are loaded ahead of the K loop: the old x
    // fragments of the wave's 32 x TN block (each x element belongs to one
    // tile, so nothing else writes them meanwhile) and the column constants
    // (into LDS).
    half8_t xold[XF];
    float cb = 0.f, cl = 0.f;
    auto x_frag = [&](int m0, int n0, int i) {
        const Frag<T> f(m0, n0);
        const int mb = min(f.m_base / 32, mblocks - 1);  // a wave past the rows re-reads the last block
        return p.x + ((size_t)mb * (kHidden / 16) + f.n_base / 16 + i) * 512 + lane * 8;
    };
    gemm_tile_dma<T, 1, KT>(
        al, wd, wb0, wb1, wb2, NT, NT * ((p.rows + T::BM - 1) / T::BM), p.k / T::BK,
        [&](int m0, int n0) {
#pragma unroll
            for (int i = 0; i < XF; ++i) xold[i] = *(const half8_t*)x_frag(m0, n0, i);
            if (tid < T::BN) {
                cb = p.bias[n0 + tid];
                cl = p.ls[n0 + tid];
            }
        },
        [&] {
            if (tid < T::BN) {
                cst[0][tid] = cb * cl;  // ls * (acc + b) = acc * ls + b * ls: one FMA per output
                cst[1][tid] = cl;
            }
        },
        [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        if (f.m_base / 32 >= mblocks) return;  // uniform per wave
        const int m = f.m_base + f.l32;
        const bool valid = m < p.rows;
#pragma unroll
        for (int s2 = 0; s2 < T::TN / 64; ++s2) {
            float v[32];
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
                const int i = 2 * s2 + i2;  // 32-column MFMA tile of the wave
                float4_t u[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int nt = f.col(i, g) - n0;  // column in the tile
                    const float4_t bl = *(const float4_t*)&cst[0][nt], l = *(const float4_t*)&cst[1][nt];
                    u[g] = group4(acc.v[i][0], g) * l + bl;
                }
                frag_swap(u[0], u[1]);
                frag_swap(u[2], u[3]);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const half8_t old = xold[2 * i + kk];
                    half8_t h;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        h[e] = (half_t)((float)old[e] + u[2 * kk][e]);
                        h[e + 4] = (half_t)((float)old[e + 4] + u[2 * kk + 1][e]);
                    }
                    if (valid) *(half8_t*)x_frag(m0, n0, 2 * i + kk) = h;
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[(i2 * 2 + kk) * 8 + e] = (float)h[e];
                }
            }
            if constexpr (STATS) pair_stats(p.stats, m, f.n_base / 64 + s2, v, f.hi, valid);
        }
    });
}

// SwiGLU dual GEMM. W rows are packed as blocks of 32 gate rows followed by
// the 32 matching up rows, so a wave's 128 columns are two gate/up pairs of
// 32 outputs each. The tile's column constants (bias, and wsum with the
// folded LayerNorm) and its rows' statistics are loaded before the K loop;
// the constants wait in LDS. The epilogue turns each 16-column half of a
// 32-column act block into a fragment in registers (frag_swap) and writes
// it whole (act is in fragment order).
// NS: N slices of the XCD tile split (xcd_tile_split); the launcher picks
// it by the launch's size.
template <class T, bool LN, int NS>
__global__ __launch_bounds__(T::THREADS, T::FM == 1 ? 3 : 2) void swiglu_kernel(SwigluArgs p) {
    static_assert(T::TN % 64 == 0 && T::WGN == 1, "whole gate/up pairs, whole rows per wave");
    static_assert(T::BN <= T::THREADS, "one thread per column constant");
    static_assert(kHidden / T::BK > T::FN, "a K-loop step for every column block's LayerNorm mean term");
    __shared__ __attribute__((aligned(16))) half_t wb0[T::WF_HALFS], wb1[T::WF_HALFS], wb2[T::WF_HALFS];
    __shared__ __attribute__((aligned(16))) float cst[2][T::BN];  // bias, wsum
    constexpr int NT = 2 * kFF / T::BN;
    const int tid = threadIdx.x;
    ActFrags<T> al[2];
    init_frags(al, p.h, p.rows, kHidden);
    WeightDma<T> wd(p.w, 2 * kFF, kHidden);
    float4_t raw[T::FM][3];
    RowNorm rn[T::FM];
    float cb = 0.f, cw = 0.f;
    gemm_tile_dma<T, NS, kHidden / T::BK>(
        al, wd, wb0, wb1, wb2, NT, NT * ((p.rows + T::BM - 1) / T::BM), kHidden / T::BK,
        [&](int m0, int n0) {
            const Frag<T> f(m0, n0);
            if constexpr (LN) {
#pragma unroll
                for (int j = 0; j < T::FM; ++j) {
                    const float4_t* sp = (const float4_t*)(p.stats + (size_t)min(f.row(j), p.rows - 1) * kStatFloats);
                    raw[j][0] = sp[0];
                    raw[j][1] = sp[1];
                    raw[j][2] = sp[2];
                }
            }
            if (tid < T::BN) {
                cb = p.bias[n0 + tid];
                if constexpr (LN) cw = p.wsum[n0 + tid];
            }
        },
        [&] {
            if (tid < T::BN) {
                // Gate columns (the first 32 of each 64) are kept scaled by
                // -log2(e), up columns by -ln(2); see the epilogue.
                cst[0][tid] = cb * (tid % 64 < 32 ? -kLog2e : -kLn2);
                cst[1][tid] = cw;
            }
#pragma unroll
            for (int j = 0; j < T::FM; ++j) rn[j] = LN ? row_norm(raw[j][0], raw[j][1], raw[j][2]) : RowNorm{0.f, 1.f};
        },
        [&](const Acc<T>& acc, int m0, int n0) {
        const Frag<T> f(m0, n0);
        const int lane = threadIdx.x & 63, mblocks = (p.rows + 31) / 32;
        // Pair q of the wave: gate = acc.v[2q], up = acc.v[2q + 1], outputs
        // 32q .. 32q+31 of the wave's OW, i.e. act fragments 2q and 2q + 1.
        // With gate g and up u (after LayerNorm folding and bias), the output
        // silu(g) u = g u / (1 + e^-g) is computed from gs = -g log2(e) and
        // us = -u ln(2) as gs us / (1 + 2^gs) (gs us = g u): the scales ride
        // on the FMAs that apply rstd and the bias, which saves the multiply
        // that would otherwise form the exponent.
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int mb = f.m_base / 32 + j;
            if (mb >= mblocks) break;  // uniform per wave
            const float sg = rn[j].rstd * -kLog2e, su = rn[j].rstd * -kLn2;
            const WtOut act(p.act + (size_t)mb * (kFF / 16) * 512, 32 * kFF * 2);
#pragma unroll
            for (int q = 0; q < T::FN / 2; ++q) {
                half4_t y[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = g * 8 + f.hi * 4, nl = f.n_base - n0 + 64 * q + c;
                    float4_t gate = group4(acc.v[2 * q][j], g), up = group4(acc.v[2 * q + 1][j], g);
                    const float4_t gs = gate * sg + *(const float4_t*)&cst[0][nl];
                    const float4_t us = up * su + *(const float4_t*)&cst[0][nl + 32];
                    float4_t r;
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[e] = gs[e] * us[e] * fast_rcp(1.0f + fast_exp2(gs[e]));
                    y[g] = to_half4(r);
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    act.store(((f.n_base / 32 + 2 * q + kk) * 512 + lane * 8) * 2, frag_swap(y[2 * kk], y[2 * kk + 1]));
            }
        }
    },
    // The folded LayerNorm's -mean * wsum, added to column block i of the
    // accumulators at step i + 1 of the K loop (an additive term may join
    // the sum at any point), where its FMAs issue beside the MFMAs instead
    // of lengthening the epilogue.
    [&](Acc<T>& acc, int s) {
        if constexpr (LN) {
            static_for<T::FN>([&](auto I) {
                constexpr int i = decltype(I)::value;
                if (s == i + 1) {
                    const int hi = (threadIdx.x & 63) >> 5;
                    float4_t w[4];
#pragma unroll
                    for (int g = 0; g < 4; ++g) w[g] = *(const float4_t*)&cst[1][32 * i + 8 * g + 4 * hi];
#pragma unroll
                    for (int j = 0; j < T::FM; ++j)
#pragma unroll
                        for (int g = 0; g < 4; ++g)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                acc.v[i][j][4 * g + e] = fmaf(-rn[j].mean, w[g][e], acc.v[i][j][4 * g + e]);
                }
            });
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
struct SplitActFrags : ActFrags<T> {
    SplitDecode<T> d;
    __device__ __forceinline__ void load(int m0, int n0, int kt, int tid) {
        this->ks_off = d.split(m0) * (d.kc / 16);
        ActFrags<T>::load(d.row0(m0), n0, kt, tid);
    }
};

template <class T, int KT = 0>
__global__ __launch_bounds__(T::THREADS, 3) void splitk_kernel(SplitKArgs p) {
    __shared__ __attribute__((aligned(16))) half_t wb0[T::WF_HALFS], wb1[T::WF_HALFS], wb2[T::WF_HALFS];
    constexpr int NT = kHidden / T::BN;
    const int MT = (p.rows + T::BM - 1) / T::BM;
    const SplitDecode<T> d{MT, p.k / p.splits};
    ActFrags<T> base[2];
    init_frags(base, p.a, p.rows, p.k);
    SplitActFrags<T> al[2] = {{base[0], d}, {base[1], d}};
    WeightDma<T> wd(p.w, kHidden, p.k);
    gemm_tile_dma<T, 1, KT>(
        al, wd, wb0, wb1, wb2, NT, NT * MT * p.splits, d.kc / T::BK,
        [&](int m0, int) { wd.ks_off = d.split(m0) * (d.kc / 16); }, [] {},
        [&](const Acc<T>& acc, int m0, int n0) {
            const Frag<T> f(d.row0(m0), n0);
            float* slab = p.partials + (size_t)d.split(m0) * p.rows * kHidden;
            const int m = f.row(0);
            if (m >= p.rows) return;
#pragma unroll
            for (int i = 0; i < T::FN; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *(float4_t*)(slab + (size_t)m * kHidden + f.col(i, g)) = group4(acc.v[i][0], g);
        });
}

}  // namespace gemm
}  // namespace dhx
