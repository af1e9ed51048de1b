// f16 MFMA GEMM family for gfx950: C[m][n] = sum_k A[m][k] * W[n][k] with
// fp32 accumulation and fused epilogues. Replaces the reference's Loom GEMMs
// (kernels/matmul_bias_f16_wmma.loom, matmul_qkv_rope_f16_wmma.loom,
// matmul_resid_f16_wmma.loom, matmul_swiglu_f16_wmma.loom,
// matmul_splitk_f16_wmma.loom) and the embed scatter
// (kernels/embed_scatter_f32.loom), which is fused into the patch epilogue.
//
// Structure (all variants): 256 threads = 4 waves; a workgroup owns a BM x BN
// output tile; the K loop walks 64-wide stages through two LDS buffers
// (global loads for stage s+1 are in flight while stage s feeds the MFMAs;
// one barrier per stage). Each wave owns a TM x TN sub-tile made of 32x32
// v_mfma_f32_32x32x16_f16 tiles. The MFMA's first operand is the weight row
// (n) and its second the activation row (m), so every lane ends up holding 4
// consecutive output columns of one row: epilogues write 8- or 16-byte
// vectors, and the RoPE partner channel c+32 / the SwiGLU up value sits in
// the same lane as channel c / the gate value.
#include "launch.hpp"

namespace dhx {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int LDK = BK + 8;  // LDS row pitch in halfs (144 B): 16-byte fragment reads are conflict-free

template <int BM_, int BN_, int WGM_, int WGN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
    static_assert(WGM * WGN == 4, "four waves per workgroup");
    static constexpr int TM = BM / WGM, TN = BN / WGN;
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile is a multiple of the 32x32 MFMA tile");
    static constexpr int FM = TM / 32, FN = TN / 32;
    static constexpr int LDS_HALFS = 2 * (BM + BN) * LDK;
};

__device__ __forceinline__ half8_t zero8() {
    half8_t z = {};
    return z;
}

// A operand: f16 row-major rows m0 .. m0+BM-1 of an [M][lda] matrix starting
// at column k_off; rows past M load as zero.
template <class T>
struct HalfRows {
    static constexpr int CHUNKS = T::BM * BK / 8 / kThreads;
    static_assert(T::BM * BK / 8 % kThreads == 0, "A tile splits evenly");
    const half_t* a;
    int lda, m0, M, k_off;
    half8_t r[CHUNKS];
    __device__ __forceinline__ void load(int kt, int tid) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            const int m = m0 + row;
            r[i] = m < M ? *(const half8_t*)(a + (size_t)m * lda + k_off + kt * BK + col) : zero8();
        }
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            *(half8_t*)(s + row * LDK + col) = r[i];
        }
    }
};

// Weight operand: rows n0 .. n0+BN-1 of W[N][ldw] (always in range: the
// launchers only use N that are multiples of BN).
template <class T>
struct WeightRows {
    static constexpr int CHUNKS = T::BN * BK / 8 / kThreads;
    static_assert(T::BN * BK / 8 % kThreads == 0, "W tile splits evenly");
    const half_t* w;
    int ldw, n0, k_off;
    half8_t r[CHUNKS];
    __device__ __forceinline__ void load(int kt, int tid) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            r[i] = *(const half8_t*)(w + (size_t)(n0 + row) * ldw + k_off + kt * BK + col);
        }
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            *(half8_t*)(s + row * LDK + col) = r[i];
        }
    }
};

// A operand of the patch embedding, gathered from NCHW f32 pixels (im2col of
// lib.rs:265-280): row m = image*P + gy*G + gx, column k = c*256 + dy*16 + dx.
// A 64-wide stage covers one channel and four pixel rows dy of the patch;
// consecutive lanes read consecutive 16-byte pieces of a pixel row, and
// neighbouring patches of one grid row are adjacent in memory.
template <class T>
struct PatchRows {
    static constexpr int CHUNKS = T::BM * BK / 4 / kThreads;
    static_assert(T::BM * BK / 4 % kThreads == 0, "patch tile splits evenly");
    const float* px;
    int m0, M, G, P, S;
    float4_t r[CHUNKS];
    __device__ __forceinline__ void load(int kt, int tid) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads;
            const int dxq = c & 3, row = (c >> 2) % T::BM, dyl = c / (4 * T::BM);
            const int m = m0 + row;
            if (m < M) {
                const int img = m / P, p = m - img * P, gy = p / G, gx = p - gy * G;
                const int ch = kt >> 2, dy = (kt & 3) * 4 + dyl;
                r[i] = *(const float4_t*)(px + (((size_t)img * 3 + ch) * S + gy * 16 + dy) * S + gx * 16 + dxq * 4);
            } else {
                r[i] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + i * kThreads;
            const int dxq = c & 3, row = (c >> 2) % T::BM, dyl = c / (4 * T::BM);
            half4_t h = {(half_t)r[i][0], (half_t)r[i][1], (half_t)r[i][2], (half_t)r[i][3]};
            *(half4_t*)(s + row * LDK + dyl * 16 + dxq * 4) = h;
        }
    }
};

// The shared main loop. acc[i][j] is the 32x32 tile of weight rows
// wn*TN + 32i .. and activation rows wm*TM + 32j ..; lane l holds activation
// row (l % 32) and weight rows 8*(r/4) + 4*(l/32) + r%4.
template <class T, class AL, class WL>
__device__ __forceinline__ void gemm_main(AL& al, WL& wl, int k_tiles, half_t* lds,
                                          float16_t (&acc)[T::FN][T::FM]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % T::WGM, wn = wave / T::WGM;
    const int l32 = lane & 31, hi = lane >> 5;
    half_t* const sA0 = lds;
    half_t* const sW0 = lds + T::BM * LDK;
    constexpr int kStage = (T::BM + T::BN) * LDK;
#pragma unroll
    for (int i = 0; i < T::FN; ++i)
#pragma unroll
        for (int j = 0; j < T::FM; ++j) acc[i][j] = float16_t{};

    al.load(0, tid);
    wl.load(0, tid);
    al.store(sA0, tid);
    wl.store(sW0, tid);
    __syncthreads();
    for (int kt = 0; kt < k_tiles; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < k_tiles;
        if (more) {
            al.load(kt + 1, tid);
            wl.load(kt + 1, tid);
        }
        const half_t* a_s = sA0 + buf * kStage + (wm * T::TM + l32) * LDK + hi * 8;
        const half_t* w_s = sW0 + buf * kStage + (wn * T::TN + l32) * LDK + hi * 8;
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            half8_t wf[T::FN], af[T::FM];
#pragma unroll
            for (int i = 0; i < T::FN; ++i) wf[i] = *(const half8_t*)(w_s + i * 32 * LDK + kk * 16);
#pragma unroll
            for (int j = 0; j < T::FM; ++j) af[j] = *(const half8_t*)(a_s + j * 32 * LDK + kk * 16);
#pragma unroll
            for (int i = 0; i < T::FN; ++i)
#pragma unroll
                for (int j = 0; j < T::FM; ++j) acc[i][j] = mfma32x32x16(wf[i], af[j], acc[i][j]);
        }
        if (more) {
            al.store(sA0 + (buf ^ 1) * kStage, tid);
            wl.store(sW0 + (buf ^ 1) * kStage, tid);
        }
        __syncthreads();
    }
}

__device__ __forceinline__ float4_t group4(const float16_t& a, int g) {
    return float4_t{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
}

__device__ __forceinline__ half4_t to_half4(float4_t v) {
    return half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

__device__ __forceinline__ float4_t ld4(const float* p) { return *(const float4_t*)p; }

// ---------------------------------------------------------------------------
// Patch embedding + CLS/register scatter (reference kernels 0 and 1).
using PatchTile = Tile<64, 128, 2, 2>;

__global__ __launch_bounds__(kThreads) void patch_embed_kernel(PatchEmbedArgs p) {
    using T = PatchTile;
    __shared__ half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * P;
    constexpr int NT = kHidden / T::BN;
    const int MT = (M + T::BM - 1) / T::BM;
    const int t = xcd_remap(blockIdx.x, NT * MT);
    const int n0 = (t % NT) * T::BN, m0 = (t / NT) * T::BM;

    PatchRows<T> al{p.pixels, m0, M, p.grid, P, 16 * p.grid};
    WeightRows<T> wl{p.w, 768, n0, 0};
    float16_t acc[T::FN][T::FM];
    gemm_main<T>(al, wl, 768 / BK, lds, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int m_base = m0 + (wave % T::WGM) * T::TM, n_base = n0 + (wave / T::WGM) * T::TN;
#pragma unroll
    for (int j = 0; j < T::FM; ++j) {
        const int m = m_base + j * 32 + l32;
        if (m >= M) continue;
        const int img = m / P, patch = m - img * P;
        half_t* dst = p.x + ((size_t)img * Tok + kPrefix + patch) * kHidden;
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n_base + i * 32 + g * 8 + hi * 4;
                *(half4_t*)(dst + n) = to_half4(group4(acc[i][j], g) + ld4(p.bias + n));
            }
    }
    // CLS + registers of every image whose first patch row lies in this tile.
    const int m_end = min(m0 + T::BM, M);
    for (int img = (m0 + P - 1) / P; img * P < m_end; ++img)
        for (int idx = threadIdx.x; idx < kPrefix * T::BN; idx += kThreads) {
            const int row = idx / T::BN, col = n0 + idx % T::BN;
            p.x[((size_t)img * Tok + row) * kHidden + col] = (half_t)p.prefix[row * kHidden + col];
        }
}

// ---------------------------------------------------------------------------
// QKV + bias + 2D RoPE (reference kernel 4). A wave's 64 columns are exactly
// one head of q, k or v, so channel c and its rotation partner c+32 are the
// acc[0] / acc[1] entries of the same lane.
using QkvTile = Tile<128, 128, 2, 2>;
static_assert(QkvTile::TN == kHeadDim, "one head per wave");

__global__ __launch_bounds__(kThreads) void qkv_rope_kernel(QkvArgs p) {
    using T = QkvTile;
    __shared__ half_t lds[T::LDS_HALFS];
    const int P = p.grid * p.grid, Tok = P + kPrefix, M = p.images * Tok;
    constexpr int NT = 3 * kHidden / T::BN;
    const int MT = (M + T::BM - 1) / T::BM;
    const int t = xcd_remap(blockIdx.x, NT * MT);
    const int n0 = (t % NT) * T::BN, m0 = (t / NT) * T::BM;

    HalfRows<T> al{p.h, kHidden, m0, M, 0};
    WeightRows<T> wl{p.w, kHidden, n0, 0};
    float16_t acc[T::FN][T::FM];
    gemm_main<T>(al, wl, kHidden / BK, lds, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int m_base = m0 + (wave % T::WGM) * T::TM, n_base = n0 + (wave / T::WGM) * T::TN;
    const int part = n_base / kHidden, head = (n_base % kHidden) / kHeadDim;
#pragma unroll
    for (int j = 0; j < T::FM; ++j) {
        const int m = m_base + j * 32 + l32;
        if (m >= M) continue;
        const int img = m / Tok, tok = m - img * Tok;
        const size_t bh = (size_t)img * kHeads + head;
        const bool rotate = part < 2 && tok >= kPrefix;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = g * 8 + hi * 4;  // channel in the head, 0..31; partner c + 32
            float4_t lo = group4(acc[0][j], g) + ld4(p.bias + n_base + c);
            float4_t up = group4(acc[1][j], g) + ld4(p.bias + n_base + 32 + c);
            if (rotate) {
                const int pos = tok - kPrefix;
                const float4_t cl = ld4(p.cos + pos * 64 + c), sl = ld4(p.sin + pos * 64 + c);
                const float4_t ch = ld4(p.cos + pos * 64 + 32 + c), sh = ld4(p.sin + pos * 64 + 32 + c);
                const float4_t nlo = lo * cl - up * sl;  // x[c]cos - x[c+32]sin
                const float4_t nup = up * ch + lo * sh;  // x[c+32]cos + x[c]sin
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
}

// ---------------------------------------------------------------------------
// Residual GEMM: x += ls * (A W^T + b) (reference kernels 6 and 7).
using ResidTile = Tile<64, 128, 2, 2>;

__global__ __launch_bounds__(kThreads) void resid_kernel(ResidArgs p) {
    using T = ResidTile;
    __shared__ half_t lds[T::LDS_HALFS];
    constexpr int NT = kHidden / T::BN;
    const int MT = (p.rows + T::BM - 1) / T::BM;
    const int t = xcd_remap(blockIdx.x, NT * MT);
    const int n0 = (t % NT) * T::BN, m0 = (t / NT) * T::BM;

    HalfRows<T> al{p.a, p.k, m0, p.rows, 0};
    WeightRows<T> wl{p.w, p.k, n0, 0};
    float16_t acc[T::FN][T::FM];
    gemm_main<T>(al, wl, p.k / BK, lds, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int m_base = m0 + (wave % T::WGM) * T::TM, n_base = n0 + (wave / T::WGM) * T::TN;
#pragma unroll
    for (int j = 0; j < T::FM; ++j) {
        const int m = m_base + j * 32 + l32;
        if (m >= p.rows) continue;
        half_t* xr = p.x + (size_t)m * kHidden;
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n_base + i * 32 + g * 8 + hi * 4;
                const half4_t old = *(const half4_t*)(xr + n);
                const float4_t upd = (group4(acc[i][j], g) + ld4(p.bias + n)) * ld4(p.ls + n);
                const float4_t xo = float4_t{(float)old[0], (float)old[1], (float)old[2], (float)old[3]};
                *(half4_t*)(xr + n) = to_half4(xo + upd);
            }
    }
}

// ---------------------------------------------------------------------------
// SwiGLU dual GEMM (reference kernel 8). W rows are packed as blocks of 32
// gate rows followed by the 32 matching up rows, so a wave's 64 columns are
// 32 gate / 32 up columns of the same 32 outputs.
using SwigluTile = Tile<128, 128, 2, 2>;
static_assert(SwigluTile::TN == 64, "gate/up pair per wave");

__global__ __launch_bounds__(kThreads) void swiglu_kernel(SwigluArgs p) {
    using T = SwigluTile;
    __shared__ half_t lds[T::LDS_HALFS];
    constexpr int NT = 2 * kFF / T::BN;
    const int MT = (p.rows + T::BM - 1) / T::BM;
    const int t = xcd_remap(blockIdx.x, NT * MT);
    const int n0 = (t % NT) * T::BN, m0 = (t / NT) * T::BM;

    HalfRows<T> al{p.h, kHidden, m0, p.rows, 0};
    WeightRows<T> wl{p.w, kHidden, n0, 0};
    float16_t acc[T::FN][T::FM];
    gemm_main<T>(al, wl, kHidden / BK, lds, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int m_base = m0 + (wave % T::WGM) * T::TM, n_base = n0 + (wave / T::WGM) * T::TN;
    const int out_base = n_base / 2;
#pragma unroll
    for (int j = 0; j < T::FM; ++j) {
        const int m = m_base + j * 32 + l32;
        if (m >= p.rows) continue;
        half_t* dst = p.act + (size_t)m * kFF + out_base;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = g * 8 + hi * 4;
            const float4_t gate = group4(acc[0][j], g) + ld4(p.bias + n_base + c);
            const float4_t up = group4(acc[1][j], g) + ld4(p.bias + n_base + 32 + c);
            const float4_t y = float4_t{silu(gate[0]), silu(gate[1]), silu(gate[2]), silu(gate[3])} * up;
            *(half4_t*)(dst + c) = to_half4(y);
        }
    }
}

// ---------------------------------------------------------------------------
// Split-K GEMM into f32 slabs (reference kernel 9); no atomics, so the
// result does not depend on scheduling.
using SplitTile = Tile<64, 128, 2, 2>;

__global__ __launch_bounds__(kThreads) void splitk_kernel(SplitKArgs p) {
    using T = SplitTile;
    __shared__ half_t lds[T::LDS_HALFS];
    constexpr int NT = kHidden / T::BN;
    const int MT = (p.rows + T::BM - 1) / T::BM;
    const int tiles = NT * MT;
    const int t = xcd_remap(blockIdx.x, tiles * p.splits);
    const int split = t / tiles, tt = t - split * tiles;
    const int n0 = (tt % NT) * T::BN, m0 = (tt / NT) * T::BM;
    const int kc = p.k / p.splits;

    HalfRows<T> al{p.a, p.k, m0, p.rows, split * kc};
    WeightRows<T> wl{p.w, p.k, n0, split * kc};
    float16_t acc[T::FN][T::FM];
    gemm_main<T>(al, wl, kc / BK, lds, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int m_base = m0 + (wave % T::WGM) * T::TM, n_base = n0 + (wave / T::WGM) * T::TN;
    float* slab = p.partials + (size_t)split * p.rows * kHidden;
#pragma unroll
    for (int j = 0; j < T::FM; ++j) {
        const int m = m_base + j * 32 + l32;
        if (m >= p.rows) continue;
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n_base + i * 32 + g * 8 + hi * 4;
                *(float4_t*)(slab + (size_t)m * kHidden + n) = group4(acc[i][j], g);
            }
    }
}

template <class T>
int tiles_for(int rows, int n) {
    return (n / T::BN) * ((rows + T::BM - 1) / T::BM);
}

}  // namespace

hipError_t launch_patch_embed(const PatchEmbedArgs& a, hipStream_t s) {
    const int blocks = tiles_for<PatchTile>(a.images * a.grid * a.grid, kHidden);
    hipLaunchKernelGGL(patch_embed_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t s) {
    const int blocks = tiles_for<QkvTile>(a.images * (a.grid * a.grid + kPrefix), 3 * kHidden);
    hipLaunchKernelGGL(qkv_rope_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_resid(const ResidArgs& a, hipStream_t s) {
    const int blocks = tiles_for<ResidTile>(a.rows, kHidden);
    hipLaunchKernelGGL(resid_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t s) {
    const int blocks = tiles_for<SwigluTile>(a.rows, 2 * kFF);
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_splitk(const SplitKArgs& a, hipStream_t s) {
    const int blocks = tiles_for<SplitTile>(a.rows, kHidden) * a.splits;
    hipLaunchKernelGGL(splitk_kernel, dim3(blocks), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dhx
