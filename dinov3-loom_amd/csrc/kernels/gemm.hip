// Production tile shapes of the GEMM variants (kernels in gemm_kernels.hpp)
// and their launchers.
#include "gemm_kernels.hpp"

namespace dhx {
namespace {

using gemm::Tile;
using gemm::tiles_for;

// The patch embedding stages both operands in LDS (its A operand is gathered
// from pixels); the others take activations in fragment order straight into
// registers, waves stacked along M. The residual GEMMs (N = 384: too few
// 128x128 tiles to fill 256 CUs) use 128x64 tiles, twice as many workgroups
// of a quarter of the registers.
using PatchTile = Tile<64, 128, 2, 2>;
// QKV on 32-deep stages (24 KB of weight buffers; its RoPE angles wait in
// LDS, not registers): four workgroups per CU, so a batch of 64 (909 tiles)
// runs as one round of workgroups.
using QkvTile = Tile<128, 128, 4, 1, 32>;
// QKV for launches of fewer rows (batch 32's and 512x512 batch 8's image
// groups, small batches): 128x64 tiles (one head per wave), twice the
// workgroups. Same stage depth, and the LayerNorm fold is applied in the
// epilogue, so a row's result is bitwise the same on either shape.
using QkvTileS = Tile<128, 64, 4, 1, 32>;
constexpr int kQkvSmallRows = 5120;
using ResidTile = Tile<128, 64, 4, 1>;
using ResidTileK = Tile<128, 64, 4, 1, 128>;  // down projection (k = 1536)
using SwigluTile = Tile<256, 128, 4, 1, 64>;
// SwiGLU for launches of fewer rows (batch 32's and 512x512 batch 8's image
// groups of 3216 and 4116 rows, small batches): 128-row tiles, three
// workgroups per CU instead of two. Measured in the two-group forward: the
// 128-row tiles win at 3216 and 4116 rows (at 4116 the 256-row tiling's
// last tile holds 20 rows), the 256-row ones at 6432 (batch 64's groups).
using SwigluTileS = Tile<128, 128, 4, 1, 64>;
constexpr int kSwigluSmallRows = 5120;
// Launches of up to this many rows take four XCD N slices, larger ones two.
constexpr int kSwigluSplit4Rows = 8192;
// The folded LayerNorm's -mean * wsum term joins column block i's
// accumulators at K step i + 1, so where it enters the fp32 sum depends on
// the stage depth. Both tile shapes must share it for a row's result to be
// bitwise the same whichever shape its launch takes (the image groupings of
// the forward and the allocation-free entry point rely on that).
static_assert(SwigluTile::BK == SwigluTileS::BK, "one stage depth for every SwiGLU tile shape");
using SplitTile = Tile<128, 128, 4, 1>;

template <class T, class Args>
hipError_t launch(void (*kernel)(Args), int tiles, const Args& a, hipStream_t s) {
    hipLaunchKernelGGL(kernel, dim3(gemm::tile_grid(tiles)), dim3(T::THREADS), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_patch_embed(const PatchEmbedArgs& a, hipStream_t s) {
    const int tiles = tiles_for<PatchTile>(a.images * a.grid * a.grid, kHidden);
    return a.stats ? launch<PatchTile>(gemm::patch_embed_kernel<PatchTile, true>, tiles, a, s)
                   : launch<PatchTile>(gemm::patch_embed_kernel<PatchTile, false>, tiles, a, s);
}

template <class T>
static hipError_t launch_qkv_tiles(const QkvArgs& a, hipStream_t s) {
    const int tiles = tiles_for<T>(a.images * (a.grid * a.grid + kPrefix), 3 * kHidden);
    const dim3 grid(gemm::tile_grid(tiles));
    const size_t lds = gemm::rope_lds_bytes(a.grid);
    if (a.stats) hipLaunchKernelGGL((gemm::qkv_rope_kernel<T, true>), grid, dim3(T::THREADS), lds, s, a);
    else hipLaunchKernelGGL((gemm::qkv_rope_kernel<T, false>), grid, dim3(T::THREADS), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t s) {
    const int rows = a.images * (a.grid * a.grid + kPrefix);
    return rows < kQkvSmallRows ? launch_qkv_tiles<QkvTileS>(a, s) : launch_qkv_tiles<QkvTile>(a, s);
}

hipError_t launch_resid(const ResidArgs& a, hipStream_t s) {
    // The K loop walks its stages six at a time (gemm_main_dma).
    if (a.k % (6 * ResidTile::BK) != 0) return hipErrorInvalidValue;
    if (a.k == kHidden) {  // the o-projection: three 128-deep stages, unrolled
        const int tiles = tiles_for<ResidTileK>(a.rows, kHidden);
        return a.stats ? launch<ResidTileK>(gemm::resid_kernel<ResidTileK, true, kHidden / 128>, tiles, a, s)
                       : launch<ResidTileK>(gemm::resid_kernel<ResidTileK, false, kHidden / 128>, tiles, a, s);
    }
    if (a.k == kFF) {  // the down projection: twelve 128-deep stages, unrolled
        const int tiles = tiles_for<ResidTileK>(a.rows, kHidden);
        return a.stats ? launch<ResidTileK>(gemm::resid_kernel<ResidTileK, true, kFF / 128>, tiles, a, s)
                       : launch<ResidTileK>(gemm::resid_kernel<ResidTileK, false, kFF / 128>, tiles, a, s);
    }
    if (a.k % (6 * ResidTileK::BK) == 0) {
        const int tiles = tiles_for<ResidTileK>(a.rows, kHidden);
        return a.stats ? launch<ResidTileK>(gemm::resid_kernel<ResidTileK, true>, tiles, a, s)
                       : launch<ResidTileK>(gemm::resid_kernel<ResidTileK, false>, tiles, a, s);
    }
    const int tiles = tiles_for<ResidTile>(a.rows, kHidden);
    return a.stats ? launch<ResidTile>(gemm::resid_kernel<ResidTile, true>, tiles, a, s)
                   : launch<ResidTile>(gemm::resid_kernel<ResidTile, false>, tiles, a, s);
}

template <class T, int NS>
static hipError_t launch_swiglu_tiles(const SwigluArgs& a, hipStream_t s) {
    static_assert(kHidden % (6 * T::BK) == 0, "the K loop walks its stages six at a time");
    const int grid = gemm::tile_grid_split<NS>((a.rows + T::BM - 1) / T::BM, 2 * kFF / T::BN);
    if (a.stats) hipLaunchKernelGGL((gemm::swiglu_kernel<T, true, NS>), dim3(grid), dim3(T::THREADS), 0, s, a);
    else hipLaunchKernelGGL((gemm::swiglu_kernel<T, false, NS>), dim3(grid), dim3(T::THREADS), 0, s, a);
    return hipGetLastError();
}

// The XCD split (each XCD's L2 keeps 1/NS of the weights): two N slices for
// the whole batch-64 launch, four for the image groups of 5120 - 8191 rows
// that the forward runs concurrently (measured: forward +0.9 % at batch 64,
// the whole-batch launch 2 % slower with four).
hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t s) {
    if (a.rows < kSwigluSmallRows) return launch_swiglu_tiles<SwigluTileS, 2>(a, s);
    return a.rows < kSwigluSplit4Rows ? launch_swiglu_tiles<SwigluTile, 4>(a, s) : launch_swiglu_tiles<SwigluTile, 2>(a, s);
}

hipError_t launch_splitk(const SplitKArgs& a, hipStream_t s) {
    // Each split's K loop walks its stages six at a time (gemm_main_dma).
    if (a.splits < 1 || a.k % a.splits != 0 || (a.k / a.splits) % (6 * SplitTile::BK) != 0) return hipErrorInvalidValue;
    const int tiles = tiles_for<SplitTile>(a.rows, kHidden) * a.splits;
    if (a.k / a.splits == kHidden)  // the model's b = 1 down projection: 4 splits of 384, six stages unrolled
        return launch<SplitTile>(gemm::splitk_kernel<SplitTile, kHidden / SplitTile::BK>, tiles, a, s);
    return launch<SplitTile>(gemm::splitk_kernel<SplitTile>, tiles, a, s);
}

}  // namespace dhx
