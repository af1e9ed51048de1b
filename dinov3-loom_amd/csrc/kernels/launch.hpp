// Host-side launchers for the forward-pass kernels. Each launcher assumes the
// engine has already checked every binding's size against the shapes below
// (engine.cpp: required_bytes); they only derive grids and launch.
//
// The f16 activations x, h, attn and act are stored in fragment order
// (common.hpp: frag_piece), rows padded to a multiple of 32; "[rows][K] frag"
// below means that layout.
#pragma once
#include <hip/hip_runtime.h>
#include "common.hpp"

namespace dhx {

// Row LayerNorm over 384 channels, eps 1e-5, fp32 statistics.
// x [rows][384] frag -> out [rows][384] frag f16 (or row-major f32 when
// f32_out).
struct LayerNormArgs {
    const half_t* x;
    const float* gamma;
    const float* beta;
    void* out;
    int rows;
    int f32_out;
};

// Fused patch embedding: im2col of NCHW f32 pixels (patch order (gy, gx),
// k order (c, dy, dx)), GEMM with patch_w [384][768] f16, + bias, narrowed to
// f16 and scattered into x [images*T][384] frag after the CLS + 4 register
// rows, which are copied from prefix [5][384] f32.
struct PatchEmbedArgs {
    const float* pixels;
    const half_t* w;
    const float* bias;
    const float* prefix;
    half_t* x;
    int images;
    int grid;  // patches per side G; image side 16*G, T = G*G + 5
    // Optional (both or neither): row statistics of x for a fused LayerNorm
    // consumer; prefix_stats holds those of the 5 prefix rows [5][6][2].
    const float* prefix_stats = nullptr;
    float* stats = nullptr;
};

// Row statistics of the residual stream x for LayerNorm fused into the next
// GEMM: stats[row][slot][2] = (mean, M2) of the f16 values of x in columns
// 64*slot .. 64*slot+63, slot 0..5 (M2 = sum of squared deviations from that
// slot's mean). A consumer combines the six slots (Chan et al.'s pairwise
// update) into the row mean and variance.
constexpr int kStatSlots = kHidden / 64;
constexpr int kStatFloats = 2 * kStatSlots;

// h [rows][384] frag . Wqkv[1152][384]^T + b, 2D RoPE on q and k of patch
// tokens, written per (image, head): q, k, v [images][6] matrices of
// [tpad][64] in fragment order (rows past the image's tokens are never
// written). cos / sin are [patches][64] with columns
// 32..63 repeating 0..31 (the rotation of channels c and c+32 uses angle c);
// only columns 0..31 are read.
// With stats == nullptr: h = LN1(x) is given and out = h.W^T + bias. With
// stats: h is the raw residual x, w holds W' = gamma (.) W (per input
// channel), wsum[n] = sum_k W'[n][k] and bias holds t = b + beta.W^T, so
// out = rstd * (x.W'^T - mean * wsum) + t = LN(x).W^T + b.
struct QkvArgs {
    const half_t* h;
    const half_t* w;
    const float* bias;
    const float* cos;
    const float* sin;
    half_t* q;
    half_t* k;
    half_t* v;
    int images;
    int grid;
    int tpad;
    const float* stats = nullptr;
    const float* wsum = nullptr;
};

// softmax(q k^T / 8) v per (image, head) over that image's T tokens, with
// q, k, v as written by the QKV kernel; rows T .. tpad-1 of v must be finite
// (the engine zeroes buffers at allocation and nothing writes those rows).
// out [images*T][384] frag (head h in columns 64h .. 64h+63).
struct AttentionArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    half_t* out;
    int images;
    int tokens;
    int tpad;
};

// x[rows][384] += ls * (a[rows][k] . W[384][k]^T + b), f16 residual in place
// (a and x frag).
struct ResidArgs {
    const half_t* a;
    const half_t* w;
    const float* bias;
    const float* ls;
    half_t* x;
    int rows;
    int k;
    float* stats = nullptr;  // optional: row statistics of the updated x
};

// act[rows][1536] frag = silu(h.Wg^T + bg) * (h.Wu^T + bu), h frag; W and b are packed
// with gate and up rows interleaved in blocks of 32.
// stats / wsum: LayerNorm fused as in QkvArgs.
struct SwigluArgs {
    const half_t* h;
    const half_t* w;
    const float* bias;
    half_t* act;
    int rows;
    const float* stats = nullptr;
    const float* wsum = nullptr;
};

// partials[s][rows][384] = a[:, s*k/splits ...] . W[:, s*k/splits ...]^T
// (f32 row-major; a frag).
struct SplitKArgs {
    const half_t* a;
    const half_t* w;
    float* partials;
    int rows;
    int k;
    int splits;
};

// x[rows][384] frag += ls * (sum_s partials[s] + b).
struct ReduceArgs {
    const float* partials;
    const float* bias;
    const float* ls;
    half_t* x;
    int rows;
    int splits;
    float* stats = nullptr;  // optional: row statistics of the updated x
};

// Rows tokens .. tpad-1 of q, k and v ([images][6] fragment-order [tpad][64]
// matrices) set to zero:
// attention reads them as masked keys, so they must be finite. For buffers
// that did not come zeroed from the engine (the allocation-free forward's
// scratch, which keeps earlier calls' data). A fill kernel, not a memset, so
// that the launch can be captured into a graph.
struct PadRowsArgs {
    half_t* q;
    half_t* k;
    half_t* v;
    int images;
    int tokens;
    int tpad;
};

hipError_t launch_layernorm(const LayerNormArgs& a, hipStream_t s);
hipError_t launch_zero_pad_rows(const PadRowsArgs& a, hipStream_t s);
hipError_t launch_patch_embed(const PatchEmbedArgs& a, hipStream_t s);
hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t s);
hipError_t launch_attention(const AttentionArgs& a, hipStream_t s);
hipError_t launch_resid(const ResidArgs& a, hipStream_t s);
hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t s);
hipError_t launch_splitk(const SplitKArgs& a, hipStream_t s);
hipError_t launch_splitk_reduce(const ReduceArgs& a, hipStream_t s);

}  // namespace dhx
