// Weight validation and packing (weights.rs:6-146), the seeded random-init
// generator, synthetic pixels and host patchify (lib.rs:265-280).
#pragma once
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace dhx {

// Named device-ready byte blobs in upload order.
using Packed = std::vector<std::pair<std::string, std::vector<uint8_t>>>;

// weights.rs:6-17: float32 -> float16 (round to nearest even), rejecting
// values that do not stay finite.
std::vector<uint8_t> pack_f16(const std::string& name, const float* values, size_t n);

// weights.rs:19-146, with the RoPE tables built for a grid x grid patch grid.
// Packed names: patch_w, patch_b, prefix, prefix_stats, l{i}_{norm1_w,
// norm1_b, norm2_w, norm2_b, ls1, ls2, qkv_w, qkv_b, qkv_wln, qkv_wsum,
// qkv_t, gateup_w, gateup_b, gateup_wln, gateup_wsum, gateup_t, o_w, o_b,
// down_w, down_b}, norm_w, norm_b, rope_cos, rope_sin. gateup_* rows are
// interleaved in blocks of 32 gate rows then the 32 matching up rows;
// qkv_w, qkv_wln, gateup_w, gateup_wln, o_w and down_w are in fragment order (32-row x
// 16-column blocks, as the GEMMs' weight DMA reads them). The
// *_wln / *_wsum / *_t tensors fold the preceding LayerNorm into the GEMM
// (see DHX_K_QKV_ROPE_LN in dinov3_engine.h).
Packed load_weights(const std::string& path, uint32_t grid);

void write_random_weights(const std::string& path, uint64_t seed, int preset);
void random_pixels(uint64_t seed, uint64_t images, uint32_t image_size, float* out);
void patchify(const float* pixels, uint64_t images, uint32_t image_size, float* out);

}  // namespace dhx
