// Minimal safetensors reader/writer (format: 8-byte little-endian header
// length, JSON header {name: {dtype, shape, data_offsets}}, raw data).
// Replaces the `safetensors` crate calls of weights.rs:19-21.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace dhx {

struct TensorView {
    std::string dtype;
    std::vector<uint64_t> shape;
    const uint8_t* data = nullptr;
    uint64_t bytes = 0;
};

class SafeTensors {
public:
    // Takes ownership of the file bytes; throws dhx::Error on malformed input.
    explicit SafeTensors(std::vector<uint8_t> file);
    const TensorView* find(const std::string& name) const;
    const std::map<std::string, TensorView>& tensors() const { return tensors_; }

private:
    std::vector<uint8_t> file_;
    std::map<std::string, TensorView> tensors_;
};

struct OwnedTensor {
    std::string name;
    std::vector<uint64_t> shape;
    std::vector<float> values;
};

// Writes float32 tensors in the given order.
void write_f32_safetensors(const std::string& path, const std::vector<OwnedTensor>& tensors);

std::vector<uint8_t> read_file(const std::string& path);

}  // namespace dhx
