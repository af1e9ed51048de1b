#include "weights.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>

#include "errors.hpp"
#include "safetensors.hpp"

namespace dhx {
namespace {

std::string shape_text(const std::vector<uint64_t>& s) {
    std::string out = "[";
    for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
    return out + "]";
}

std::string float_text(float v) {
    char buf[64];
    std::snprintf(buf, sizeof buf, "%.9g", (double)v);
    return buf;
}

float bf16_to_f32(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// weights.rs:22-51 (`get`): look up, check shape, widen F32/F16/BF16 to f32,
// require finite values.
std::vector<float> get(const SafeTensors& st, const std::string& name, const std::vector<uint64_t>& shape) {
    const TensorView* t = st.find(name);
    if (!t) throw Error("missing tensor " + name);
    if (t->shape != shape) throw Error(name + ": expected " + shape_text(shape) + ", found " + shape_text(t->shape));
    std::vector<float> v;
    if (t->dtype == "F32") {
        v.resize(t->bytes / 4);
        std::memcpy(v.data(), t->data, t->bytes);
    } else if (t->dtype == "F16") {
        v.resize(t->bytes / 2);
        for (size_t i = 0; i < v.size(); ++i) {
            _Float16 h;
            std::memcpy(&h, t->data + 2 * i, 2);
            v[i] = (float)h;
        }
    } else if (t->dtype == "BF16") {
        v.resize(t->bytes / 2);
        for (size_t i = 0; i < v.size(); ++i) {
            uint16_t b;
            std::memcpy(&b, t->data + 2 * i, 2);
            v[i] = bf16_to_f32(b);
        }
    } else {
        throw Error("unsupported dtype " + t->dtype + " for " + name);
    }
    for (float x : v)
        if (!std::isfinite(x)) throw Error("non-finite tensor " + name);
    return v;
}

std::vector<uint8_t> f32_bytes(const std::vector<float>& v) {
    std::vector<uint8_t> b(v.size() * 4);
    std::memcpy(b.data(), v.data(), b.size());
    return b;
}

// LayerNorm folded into the following GEMM: W' = f16(gamma[k] * W[n][k]),
// wsum[n] = sum_k W'[n][k] (of the rounded values, so x.W'^T - mean*wsum is
// exactly (x - mean).W'^T), t[n] = b[n] + sum_k beta[k] * W[n][k].
struct Folded {
    std::vector<uint8_t> w;
    std::vector<float> wsum, t;
};

Folded fold_layernorm(const std::string& name, const std::vector<float>& w, const std::vector<float>& b,
                      const std::vector<float>& gamma, const std::vector<float>& beta, size_t n, size_t k);

std::vector<float> prefix_stats(const std::vector<float>& prefix);

// Row-major f16 [n][k] -> the fragment order the GEMMs' weight DMA reads:
// 32-row x 16-column blocks, block (nb, ks) at (nb * k/16 + ks) * 512
// halfs, lane hi*32 + l of a block holding row 32nb + l, columns
// 16ks + 8hi .. +7 (n a multiple of 32, k of 16).
std::vector<uint8_t> fragment_order(const std::vector<uint8_t>& rows, size_t n, size_t k) {
    std::vector<uint8_t> out(rows.size());
    for (size_t r = 0; r < n; ++r)
        for (size_t c8 = 0; c8 < k; c8 += 8) {
            const size_t dst = ((r / 32) * (k / 16) + c8 / 16) * 512 + ((c8 / 8) % 2 * 32 + r % 32) * 8;
            std::memcpy(&out[dst * 2], &rows[(r * k + c8) * 2], 16);
        }
    return out;
}

}  // namespace

std::vector<uint8_t> pack_f16(const std::string& name, const float* values, size_t n) {
    std::vector<uint8_t> bytes(n * 2);
    for (size_t i = 0; i < n; ++i) {
        const _Float16 h = (_Float16)values[i];  // IEEE round to nearest, ties to even
        if (!std::isfinite((float)h))
            throw Error("tensor " + name + "[" + std::to_string(i) + "] cannot be represented as finite float16: " +
                        float_text(values[i]));
        std::memcpy(bytes.data() + 2 * i, &h, 2);
    }
    return bytes;
}

namespace {

Folded fold_layernorm(const std::string& name, const std::vector<float>& w, const std::vector<float>& b,
                      const std::vector<float>& gamma, const std::vector<float>& beta, size_t n, size_t k) {
    std::vector<float> scaled(n * k);
    for (size_t r = 0; r < n; ++r)
        for (size_t c = 0; c < k; ++c) scaled[r * k + c] = gamma[c] * w[r * k + c];
    Folded f{pack_f16(name, scaled.data(), scaled.size()), std::vector<float>(n), std::vector<float>(n)};
    for (size_t r = 0; r < n; ++r) {
        double sum = 0.0, shift = b[r];
        for (size_t c = 0; c < k; ++c) {
            _Float16 h;
            std::memcpy(&h, f.w.data() + 2 * (r * k + c), 2);
            sum += (double)(float)h;
            shift += (double)beta[c] * (double)w[r * k + c];
        }
        f.wsum[r] = (float)sum;
        f.t[r] = (float)shift;
    }
    return f;
}

// Row statistics of the 5 prefix rows as stored in x (f16): per 64-column
// slot, (mean, sum of squared deviations), laid out [row][slot][2].
std::vector<float> prefix_stats(const std::vector<float>& prefix) {
    std::vector<float> out(5 * 12);
    for (int r = 0; r < 5; ++r)
        for (int slot = 0; slot < 6; ++slot) {
            double v[64], mean = 0.0, m2 = 0.0;
            for (int c = 0; c < 64; ++c) {
                v[c] = (double)(float)(_Float16)prefix[r * 384 + slot * 64 + c];
                mean += v[c];
            }
            mean /= 64.0;
            for (int c = 0; c < 64; ++c) m2 += (v[c] - mean) * (v[c] - mean);
            out[r * 12 + slot * 2] = (float)mean;
            out[r * 12 + slot * 2 + 1] = (float)m2;
        }
    return out;
}

}  // namespace

Packed load_weights(const std::string& path, uint32_t grid) {
    const SafeTensors st(read_file(path));
    Packed out;
    auto emit = [&](const std::string& name, const std::vector<float>& v, bool half) {
        out.emplace_back(name, half ? pack_f16(name, v.data(), v.size()) : f32_bytes(v));
    };
    // patch_w first: an unrepresentable value fails here, before any other
    // tensor is read and before the GPU is touched (tests/model.rs:29-59).
    emit("patch_w", get(st, "embeddings.patch_embeddings.weight", {384, 3, 16, 16}), true);
    emit("patch_b", get(st, "embeddings.patch_embeddings.bias", {384}), false);
    std::vector<float> prefix = get(st, "embeddings.cls_token", {1, 1, 384});
    const std::vector<float> reg = get(st, "embeddings.register_tokens", {1, 4, 384});
    prefix.insert(prefix.end(), reg.begin(), reg.end());
    emit("prefix", prefix, false);
    emit("prefix_stats", prefix_stats(prefix), false);
    for (int i = 0; i < 12; ++i) {
        const std::string p = "layer." + std::to_string(i) + ".";
        const std::string l = "l" + std::to_string(i) + "_";
        const std::pair<const char*, const char*> vectors[] = {
            {"norm1_w", "norm1.weight"}, {"norm1_b", "norm1.bias"}, {"norm2_w", "norm2.weight"},
            {"norm2_b", "norm2.bias"},   {"ls1", "layer_scale1.lambda1"}, {"ls2", "layer_scale2.lambda1"}};
        for (auto& v : vectors) emit(l + v.first, get(st, p + v.second, {384}), false);
        // weights.rs:91-108: q, k, v rows concatenated; k has no bias.
        std::vector<float> qw, qb;
        for (const char* q : {"q", "k", "v"}) {
            const std::vector<float> w = get(st, p + "attention." + q + "_proj.weight", {384, 384});
            qw.insert(qw.end(), w.begin(), w.end());
            if (std::string(q) == "k") {
                qb.insert(qb.end(), 384, 0.0f);
            } else {
                const std::vector<float> b = get(st, p + "attention." + q + "_proj.bias", {384});
                qb.insert(qb.end(), b.begin(), b.end());
            }
        }
        out.emplace_back(l + "qkv_w", fragment_order(pack_f16(l + "qkv_w", qw.data(), qw.size()), 1152, 384));
        emit(l + "qkv_b", qb, false);
        {
            Folded f = fold_layernorm(l + "qkv_wln", qw, qb, get(st, p + "norm1.weight", {384}),
                                      get(st, p + "norm1.bias", {384}), 1152, 384);
            out.emplace_back(l + "qkv_wln", fragment_order(f.w, 1152, 384));
            emit(l + "qkv_wsum", f.wsum, false);
            emit(l + "qkv_t", f.t, false);
        }
        // Gate and up rows, interleaved in blocks of 32 so one wave's 64
        // GEMM columns are 32 gate outputs and the same 32 up outputs.
        const std::vector<float> gw = get(st, p + "mlp.gate_proj.weight", {1536, 384});
        const std::vector<float> uw = get(st, p + "mlp.up_proj.weight", {1536, 384});
        const std::vector<float> gb = get(st, p + "mlp.gate_proj.bias", {1536});
        const std::vector<float> ub = get(st, p + "mlp.up_proj.bias", {1536});
        std::vector<float> w(3072 * 384), b(3072);
        for (int blk = 0; blk < 1536 / 32; ++blk)
            for (int r = 0; r < 32; ++r) {
                const int src = blk * 32 + r;
                std::memcpy(&w[(size_t)(blk * 64 + r) * 384], &gw[(size_t)src * 384], 384 * 4);
                std::memcpy(&w[(size_t)(blk * 64 + 32 + r) * 384], &uw[(size_t)src * 384], 384 * 4);
                b[blk * 64 + r] = gb[src];
                b[blk * 64 + 32 + r] = ub[src];
            }
        out.emplace_back(l + "gateup_w", fragment_order(pack_f16(l + "gateup_w", w.data(), w.size()), 3072, 384));
        emit(l + "gateup_b", b, false);
        {
            Folded f = fold_layernorm(l + "gateup_wln", w, b, get(st, p + "norm2.weight", {384}),
                                      get(st, p + "norm2.bias", {384}), 3072, 384);
            out.emplace_back(l + "gateup_wln", fragment_order(f.w, 3072, 384));
            emit(l + "gateup_wsum", f.wsum, false);
            emit(l + "gateup_t", f.t, false);
        }
        for (auto& v : {std::make_pair("o", std::make_pair("attention.o_proj", 384u)),
                        std::make_pair("down", std::make_pair("mlp.down_proj", 1536u))}) {
            const std::vector<float> w = get(st, p + v.second.first + ".weight", {384, v.second.second});
            out.emplace_back(l + v.first + "_w",
                             fragment_order(pack_f16(l + v.first + "_w", w.data(), w.size()), 384, v.second.second));
            emit(l + v.first + "_b", get(st, p + v.second.first + ".bias", {384}), false);
        }
    }
    emit("norm_w", get(st, "norm.weight", {384}), false);
    emit("norm_b", get(st, "norm.bias", {384}), false);
    // weights.rs:127-144 with 14 -> grid: per patch (y, x) the 64 entries
    // [y x16, x x16, y x16, x x16], angle = 2 pi (2(pos+0.5)/G - 1) / 100^(j/16).
    std::vector<float> cs, sn;
    cs.reserve((size_t)grid * grid * 64);
    sn.reserve((size_t)grid * grid * 64);
    for (uint32_t y = 0; y < grid; ++y)
        for (uint32_t x = 0; x < grid; ++x)
            for (int rep = 0; rep < 2; ++rep)
                for (uint32_t pos : {y, x})
                    for (int j = 0; j < 16; ++j) {
                        const double coord = 2.0 * ((double)pos + 0.5) / (double)grid - 1.0;
                        const double a = 2.0 * M_PI * coord / std::pow(100.0, (double)j / 16.0);
                        cs.push_back((float)std::cos(a));
                        sn.push_back((float)std::sin(a));
                    }
    emit("rope_cos", cs, false);
    emit("rope_sin", sn, false);
    return out;
}

// ---------------------------------------------------------------------------
// Seeded random init. Generator: xoshiro256** seeded through splitmix64 from
// (seed, tensor index); uniforms are the top 53 bits; normals are Box-Muller
// (cos branch, one normal per two uniforms); trunc-normal rejects |z| > 2
// before scaling by the standard deviation.
namespace {

uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s[4];
    Rng(uint64_t seed, uint64_t stream) {
        uint64_t x = seed ^ (0xD1B54A32D192ED03ull * (stream + 1));
        for (auto& v : s) v = splitmix64(x);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t result = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return result;
    }
    double uniform() { return (double)(next() >> 11) * 0x1.0p-53; }
    double normal() {
        const double u1 = uniform(), u2 = uniform();
        return std::sqrt(-2.0 * std::log(1.0 - u1)) * std::cos(2.0 * M_PI * u2);
    }
    double trunc_normal(double std_dev) {
        for (;;) {
            const double z = normal();
            if (std::fabs(z) <= 2.0) return z * std_dev;
        }
    }
};

enum class Init { TruncNormal, Normal, Constant, OnePlusNormal };

struct Spec {
    Init kind;
    double a;  // std or constant
};

}  // namespace

void write_random_weights(const std::string& path, uint64_t seed, int preset) {
    if (preset != 0 && preset != 1) throw Error("unknown weight preset " + std::to_string(preset));
    const bool stress = preset == 1;
    std::vector<OwnedTensor> tensors;
    uint64_t stream = 0;
    auto add = [&](const std::string& name, std::vector<uint64_t> shape, Spec spec) {
        OwnedTensor t{name, shape, {}};
        uint64_t n = 1;
        for (uint64_t d : shape) n *= d;
        t.values.resize(n);
        Rng rng(seed, stream++);
        for (auto& v : t.values) {
            switch (spec.kind) {
                case Init::TruncNormal: v = (float)rng.trunc_normal(spec.a); break;
                case Init::Normal: v = (float)(rng.normal() * spec.a); break;
                case Init::Constant: v = (float)spec.a; break;
                case Init::OnePlusNormal: v = (float)(1.0 + rng.normal() * spec.a); break;
            }
        }
        tensors.push_back(std::move(t));
    };
    const Spec w02{Init::TruncNormal, 0.02};
    const Spec bias = stress ? Spec{Init::Normal, 0.02} : Spec{Init::Constant, 0.0};
    const Spec gamma = stress ? Spec{Init::OnePlusNormal, 0.1} : Spec{Init::Constant, 1.0};
    const Spec beta = stress ? Spec{Init::Normal, 0.1} : Spec{Init::Constant, 0.0};
    const Spec ls{Init::Constant, stress ? 1.0 : 1e-5};
    const Spec qk = stress ? Spec{Init::TruncNormal, 0.06} : w02;
    add("embeddings.patch_embeddings.weight", {384, 3, 16, 16}, w02);
    add("embeddings.patch_embeddings.bias", {384}, bias);
    add("embeddings.cls_token", {1, 1, 384}, w02);
    add("embeddings.register_tokens", {1, 4, 384}, w02);
    add("embeddings.mask_token", {1, 1, 384}, Spec{Init::Constant, 0.0});
    for (int i = 0; i < 12; ++i) {
        const std::string p = "layer." + std::to_string(i) + ".";
        add(p + "norm1.weight", {384}, gamma);
        add(p + "norm1.bias", {384}, beta);
        add(p + "attention.q_proj.weight", {384, 384}, qk);
        add(p + "attention.q_proj.bias", {384}, bias);
        add(p + "attention.k_proj.weight", {384, 384}, qk);
        add(p + "attention.v_proj.weight", {384, 384}, w02);
        add(p + "attention.v_proj.bias", {384}, bias);
        add(p + "attention.o_proj.weight", {384, 384}, w02);
        add(p + "attention.o_proj.bias", {384}, bias);
        add(p + "layer_scale1.lambda1", {384}, ls);
        add(p + "norm2.weight", {384}, gamma);
        add(p + "norm2.bias", {384}, beta);
        add(p + "mlp.gate_proj.weight", {1536, 384}, w02);
        add(p + "mlp.gate_proj.bias", {1536}, bias);
        add(p + "mlp.up_proj.weight", {1536, 384}, w02);
        add(p + "mlp.up_proj.bias", {1536}, bias);
        add(p + "mlp.down_proj.weight", {384, 1536}, w02);
        add(p + "mlp.down_proj.bias", {384}, bias);
        add(p + "layer_scale2.lambda1", {384}, ls);
    }
    add("norm.weight", {384}, gamma);
    add("norm.bias", {384}, beta);
    write_f32_safetensors(path, tensors);
}

void random_pixels(uint64_t seed, uint64_t images, uint32_t image_size, float* out) {
    Rng rng(seed, 0);
    const uint64_t n = images * 3ull * image_size * image_size;
    for (uint64_t i = 0; i < n; ++i) out[i] = (float)rng.normal();
}

void patchify(const float* pixels, uint64_t images, uint32_t image_size, float* out) {
    const uint32_t G = image_size / 16, S = image_size;
    size_t o = 0;
    for (uint64_t n = 0; n < images; ++n) {
        const float* img = pixels + n * 3ull * S * S;
        for (uint32_t gy = 0; gy < G; ++gy)
            for (uint32_t gx = 0; gx < G; ++gx)
                for (uint32_t c = 0; c < 3; ++c)
                    for (uint32_t dy = 0; dy < 16; ++dy) {
                        std::memcpy(out + o, img + ((size_t)c * S + gy * 16 + dy) * S + gx * 16, 16 * sizeof(float));
                        o += 16;
                    }
    }
}

}  // namespace dhx
