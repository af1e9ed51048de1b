// Host-only driver for the safetensors parser and the weight loader, built
// with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_host_sanitize.py (no GPU code, no HIP runtime). Commands:
//   parse FILE...           parse each file; prints "ok <tensors>" or "error: <message>"
//   same-pack A B GRID      load_weights on both files; prints "equal <blobs>" or "differ <name>"
//   pack-kat                weights.rs:152-169 through pack_f16, plus the 65520 overflow text
//   generate PATH PRESET    write_random_weights(PATH, 0, PRESET), then load it at grids 14 and 32
//   mutate FILE N SEED      parse N copies of FILE with random bytes of the header changed
// Exit status 0 unless a check fails; any sanitizer report aborts the run.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../dinov3-loom_amd/csrc/errors.hpp"
#include "../dinov3-loom_amd/csrc/safetensors.hpp"
#include "../dinov3-loom_amd/csrc/weights.hpp"

namespace dhx {
// The library defines these beside its C ABI (model.cpp), which this driver
// does not link.
void set_global_error(const std::string&) {}
const char* global_error() { return ""; }
}  // namespace dhx

namespace {

int parse(int argc, char** argv) {
    for (int i = 2; i < argc; ++i) {
        try {
            const dhx::SafeTensors st(dhx::read_file(argv[i]));
            uint64_t bytes = 0;
            for (auto& kv : st.tensors()) bytes += kv.second.bytes;
            std::printf("%s: ok %zu %llu\n", argv[i], st.tensors().size(), (unsigned long long)bytes);
        } catch (const dhx::Error& e) {
            std::printf("%s: error: %s\n", argv[i], e.what());
        }
    }
    return 0;
}

int same_pack(const char* a, const char* b, int grid) {
    const dhx::Packed pa = dhx::load_weights(a, (uint32_t)grid), pb = dhx::load_weights(b, (uint32_t)grid);
    if (pa.size() != pb.size()) {
        std::printf("differ count %zu %zu\n", pa.size(), pb.size());
        return 0;
    }
    for (size_t i = 0; i < pa.size(); ++i)
        if (pa[i].first != pb[i].first || pa[i].second != pb[i].second) {
            std::printf("differ %s\n", pa[i].first.c_str());
            return 0;
        }
    std::printf("equal %zu\n", pa.size());
    return 0;
}

int pack_kat() {
    const float in[8] = {0.f, -0.f, 1.f, -1.f, 65504.f, -65504.f, 65519.f, -65519.f};
    const uint16_t want[8] = {0x0000, 0x8000, 0x3c00, 0xbc00, 0x7bff, 0xfbff, 0x7bff, 0xfbff};
    const std::vector<uint8_t> b = dhx::pack_f16("weights", in, 8);
    for (int i = 0; i < 8; ++i) {
        const uint16_t got = (uint16_t)(b[2 * i] | (b[2 * i + 1] << 8));
        if (got != want[i]) {
            std::printf("pack-kat: value %d gives 0x%04x, want 0x%04x\n", i, got, want[i]);
            return 1;
        }
    }
    const float over[3] = {0.f, 1.f, 65520.f};
    try {
        dhx::pack_f16("w", over, 3);
        std::printf("pack-kat: 65520 was accepted\n");
        return 1;
    } catch (const dhx::Error& e) {
        if (std::strcmp(e.what(), "tensor w[2] cannot be represented as finite float16: 65520") != 0) {
            std::printf("pack-kat: wrong message: %s\n", e.what());
            return 1;
        }
    }
    std::printf("pack-kat ok\n");
    return 0;
}

int generate(const char* path, int preset) {
    dhx::write_random_weights(path, 0, preset);
    const dhx::Packed p14 = dhx::load_weights(path, 14), p32 = dhx::load_weights(path, 32);
    std::printf("generate ok %zu %zu\n", p14.size(), p32.size());
    return 0;
}

// xorshift64*: a reproducible byte stream for the mutations.
uint64_t next(uint64_t& s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1Dull;
}

int mutate(const char* path, int n, uint64_t seed) {
    const std::vector<uint8_t> base = dhx::read_file(path);
    uint64_t hdr = 0;
    for (int i = 7; i >= 0; --i) hdr = (hdr << 8) | base[i];
    const uint64_t span = std::min<uint64_t>(base.size(), 8 + hdr + 16);
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    int ok = 0, rejected = 0;
    for (int it = 0; it < n; ++it) {
        std::vector<uint8_t> f = base;
        const int edits = 1 + (int)(next(s) % 4);
        for (int e = 0; e < edits; ++e) {
            const uint64_t at = next(s) % std::min<uint64_t>(span, f.size());
            switch (next(s) % 4) {
                case 0: f[at] = (uint8_t)next(s); break;                     // random byte
                case 1: f[at] = "{}[]\":,0123456789-.eE \\u"[next(s) % 25]; break;  // JSON punctuation
                case 2: f.erase(f.begin() + (long)at); break;                // drop a byte
                default: f.resize(at); break;                                 // truncate
            }
            if (f.empty()) break;
        }
        try {
            const dhx::SafeTensors st(std::move(f));
            for (auto& kv : st.tensors()) {
                // touch every byte of every accepted tensor: ASan flags reads past the file
                volatile uint8_t sink = 0;
                for (uint64_t i = 0; i < kv.second.bytes; i += 61) sink ^= kv.second.data[i];
                if (kv.second.bytes) sink ^= kv.second.data[kv.second.bytes - 1];
            }
            ++ok;
        } catch (const dhx::Error&) {
            ++rejected;
        }
    }
    std::printf("mutate ok=%d rejected=%d\n", ok, rejected);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string cmd = argv[1];
    try {
        if (cmd == "parse") return parse(argc, argv);
        if (cmd == "same-pack" && argc == 5) return same_pack(argv[2], argv[3], std::atoi(argv[4]));
        if (cmd == "pack-kat") return pack_kat();
        if (cmd == "generate" && argc == 4) return generate(argv[2], std::atoi(argv[3]));
        if (cmd == "mutate" && argc == 5) return mutate(argv[2], std::atoi(argv[3]), std::strtoull(argv[4], nullptr, 10));
    } catch (const dhx::Error& e) {
        std::printf("error: %s\n", e.what());
        return 3;
    }
    return 2;
}
