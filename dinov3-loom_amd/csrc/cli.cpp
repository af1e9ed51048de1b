// Command-line front end over the model C ABI (include/dinov3.h), mirroring
// the reference binary src/main.rs:6-88: read little-endian float32 NCHW RGB
// images from --input, run one forward and write the float32 tokens to
// --output (or to stdout when not benchmarking); with --benchmark N, print
// the resident timings of dinov3_benchmark to stderr and the warm end-to-end
// distribution (transfers included) to stdout as JSON lines with the
// reference's keys. Errors print as "Error: <message>" with exit status 1.
//
//   dinov3-hrx --input px.f32 [--model m.safetensors] [--offline]
//              [--output tokens.f32] [--device 0] [--max-batch 16]
//              [--benchmark N] [--image-size 224]
//
// Without --model the weights come from the local Hugging Face cache
// (hub.rs:17-54); there is no download path here, so --offline only keeps
// the reference's flag.
#include <algorithm>
#include <charconv>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <vector>

#include "dinov3.h"

namespace {

struct Args {
    std::string model;
    bool offline = false;
    std::string input;
    std::string output;
    int32_t device = 0;
    uint64_t max_batch = 16;  // main.rs:20-21
    uint64_t benchmark = 0;
    uint32_t image_size = 224;
};

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error(msg); }

uint64_t parse_u64(const std::string& flag, const std::string& v) {
    uint64_t x = 0;
    auto [p, ec] = std::from_chars(v.data(), v.data() + v.size(), x);
    if (ec != std::errc() || p != v.data() + v.size()) fail("invalid value '" + v + "' for '" + flag + "'");
    return x;
}

int32_t parse_i32(const std::string& flag, const std::string& v) {
    int32_t x = 0;
    auto [p, ec] = std::from_chars(v.data(), v.data() + v.size(), x);
    if (ec != std::errc() || p != v.data() + v.size()) fail("invalid value '" + v + "' for '" + flag + "'");
    return x;
}

// --flag value and --flag=value; --max-batch also as --max_batch.
Args parse(int argc, char** argv) {
    Args a;
    bool have_input = false;
    for (int i = 1; i < argc; ++i) {
        std::string s = argv[i], v;
        auto eq = s.find('=');
        bool inline_value = eq != std::string::npos;
        if (inline_value) {
            v = s.substr(eq + 1);
            s = s.substr(0, eq);
        }
        std::replace(s.begin(), s.end(), '_', '-');
        auto value = [&]() -> std::string {
            if (inline_value) return v;
            if (i + 1 >= argc) fail("a value is required for '" + s + "'");
            return argv[++i];
        };
        if (s == "--model") a.model = value();
        else if (s == "--offline") a.offline = true;
        else if (s == "--input") a.input = value(), have_input = true;
        else if (s == "--output") a.output = value();
        else if (s == "--device") a.device = parse_i32(s, value());
        else if (s == "--max-batch") a.max_batch = parse_u64(s, value());
        else if (s == "--benchmark") a.benchmark = parse_u64(s, value());
        else if (s == "--image-size") a.image_size = static_cast<uint32_t>(parse_u64(s, value()));
        else fail("unexpected argument '" + std::string(argv[i]) + "'");
    }
    if (!have_input) fail("the following required arguments were not provided: --input <INPUT>");
    return a;
}

std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail(path + ": " + std::strerror(errno));
    return std::vector<char>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

void write_all(FILE* f, const void* p, size_t n) {
    if (n && std::fwrite(p, 1, n, f) != n) fail(std::string("write failed: ") + std::strerror(errno));
}

// Shortest round-trip decimal, with a ".0" on integral values (serde_json's
// rendering of f64).
std::string json_number(double x) {
    char buf[64];
    auto [p, ec] = std::to_chars(buf, buf + sizeof buf, x);
    std::string s(buf, ec == std::errc() ? p : buf);
    if (s.find_first_of(".eE") == std::string::npos && std::isfinite(x)) s += ".0";
    return s;
}

void check(int rc, const dinov3_model* m) {
    if (rc != 0) fail(dinov3_last_error(m));
}

int run(const Args& a) {
    if (a.max_batch < 1 || a.max_batch > 64) fail("max_batch must be 1..=64");  // main.rs:28-31
    std::vector<char> bytes = read_file(a.input);
    auto setup = std::chrono::steady_clock::now();
    std::string model_path = a.model;
    if (model_path.empty()) {
        std::vector<char> path(4096);
        check(dinov3_hub_weights(path.data(), path.size()), nullptr);
        model_path = path.data();
    }
    if (bytes.size() % 4 != 0) fail("input must be little-endian float32 NCHW RGB");  // main.rs:37-40
    std::vector<float> pixels(bytes.size() / 4);
    std::memcpy(pixels.data(), bytes.data(), bytes.size());
    bytes = {};

    dinov3_options opts;
    dinov3_options_default(&opts);
    opts.device = a.device;
    opts.max_batch = a.max_batch;
    opts.image_size = a.image_size;
    dinov3_model* m = nullptr;
    check(dinov3_load(model_path.c_str(), &opts, &m), nullptr);
    struct Free {
        dinov3_model* m;
        ~Free() { dinov3_free(m); }
    } owner{m};
    double setup_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - setup).count();

    if (a.benchmark > 0) {
        dinov3_timings t{};
        check(dinov3_benchmark(m, pixels.data(), pixels.size(), a.benchmark, &t), m);
        std::fprintf(stderr,
                     "{\"samples\":%llu,\"graph\":{\"median_ms\":%s,\"p95_ms\":%s},"
                     "\"direct\":{\"median_ms\":%s,\"p95_ms\":%s}}\n",
                     static_cast<unsigned long long>(t.samples), json_number(t.graph.median_ms).c_str(),
                     json_number(t.graph.p95_ms).c_str(), json_number(t.direct.median_ms).c_str(),
                     json_number(t.direct.p95_ms).c_str());
    }

    uint64_t elems = dinov3_image_elements(m), per_image = dinov3_tokens(m) * DINOV3_HIDDEN;
    std::vector<float> out(elems ? pixels.size() / elems * per_image : 0);
    auto forward = [&] { check(dinov3_forward(m, pixels.data(), pixels.size(), out.data(), out.size()), m); };
    forward();
    if (!a.output.empty()) {
        FILE* f = std::fopen(a.output.c_str(), "wb");
        if (!f) fail(a.output + ": " + std::strerror(errno));
        write_all(f, out.data(), out.size() * sizeof(float));
        if (std::fclose(f) != 0) fail(a.output + ": " + std::strerror(errno));
    } else if (a.benchmark == 0) {
        write_all(stdout, out.data(), out.size() * sizeof(float));
        std::fflush(stdout);
    }

    if (a.benchmark > 0) {
        if (a.benchmark < 10) fail("use at least 10 benchmark iterations");  // main.rs:67
        for (int i = 0; i < 10; ++i) forward();
        std::vector<double> times;
        times.reserve(a.benchmark);
        for (uint64_t i = 0; i < a.benchmark; ++i) {
            auto t0 = std::chrono::steady_clock::now();
            forward();
            times.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
        }
        std::sort(times.begin(), times.end());
        size_t n = times.size();
        std::printf(
            "{\"median_ms\":%s,\"p95_ms\":%s,\"samples\":%zu,\"scope\":\"warm end-to-end, including transfers\","
            "\"setup_ms\":%s}\n",
            json_number(times[n / 2]).c_str(), json_number(times[(n * 95 + 99) / 100 - 1]).c_str(), n,
            json_number(setup_ms).c_str());
        std::fflush(stdout);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(parse(argc, argv));
    } catch (const std::exception& e) {
        std::fflush(stdout);
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
