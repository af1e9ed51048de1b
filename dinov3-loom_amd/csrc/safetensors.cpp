#include "safetensors.hpp"

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <fstream>

#include "errors.hpp"

namespace dhx {
namespace {

// Just enough JSON for a safetensors header: objects, arrays, strings,
// non-negative integers (offsets, shapes) and the odd literal in metadata.
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    uint64_t integer = 0;
    bool is_integer = false;
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;
};

class Parser {
public:
    Parser(const char* p, const char* end) : p_(p), end_(end) {}

    Json parse_document() {
        Json v = value();
        ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;
    int depth_ = 0;

    [[noreturn]] void fail(const char* what) { throw Error(std::string("invalid safetensors header: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    char peek() {
        ws();
        if (p_ >= end_) fail("unexpected end");
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) fail("unexpected character");
        ++p_;
    }
    Json value() {
        if (++depth_ > 64) fail("nesting too deep");
        Json v;
        const char c = peek();
        if (c == '{') {
            v.kind = Json::Object;
            ++p_;
            if (peek() == '}') {
                ++p_;
            } else {
                for (;;) {
                    std::string key = string();
                    expect(':');
                    v.members.emplace_back(std::move(key), value());
                    const char d = peek();
                    ++p_;
                    if (d == '}') break;
                    if (d != ',') fail("expected , or }");
                }
            }
        } else if (c == '[') {
            v.kind = Json::Array;
            ++p_;
            if (peek() == ']') {
                ++p_;
            } else {
                for (;;) {
                    v.items.push_back(value());
                    const char d = peek();
                    ++p_;
                    if (d == ']') break;
                    if (d != ',') fail("expected , or ]");
                }
            }
        } else if (c == '"') {
            v.kind = Json::String;
            v.text = string();
        } else if (c == 't' || c == 'f' || c == 'n') {
            const char* words[] = {"true", "false", "null"};
            for (const char* w : words) {
                const size_t n = std::strlen(w);
                if ((size_t)(end_ - p_) >= n && std::strncmp(p_, w, n) == 0) {
                    p_ += n;
                    v.kind = w[0] == 'n' ? Json::Null : Json::Bool;
                    --depth_;
                    return v;
                }
            }
            fail("bad literal");
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            // JSON number grammar: -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?
            // Only a plain non-negative integer that fits 64 bits is an
            // integer (shapes and offsets must be).
            v.kind = Json::Number;
            bool integer = true;
            if (*p_ == '-') {
                integer = false;
                ++p_;
            }
            auto digit = [&] { return p_ < end_ && *p_ >= '0' && *p_ <= '9'; };
            if (!digit()) fail("bad number");
            uint64_t acc = 0;
            if (*p_ == '0') {
                ++p_;
            } else {
                while (digit()) {
                    const uint64_t dgt = (uint64_t)(*p_++ - '0');
                    if (acc > (UINT64_MAX - dgt) / 10) integer = false;  // does not fit u64
                    else acc = acc * 10 + dgt;
                }
            }
            if (p_ < end_ && *p_ == '.') {
                integer = false;
                ++p_;
                if (!digit()) fail("bad number");
                while (digit()) ++p_;
            }
            if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
                integer = false;
                ++p_;
                if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
                if (!digit()) fail("bad number");
                while (digit()) ++p_;
            }
            v.integer = acc;
            v.is_integer = integer;
        } else {
            fail("unexpected character");
        }
        --depth_;
        return v;
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("bad unicode escape");
        uint32_t cp = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = *p_++;
            cp <<= 4;
            if (h >= '0' && h <= '9') cp |= h - '0';
            else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
            else fail("bad unicode escape");
        }
        return cp;
    }
    std::string string() {
        expect('"');
        std::string out;
        while (p_ < end_ && *p_ != '"') {
            if (*p_ == '\\') {
                ++p_;
                if (p_ >= end_) fail("bad escape");
                const char e = *p_++;
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        uint32_t cp = hex4();
                        if (cp >= 0xdc00 && cp <= 0xdfff) fail("lone surrogate");
                        if (cp >= 0xd800 && cp <= 0xdbff) {  // a pair: \uD8xx\uDCxx
                            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') fail("lone surrogate");
                            p_ += 2;
                            const uint32_t lo = hex4();
                            if (lo < 0xdc00 || lo > 0xdfff) fail("lone surrogate");
                            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                        }
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xc0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3f));
                        } else if (cp < 0x10000) {
                            out += (char)(0xe0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3f));
                            out += (char)(0x80 | (cp & 0x3f));
                        } else {
                            out += (char)(0xf0 | (cp >> 18));
                            out += (char)(0x80 | ((cp >> 12) & 0x3f));
                            out += (char)(0x80 | ((cp >> 6) & 0x3f));
                            out += (char)(0x80 | (cp & 0x3f));
                        }
                        break;
                    }
                    default: fail("bad escape");
                }
            } else {
                if ((unsigned char)*p_ < 0x20) fail("control character in string");
                out += *p_++;
            }
        }
        if (p_ >= end_) fail("unterminated string");
        ++p_;
        return out;
    }
};

// Bits per element of the dtypes the format defines (safetensors 0.6
// `Dtype::bitsize`); the loader itself only widens F32, F16 and BF16.
uint64_t dtype_bits(const std::string& d) {
    if (d == "F64" || d == "I64" || d == "U64" || d == "C64") return 64;
    if (d == "F32" || d == "I32" || d == "U32") return 32;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 16;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2" || d == "F8_E8M0") return 8;
    if (d == "F6_E2M3" || d == "F6_E3M2") return 6;
    if (d == "F4") return 4;
    throw Error("invalid safetensors header: unknown dtype " + d);
}

// RFC 3629 UTF-8 (no overlongs, no surrogates, at most U+10FFFF): the crate
// reads the header as a Rust str.
bool valid_utf8(const uint8_t* s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t cp, min;
        if ((c & 0xe0) == 0xc0) len = 2, cp = c & 0x1f, min = 0x80;
        else if ((c & 0xf0) == 0xe0) len = 3, cp = c & 0x0f, min = 0x800;
        else if ((c & 0xf8) == 0xf0) len = 4, cp = c & 0x07, min = 0x10000;
        else return false;
        if (n - i < (uint64_t)len) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if (cp < min || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
        i += len;
    }
    return true;
}

}  // namespace

std::vector<uint8_t> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error("read " + path + ": " + std::strerror(errno));
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    if (n < 0) throw Error("read " + path + ": cannot determine size");
    f.seekg(0, std::ios::beg);
    std::vector<uint8_t> data((size_t)n);
    if (n > 0 && !f.read(reinterpret_cast<char*>(data.data()), n)) throw Error("read " + path + ": short read");
    return data;
}

// The checks of the safetensors crate (0.6, `SafeTensors::read_metadata` and
// `Metadata::validate`): header length at most 100,000,000 bytes and within
// the file, a UTF-8 JSON object starting with '{', string-valued
// __metadata__, unique tensor names, and data ranges that, sorted by offset,
// tile the data section exactly from 0 to its end (no gaps, overlaps or
// trailing bytes), each range holding exactly shape x dtype bytes.
SafeTensors::SafeTensors(std::vector<uint8_t> file) : file_(std::move(file)) {
    constexpr uint64_t kMaxHeader = 100000000;
    if (file_.size() < 8) throw Error("invalid safetensors header: file too small");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | file_[i];
    if (n > kMaxHeader) throw Error("invalid safetensors header: header too large");
    if (n > file_.size() - 8) throw Error("invalid safetensors header: bad header length");
    if (n == 0 || file_[8] != '{') throw Error("invalid safetensors header: does not start with {");
    if (!valid_utf8(file_.data() + 8, n)) throw Error("invalid safetensors header: not UTF-8");
    const char* h = reinterpret_cast<const char*>(file_.data() + 8);
    Json doc = Parser(h, h + n).parse_document();
    if (doc.kind != Json::Object) throw Error("invalid safetensors header: not an object");
    const uint8_t* base = file_.data() + 8 + n;
    const uint64_t data_bytes = file_.size() - 8 - n;
    struct Range {
        uint64_t begin, end;
        const std::string* name;
    };
    std::vector<Range> ranges;
    for (auto& kv : doc.members) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind != Json::Object) throw Error("invalid safetensors header: __metadata__");
            for (auto& m : kv.second.members)
                if (m.second.kind != Json::String) throw Error("invalid safetensors header: __metadata__ value " + m.first);
            continue;
        }
        if (tensors_.count(kv.first)) throw Error("invalid safetensors header: duplicate tensor " + kv.first);
        const Json& t = kv.second;
        if (t.kind != Json::Object) throw Error("invalid safetensors header: tensor " + kv.first);
        TensorView view;
        const Json* offsets = nullptr;
        bool have_shape = false;
        for (auto& m : t.members) {
            if (m.first == "dtype" && m.second.kind == Json::String) view.dtype = m.second.text;
            else if (m.first == "shape" && m.second.kind == Json::Array) {
                have_shape = true;
                for (auto& d : m.second.items) {
                    if (d.kind != Json::Number || !d.is_integer) throw Error("invalid safetensors header: shape of " + kv.first);
                    view.shape.push_back(d.integer);
                }
            } else if (m.first == "data_offsets" && m.second.kind == Json::Array) {
                offsets = &m.second;
            }
        }
        if (view.dtype.empty() || !have_shape || !offsets || offsets->items.size() != 2)
            throw Error("invalid safetensors header: tensor " + kv.first);
        const Json& b = offsets->items[0];
        const Json& e = offsets->items[1];
        if (!b.is_integer || !e.is_integer || b.integer > e.integer || e.integer > data_bytes)
            throw Error("invalid safetensors header: offsets of " + kv.first);
        uint64_t numel = 1;
        for (uint64_t d : view.shape) {
            if (d != 0 && numel > UINT64_MAX / d) throw Error("invalid safetensors header: shape of " + kv.first);
            numel *= d;
        }
        const uint64_t bits = dtype_bits(view.dtype);
        if (numel > UINT64_MAX / bits) throw Error("invalid safetensors header: shape of " + kv.first);
        if (numel * bits % 8 != 0) throw Error("invalid safetensors header: misaligned size of " + kv.first);
        if (numel * bits / 8 != e.integer - b.integer) throw Error("invalid safetensors header: size of " + kv.first);
        view.data = base + b.integer;
        view.bytes = e.integer - b.integer;
        auto it = tensors_.emplace(kv.first, std::move(view)).first;
        ranges.push_back({b.integer, e.integer, &it->first});
    }
    std::sort(ranges.begin(), ranges.end(),
              [](const Range& x, const Range& y) { return x.begin != y.begin ? x.begin < y.begin : x.end < y.end; });
    uint64_t at = 0;
    for (const Range& r : ranges) {
        if (r.begin != at) throw Error("invalid safetensors header: offsets of " + *r.name);
        at = r.end;
    }
    if (at != data_bytes) throw Error("invalid safetensors header: data section is not exactly covered by tensors");
}

const TensorView* SafeTensors::find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

void write_f32_safetensors(const std::string& path, const std::vector<OwnedTensor>& tensors) {
    std::string header = "{";
    uint64_t offset = 0;
    for (size_t i = 0; i < tensors.size(); ++i) {
        const OwnedTensor& t = tensors[i];
        uint64_t numel = 1;
        for (uint64_t d : t.shape) numel *= d;
        if (numel != t.values.size()) throw Error("tensor " + t.name + ": shape does not match its values");
        if (i) header += ",";
        header += "\"" + t.name + "\":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t j = 0; j < t.shape.size(); ++j) header += (j ? "," : "") + std::to_string(t.shape[j]);
        header += "],\"data_offsets\":[" + std::to_string(offset) + "," + std::to_string(offset + numel * 4) + "]}";
        offset += numel * 4;
    }
    header += "}";
    while (header.size() % 8) header += ' ';
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw Error("write " + path + ": " + std::strerror(errno));
    uint8_t len[8];
    const uint64_t n = header.size();
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(n >> (8 * i));
    f.write(reinterpret_cast<const char*>(len), 8);
    f.write(header.data(), (std::streamsize)header.size());
    for (const OwnedTensor& t : tensors)
        f.write(reinterpret_cast<const char*>(t.values.data()), (std::streamsize)(t.values.size() * 4));
    if (!f) throw Error("write " + path + ": short write");
}

}  // namespace dhx
