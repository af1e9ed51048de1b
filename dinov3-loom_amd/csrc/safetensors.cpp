#include "safetensors.hpp"

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
            v.kind = Json::Number;
            const char* start = p_;
            bool integer = true;
            if (*p_ == '-') {
                integer = false;
                ++p_;
            }
            uint64_t acc = 0;
            while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                                 *p_ == '+' || *p_ == '-')) {
                if (*p_ >= '0' && *p_ <= '9') {
                    if (acc > (UINT64_MAX - 9) / 10) fail("number too large");
                    acc = acc * 10 + (uint64_t)(*p_ - '0');
                } else {
                    integer = false;
                }
                ++p_;
            }
            if (p_ == start) fail("bad number");
            v.integer = acc;
            v.is_integer = integer;
        } else {
            fail("unexpected character");
        }
        --depth_;
        return v;
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
                        if (end_ - p_ < 4) fail("bad unicode escape");
                        unsigned cp = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p_++;
                            cp <<= 4;
                            if (h >= '0' && h <= '9') cp |= h - '0';
                            else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                            else fail("bad unicode escape");
                        }
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xc0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3f));
                        } else {
                            out += (char)(0xe0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3f));
                            out += (char)(0x80 | (cp & 0x3f));
                        }
                        break;
                    }
                    default: fail("bad escape");
                }
            } else {
                out += *p_++;
            }
        }
        if (p_ >= end_) fail("unterminated string");
        ++p_;
        return out;
    }
};

uint64_t dtype_size(const std::string& d) {
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    throw Error("invalid safetensors header: unknown dtype " + d);
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

SafeTensors::SafeTensors(std::vector<uint8_t> file) : file_(std::move(file)) {
    if (file_.size() < 8) throw Error("invalid safetensors header: file too small");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | file_[i];
    if (n > 100u * 1024 * 1024 || n > file_.size() - 8) throw Error("invalid safetensors header: bad header length");
    const char* h = reinterpret_cast<const char*>(file_.data() + 8);
    Json doc = Parser(h, h + n).parse_document();
    if (doc.kind != Json::Object) throw Error("invalid safetensors header: not an object");
    const uint8_t* base = file_.data() + 8 + n;
    const uint64_t data_bytes = file_.size() - 8 - n;
    for (auto& kv : doc.members) {
        if (kv.first == "__metadata__") continue;
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
        const uint64_t esize = dtype_size(view.dtype);
        if (numel > UINT64_MAX / esize || numel * esize != e.integer - b.integer)
            throw Error("invalid safetensors header: size of " + kv.first);
        view.data = base + b.integer;
        view.bytes = e.integer - b.integer;
        tensors_[kv.first] = std::move(view);
    }
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
