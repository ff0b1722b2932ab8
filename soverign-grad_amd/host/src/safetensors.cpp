// safetensors.cpp -- SafeTensors read/write (interface of the reference's
// safetensors.hpp).  The format is the public one: u64 little-endian header
// length, a JSON object mapping names to {"dtype","shape","data_offsets"}
// (offsets relative to the end of the header), optional "__metadata__".
#include "sovereigngrad/safetensors.hpp"

#include <algorithm>
#include <cctype>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace sovereigngrad {
namespace safetensors {

namespace {

// Minimal JSON reader for the header: objects, arrays, strings, numbers,
// true/false/null.  Values other than the fields we need are skipped.
class HeaderParser {
public:
    explicit HeaderParser(const std::string& s) : s_(s) {}

    std::unordered_map<std::string, TensorMeta> parse() {
        std::unordered_map<std::string, TensorMeta> out;
        ws();
        expect('{');
        ws();
        if (peek() == '}') {
            ++i_;
            return out;
        }
        while (true) {
            ws();
            const std::string key = str();
            ws();
            expect(':');
            ws();
            if (key == "__metadata__") {
                skip_value();
            } else {
                out[key] = meta();
            }
            ws();
            if (peek() == ',') {
                ++i_;
                continue;
            }
            expect('}');
            break;
        }
        return out;
    }

private:
    const std::string& s_;
    size_t i_ = 0;

    [[noreturn]] void fail(const std::string& what) const {
        throw std::runtime_error("Malformed SafeTensors header: " + what + " at offset " + std::to_string(i_));
    }
    char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    void ws() {
        while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
    }
    void expect(char c) {
        if (peek() != c) fail(std::string("expected '") + c + "'");
        ++i_;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) fail("bad escape");
                const char e = s_[i_++];
                switch (e) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u':
                        if (i_ + 4 > s_.size()) fail("bad \\u escape");
                        i_ += 4;
                        out += '?';
                        break;
                    default: out += e;
                }
            } else {
                out += c;
            }
        }
        expect('"');
        return out;
    }
    int64_t integer() {
        size_t start = i_;
        if (peek() == '-') ++i_;
        while (std::isdigit(static_cast<unsigned char>(peek()))) ++i_;
        if (start == i_) fail("expected an integer");
        return std::stoll(s_.substr(start, i_ - start));
    }
    std::vector<int64_t> int_array() {
        std::vector<int64_t> out;
        expect('[');
        ws();
        if (peek() == ']') {
            ++i_;
            return out;
        }
        while (true) {
            ws();
            out.push_back(integer());
            ws();
            if (peek() == ',') {
                ++i_;
                continue;
            }
            expect(']');
            return out;
        }
    }
    void skip_value() {
        ws();
        const char c = peek();
        if (c == '"') {
            str();
        } else if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i_;
            ws();
            if (peek() == close) {
                ++i_;
                return;
            }
            while (true) {
                ws();
                if (c == '{') {
                    str();
                    ws();
                    expect(':');
                }
                skip_value();
                ws();
                if (peek() == ',') {
                    ++i_;
                    continue;
                }
                expect(close);
                return;
            }
        } else {
            while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']') ++i_;
        }
    }
    TensorMeta meta() {
        TensorMeta m;
        bool has_offsets = false;
        expect('{');
        while (true) {
            ws();
            const std::string field = str();
            ws();
            expect(':');
            ws();
            if (field == "dtype") {
                m.dtype = str();
            } else if (field == "shape") {
                m.shape = int_array();
            } else if (field == "data_offsets") {
                const auto o = int_array();
                if (o.size() != 2 || o[0] < 0 || o[1] < o[0]) fail("bad data_offsets");
                m.data_offset_start = (size_t)o[0];
                m.data_offset_end = (size_t)o[1];
                has_offsets = true;
            } else {
                skip_value();
            }
            ws();
            if (peek() == ',') {
                ++i_;
                continue;
            }
            expect('}');
            break;
        }
        if (m.dtype.empty() || !has_offsets) fail("tensor entry without dtype or data_offsets");
        return m;
    }
};

size_t dtype_size(const std::string& dt) {
    if (dt == "F32" || dt == "I32") return 4;
    if (dt == "F16") return 2;
    if (dt == "I64") return 8;
    throw std::runtime_error("Unsupported SafeTensors dtype: " + dt);
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            exp = 127 - 15 + 1;
            while ((man & 0x400) == 0) {
                man <<= 1;
                --exp;
            }
            man &= 0x3FF;
            bits = sign | (exp << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

std::pair<std::unordered_map<std::string, TensorMeta>, uint64_t> read_header(std::ifstream& in,
                                                                             const std::string& path) {
    uint64_t header_len = 0;
    in.read(reinterpret_cast<char*>(&header_len), sizeof(header_len));
    if (!in || header_len == 0 || header_len > (100ull << 20))
        throw std::runtime_error("Corrupted or invalid SafeTensors header size in: " + path);
    std::string json(header_len, '\0');
    in.read(&json[0], (std::streamsize)header_len);
    if (!in) throw std::runtime_error("Unexpected EOF while reading SafeTensors JSON header in: " + path);
    return {HeaderParser(json).parse(), header_len};
}

}  // namespace

void save_file(const std::unordered_map<std::string, Tensor>& sd, const std::string& filepath) {
    std::vector<std::string> names;
    for (const auto& kv : sd) names.push_back(kv.first);
    std::sort(names.begin(), names.end());
    std::ostringstream js;
    js << "{";
    size_t offset = 0;
    for (size_t i = 0; i < names.size(); ++i) {
        const Tensor& t = sd.at(names[i]);
        const size_t bytes = (size_t)t.numel() * 4;
        js << (i ? "," : "") << "\"" << names[i] << "\":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t d = 0; d < t.shape().size(); ++d) js << (d ? "," : "") << t.shape()[d];
        js << "],\"data_offsets\":[" << offset << "," << offset + bytes << "]}";
        offset += bytes;
    }
    js << "}";
    std::string header = js.str();
    while (header.size() % 8) header += ' ';  // keep the payload 8-byte aligned
    std::ofstream out(filepath, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Failed to open file for writing SafeTensors: " + filepath);
    const uint64_t len = header.size();
    out.write(reinterpret_cast<const char*>(&len), sizeof(len));
    out.write(header.data(), (std::streamsize)header.size());
    for (const auto& name : names) {
        const Tensor t = sd.at(name).cpu();
        out.write(reinterpret_cast<const char*>(t.data()), (std::streamsize)(t.numel() * 4));
    }
    if (!out) throw std::runtime_error("Failed while writing SafeTensors: " + filepath);
}

std::unordered_map<std::string, Tensor> load_file(const std::string& filepath, Device device) {
    std::ifstream in(filepath, std::ios::binary | std::ios::ate);
    if (!in.is_open()) throw std::runtime_error("Failed to open SafeTensors file: " + filepath);
    const uint64_t file_size = (uint64_t)in.tellg();
    in.seekg(0);
    auto [metas, header_len] = read_header(in, filepath);
    const uint64_t base = sizeof(uint64_t) + header_len;
    std::unordered_map<std::string, Tensor> sd;
    for (const auto& kv : metas) {
        const TensorMeta& m = kv.second;
        const size_t es = dtype_size(m.dtype);
        // Offsets inside the file and a payload of exactly numel elements,
        // checked before anything is allocated for the entry.
        if (m.data_offset_end > file_size - base)
            throw std::runtime_error("SafeTensors entry '" + kv.first + "' lies past the end of " + filepath);
        int64_t numel = -1;
        try {
            numel = compute_numel(m.shape);
        } catch (const std::exception&) {
        }
        if (numel < 0 || (uint64_t)numel > (file_size - base) / es ||
            m.data_offset_end - m.data_offset_start != (size_t)numel * es)
            throw std::runtime_error("SafeTensors entry '" + kv.first + "' has a payload size that does not match");
        std::vector<char> raw((size_t)numel * es);
        in.seekg((std::streamoff)(base + m.data_offset_start));
        in.read(raw.data(), (std::streamsize)raw.size());
        if (!in) throw std::runtime_error("Unexpected EOF in SafeTensors payload: " + filepath);
        Tensor t = Tensor::empty(m.shape, Device::CPU);
        float* dst = t.data();
        for (int64_t i = 0; i < numel; ++i) {
            if (m.dtype == "F32") {
                std::memcpy(dst + i, raw.data() + 4 * i, 4);
            } else if (m.dtype == "F16") {
                uint16_t h;
                std::memcpy(&h, raw.data() + 2 * i, 2);
                dst[i] = half_to_float(h);
            } else if (m.dtype == "I32") {
                int32_t v;
                std::memcpy(&v, raw.data() + 4 * i, 4);
                dst[i] = (float)v;
            } else {
                int64_t v;
                std::memcpy(&v, raw.data() + 8 * i, 8);
                dst[i] = (float)v;
            }
        }
        sd[kv.first] = device == Device::CPU ? t : t.to(device);
    }
    return sd;
}

void save_module(const nn::Module& module, const std::string& filepath) { save_file(module.state_dict(), filepath); }

void load_module(nn::Module& module, const std::string& filepath, bool strict) {
    module.load_state_dict(load_file(filepath), strict);
}

std::unordered_map<std::string, TensorMeta> inspect_file(const std::string& filepath) {
    std::ifstream in(filepath, std::ios::binary);
    if (!in.is_open()) throw std::runtime_error("Failed to open SafeTensors file: " + filepath);
    return read_header(in, filepath).first;
}

}  // namespace safetensors
}  // namespace sovereigngrad
