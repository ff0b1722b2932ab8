// serialization.cpp -- ".sgrd" checkpoints, byte format of
// src/serialization.cpp:11-101 (entries written in name order here; the
// reference writes hash order, and readers do not depend on it).
#include "sovereigngrad/serialization.hpp"

#include <algorithm>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <vector>

namespace sovereigngrad {
namespace serialization {

namespace {
const char kMagic[4] = {'S', 'G', 'R', 'D'};
constexpr uint32_t kVersion = 1;

template <typename T>
void put(std::ofstream& out, const T& v) {
    out.write(reinterpret_cast<const char*>(&v), sizeof(T));
}
template <typename T>
T get(std::ifstream& in, const std::string& path) {
    T v{};
    in.read(reinterpret_cast<char*>(&v), sizeof(T));
    if (!in) throw std::runtime_error("Unexpected end of checkpoint file: " + path);
    return v;
}
}  // namespace

void save_checkpoint(const std::unordered_map<std::string, Tensor>& sd, const std::string& filepath) {
    std::ofstream out(filepath, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Failed to open file for writing checkpoint: " + filepath);
    std::vector<std::string> names;
    for (const auto& kv : sd) names.push_back(kv.first);
    std::sort(names.begin(), names.end());
    out.write(kMagic, 4);
    put(out, kVersion);
    put(out, static_cast<uint32_t>(names.size()));
    for (const auto& name : names) {
        const Tensor t = sd.at(name).cpu();
        put(out, static_cast<uint32_t>(name.size()));
        out.write(name.data(), (std::streamsize)name.size());
        put(out, static_cast<uint32_t>(t.shape().size()));
        for (int64_t d : t.shape()) put(out, d);
        put(out, t.numel());
        out.write(reinterpret_cast<const char*>(t.data()), (std::streamsize)(t.numel() * sizeof(float)));
    }
    if (!out) throw std::runtime_error("Failed while writing checkpoint: " + filepath);
}

std::unordered_map<std::string, Tensor> load_checkpoint(const std::string& filepath, Device device) {
    std::ifstream in(filepath, std::ios::binary | std::ios::ate);
    if (!in.is_open()) throw std::runtime_error("Failed to open file for reading checkpoint: " + filepath);
    // Every length read from the file is checked against the bytes that are
    // left before anything is allocated for it: a corrupted or truncated file
    // is an error, never a huge allocation or a read past the end.
    const int64_t file_size = (int64_t)in.tellg();
    in.seekg(0);
    auto left = [&]() { return file_size - (int64_t)in.tellg(); };
    char magic[4] = {0, 0, 0, 0};
    in.read(magic, 4);
    if (!in || std::memcmp(magic, kMagic, 4) != 0)
        throw std::runtime_error("Invalid checkpoint file format or corrupted magic header in: " + filepath);
    const uint32_t version = get<uint32_t>(in, filepath);
    if (version != kVersion)
        throw std::runtime_error("Unsupported checkpoint format version: " + std::to_string(version));
    const uint32_t count = get<uint32_t>(in, filepath);
    std::unordered_map<std::string, Tensor> sd;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t name_len = get<uint32_t>(in, filepath);
        if ((int64_t)name_len > left()) throw std::runtime_error("Unexpected end of checkpoint file: " + filepath);
        std::string name(name_len, '\0');
        in.read(&name[0], name_len);
        const uint32_t rank = get<uint32_t>(in, filepath);
        if ((int64_t)rank * 8 + 8 > left()) throw std::runtime_error("Unexpected end of checkpoint file: " + filepath);
        std::vector<int64_t> shape(rank);
        for (auto& d : shape) d = get<int64_t>(in, filepath);
        const int64_t numel = get<int64_t>(in, filepath);
        int64_t expect = -1;
        try {
            expect = compute_numel(shape);
        } catch (const std::exception&) {
        }
        if (numel < 0 || numel != expect)
            throw std::runtime_error("Corrupted checkpoint entry '" + name + "': numel does not match shape");
        if (numel > left() / (int64_t)sizeof(float))
            throw std::runtime_error("Unexpected end of checkpoint file: " + filepath);
        Tensor t = Tensor::empty(shape, Device::CPU);
        in.read(reinterpret_cast<char*>(t.data()), (std::streamsize)(numel * sizeof(float)));
        if (!in) throw std::runtime_error("Unexpected end of checkpoint file: " + filepath);
        sd[name] = device == Device::CPU ? t : t.to(device);
    }
    return sd;
}

void save_module(const nn::Module& module, const std::string& filepath) { save_checkpoint(module.state_dict(), filepath); }

void load_module(nn::Module& module, const std::string& filepath, bool strict) {
    module.load_state_dict(load_checkpoint(filepath), strict);
}

}  // namespace serialization
}  // namespace sovereigngrad
