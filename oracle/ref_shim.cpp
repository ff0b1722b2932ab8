// ref_shim.cpp -- C entry points over the compiled reference library.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile together with the
// reference's own sources (read in place under the reference checkout) into
// oracle/_ref/libsgref.so.  Used to pin the C restatement (sgq_oracle.c), to
// write the golden fixtures in tests/golden/, and as the "reference" CPU
// baseline timed by bench.py.  The product library never links it.
//
// Each function wraps one reference entry point unchanged:
//   ref_quantize_int8         quantization::quantize_int8   (src/quantization.cpp:11-78)
//   ref_dequantize_int8       quantization::dequantize_int8 (src/quantization.cpp:80-111)
//   ref_quantize_int4         quantization::quantize_int4   (src/quantization.cpp:113-159)
//   ref_dequantize_int4       quantization::dequantize_int4 (src/quantization.cpp:161-187)
//   ref_quantized_matmul_int8 quantization::quantized_matmul_int8 (src/quantization.cpp:189-197)
//   ref_quantized_matmul_int4 quantization::quantized_matmul_int4 (src/quantization.cpp:199-206)
//   ref_matmul                matmul (src/ops.cpp:378-455)
//   ref_silu                  silu   (src/ops.cpp:561-575)
//   ref_mul                   mul    (src/ops.cpp:239-253)
//   ref_rms_norm              rms_norm (src/ops.cpp:1532-1556)
//   ref_softmax               softmax over the last dimension (src/ops.cpp:2101-2140)
//   ref_embedding             embedding (src/ops.cpp:2624-2650)
//   ref_qllama_block_int4     LLaMABlock::forward (include/sovereigngrad/models.hpp:217-222)
//                             written out with QuantizedLinear4Bit projections
//   ref_save_qlinear          nn::QuantizedLinear(4Bit)::from_float (nn.hpp:946-954, 984-992), then
//                             serialization::save_module (src/serialization.cpp:103-105) or
//                             safetensors::save_module (src/safetensors.cpp:288-290)
//   ref_load_qlinear_forward  a fresh nn::QuantizedLinear(4Bit) (nn.hpp:935-944, 973-982) loaded
//                             with load_module (src/serialization.cpp:107-110,
//                             src/safetensors.cpp:292-295), then forward (nn.hpp:956-958, 994-996)
//   ref_save_entries          serialization::save_checkpoint / safetensors::save_file of raw tensors
//   ref_read_entry            serialization::load_checkpoint (src/serialization.cpp:49-101) or
//                             safetensors::load_file (src/safetensors.cpp:236-286), one entry
#include "sovereigngrad/nn.hpp"
#include "sovereigngrad/quantization.hpp"
#include "sovereigngrad/ops.hpp"
#include "sovereigngrad/safetensors.hpp"
#include "sovereigngrad/serialization.hpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

using namespace sovereigngrad;
using quantization::QuantizationScheme;
using quantization::QuantizedTensor;

namespace {

std::vector<int64_t> make_shape(int64_t rows, int64_t cols, int rank) {
    if (rank == 1) return {rows * cols};
    return {rows, cols};
}

Tensor from_host(const float* p, const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (auto d : shape) n *= d;
    std::vector<float> v(p, p + n);
    return Tensor(v, shape, Device::CPU, false);
}

void to_host(const Tensor& t, float* out) {
    Tensor c = t.to(Device::CPU).contiguous();
    std::memcpy(out, c.data(), sizeof(float) * (size_t)c.numel());
}

QuantizedTensor make_qt(const float* q, const float* scales, int64_t nscales, int64_t K, int64_t N,
                        int scheme, int64_t group_size, int bits) {
    QuantizedTensor qt;
    qt.qdata = from_host(q, {K, N});
    qt.scales = from_host(scales, {nscales});
    qt.scheme = static_cast<QuantizationScheme>(scheme);
    qt.original_shape = {K, N};
    qt.group_size = group_size;
    qt.bits = bits;
    return qt;
}

// A quantized linear layer of the reference, optionally registered under
// `child` in a parent module (so its state_dict keys read "child.qdata").
struct QLinearTree {
    std::shared_ptr<nn::Module> root;
};

QLinearTree wrap(std::shared_ptr<nn::Module> layer, const char* child) {
    if (!child || !*child) return QLinearTree{layer};
    auto parent = std::make_shared<nn::Module>();
    parent->register_module(child, layer);
    return QLinearTree{parent};
}

void save_tree(const nn::Module& m, int format, const char* path) {
    if (format == 0)
        serialization::save_module(m, path);
    else
        safetensors::save_module(m, path);
}

void load_tree(nn::Module& m, int format, const char* path) {
    if (format == 0)
        serialization::load_module(m, path, true);
    else
        safetensors::load_module(m, path, true);
}

}  // namespace

extern "C" {

// scheme: 0 PerTensorSymmetric, 1 PerChannelSymmetric (quantization.hpp:11-15).
// Writes qdata[rows*cols] and scales; returns the scale count, or -1 on error.
int64_t ref_quantize_int8(const float* x, int64_t rows, int64_t cols, int rank, int scheme, float* q,
                          float* scales) {
    try {
        Tensor t = from_host(x, make_shape(rows, cols, rank));
        QuantizedTensor qt = quantization::quantize_int8(t, static_cast<QuantizationScheme>(scheme));
        to_host(qt.qdata, q);
        to_host(qt.scales, scales);
        return qt.scales.numel();
    } catch (const std::exception&) {
        return -1;
    }
}

int64_t ref_quantize_int4(const float* x, int64_t rows, int64_t cols, int rank, int64_t group_size, float* q,
                          float* scales) {
    try {
        Tensor t = from_host(x, make_shape(rows, cols, rank));
        QuantizedTensor qt = quantization::quantize_int4(t, group_size);
        to_host(qt.qdata, q);
        to_host(qt.scales, scales);
        return qt.scales.numel();
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_dequantize_int8(const float* q, const float* scales, int64_t nscales, int64_t K, int64_t N, int scheme,
                        float* out) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, scheme, K * N, 8);
        to_host(quantization::dequantize_int8(qt), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_dequantize_int4(const float* q, const float* scales, int64_t nscales, int64_t K, int64_t N,
                        int64_t group_size, float* out) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, 2, group_size, 4);
        to_host(quantization::dequantize_int4(qt), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_quantized_matmul_int8(const float* x, int64_t M, int64_t K, int64_t N, const float* q, const float* scales,
                              int64_t nscales, int scheme, const float* bias, float* out) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, scheme, K * N, 8);
        Tensor tx = from_host(x, {M, K});
        Tensor tb = bias ? from_host(bias, {1, N}) : Tensor();
        to_host(quantization::quantized_matmul_int8(tx, qt, tb), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_quantized_matmul_int4(const float* x, int64_t M, int64_t K, int64_t N, const float* q, const float* scales,
                              int64_t nscales, int64_t group_size, const float* bias, float* out) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, 2, group_size, 4);
        Tensor tx = from_host(x, {M, K});
        Tensor tb = bias ? from_host(bias, {1, N}) : Tensor();
        to_host(quantization::quantized_matmul_int4(tx, qt, tb), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_matmul(const float* a, const float* b, int64_t M, int64_t K, int64_t N, float* out) {
    try {
        to_host(matmul(from_host(a, {M, K}), from_host(b, {K, N})), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Times `reps` calls of the reference forward (dequantize + matmul + bias) on
// tensors built once outside the timed region.  bits selects the INT8 or INT4
// entry point.  Writes per-call seconds into secs[reps]; returns 0 on success.
int ref_time_quantized_matmul(int bits, const float* x, int64_t M, int64_t K, int64_t N, const float* q,
                              const float* scales, int64_t nscales, int scheme, int64_t group_size,
                              const float* bias, int reps, double* secs, float* out) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, bits == 8 ? scheme : 2,
                                     bits == 8 ? K * N : group_size, bits);
        Tensor tx = from_host(x, {M, K});
        Tensor tb = bias ? from_host(bias, {1, N}) : Tensor();
        Tensor y;
        for (int r = 0; r < reps; ++r) {
            auto t0 = std::chrono::steady_clock::now();
            y = bits == 8 ? quantization::quantized_matmul_int8(tx, qt, tb)
                          : quantization::quantized_matmul_int4(tx, qt, tb);
            auto t1 = std::chrono::steady_clock::now();
            secs[r] = std::chrono::duration<double>(t1 - t0).count();
        }
        if (out) to_host(y, out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// The same forward split into its three phases as quantization.cpp:189-206
// runs them (dequantize, x.matmul(w), out + bias): writes per-call seconds
// of each phase into secs[3*r + 0..2].
int ref_time_phases(int bits, const float* x, int64_t M, int64_t K, int64_t N, const float* q, const float* scales,
                    int64_t nscales, int scheme, int64_t group_size, const float* bias, int reps, double* secs) {
    try {
        QuantizedTensor qt = make_qt(q, scales, nscales, K, N, bits == 8 ? scheme : 2,
                                     bits == 8 ? K * N : group_size, bits);
        Tensor tx = from_host(x, {M, K});
        Tensor tb = bias ? from_host(bias, {1, N}) : Tensor();
        for (int r = 0; r < reps; ++r) {
            auto t0 = std::chrono::steady_clock::now();
            Tensor w = bits == 8 ? quantization::dequantize_int8(qt) : quantization::dequantize_int4(qt);
            auto t1 = std::chrono::steady_clock::now();
            Tensor y = tx.matmul(w);
            auto t2 = std::chrono::steady_clock::now();
            if (tb.is_defined()) y = y + tb;
            auto t3 = std::chrono::steady_clock::now();
            secs[3 * r + 0] = std::chrono::duration<double>(t1 - t0).count();
            secs[3 * r + 1] = std::chrono::duration<double>(t2 - t1).count();
            secs[3 * r + 2] = std::chrono::duration<double>(t3 - t2).count();
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Sets the OpenMP thread count of later calls (the reference parallelises
// with OpenMP only); returns the previous maximum.
int ref_set_threads(int n) {
#ifdef _OPENMP
    const int prev = omp_get_max_threads();
    omp_set_num_threads(n);
    return prev;
#else
    (void)n;
    return 1;
#endif
}

int ref_silu(const float* x, int64_t n, float* out) {
    try {
        to_host(silu(from_host(x, {n})), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_mul(const float* a, const float* b, int64_t n, float* out) {
    try {
        to_host(mul(from_host(a, {n}), from_host(b, {n})), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_rms_norm(const float* x, int64_t B, int64_t D, const float* g, float eps, float* out) {
    try {
        to_host(rms_norm(from_host(x, {B, D}), from_host(g, {D}), eps), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_softmax(const float* x, int64_t R, int64_t C, float* out) {
    try {
        to_host(softmax(from_host(x, {R, C}), -1), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_embedding(const float* idx, int64_t n, const float* w, int64_t V, int64_t E, float* out) {
    try {
        to_host(embedding(from_host(idx, {n}), from_host(w, {V, E})), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// LLaMABlock::forward (models.hpp:217-222) on x[L, D], its attention
// (CausalSelfAttention::forward, nn.hpp:533-553, non-flash branch) and MLP
// (SwiGLU::forward, nn.hpp:151-156) written out statement by statement, each
// Linear replaced by QuantizedLinear4Bit::forward (nn.hpp:994-996), i.e.
// quantized_matmul_int4 with the module's [1, N] bias.  Projection p = 0..6:
// q, k, v, out, gate, up, down; bias[p] may be NULL (no bias add).
int ref_qllama_block_int4(const float* x, int64_t L, int64_t D, int64_t H, const float* const* codes,
                          const float* const* scales, const float* const* bias, const float* g1, const float* g2,
                          float eps, float attn_scale, int64_t group_size, float* out) {
    try {
        const int64_t K[7] = {D, D, D, D, D, D, H}, N[7] = {D, D, D, D, H, H, D};
        auto proj = [&](const Tensor& in, int p) {
            const int64_t G = group_size <= 0 ? 32 : group_size;
            QuantizedTensor qt = make_qt(codes[p], scales[p], (K[p] * N[p] + G - 1) / G, K[p], N[p], 2, G, 4);
            Tensor b = bias[p] ? from_host(bias[p], {1, N[p]}) : Tensor();
            return quantization::quantized_matmul_int4(in, qt, b);
        };
        Tensor tx = from_host(x, {L, D});
        Tensor tg1 = from_host(g1, {D}), tg2 = from_host(g2, {D});
        // attn->forward(norm1->forward(x))
        Tensor n1 = rms_norm(tx, tg1, eps);
        Tensor Q = proj(n1, 0), Kt = proj(n1, 1), V = proj(n1, 2);
        Tensor K_t = Kt.transpose(0, 1).contiguous();
        Tensor scores = Q.matmul(K_t) * attn_scale;
        Tensor mask = Tensor::triu({L, L}, 1, Device::CPU);
        scores = scores.masked_fill(mask, -1e9f);
        Tensor attn_weights = softmax(scores, -1);
        Tensor context = attn_weights.matmul(V);
        Tensor h = tx + proj(context, 3);
        // mlp->forward(norm2->forward(h))
        Tensor n2 = rms_norm(h, tg2, eps);
        Tensor gate = proj(n2, 4).silu();
        Tensor up = proj(n2, 5);
        Tensor hidden = gate * up;
        to_host(h + proj(hidden, 6), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Quantizes the fp32 weight W[K, N] with the reference's own module factory
// (bits 8: QuantizedLinear::from_float, per-channel; bits 4:
// QuantizedLinear4Bit::from_float with group_size), bias b[N] (or zeros), and
// saves the module -- or a parent module holding it as `child` -- as .sgrd
// (format 0) or .safetensors (format 1).  Returns 0, or -1 on error.
int ref_save_qlinear(int format, const char* path, int bits, const float* W, int64_t K, int64_t N,
                     int64_t group_size, const float* b, const char* child) {
    try {
        nn::Linear fl(K, N, Device::CPU);
        std::memcpy(fl.W.data(), W, sizeof(float) * (size_t)(K * N));
        if (b)
            std::memcpy(fl.b.data(), b, sizeof(float) * (size_t)N);
        else
            std::memset(fl.b.data(), 0, sizeof(float) * (size_t)N);
        std::shared_ptr<nn::Module> layer;
        if (bits == 8)
            layer = nn::QuantizedLinear::from_float(fl);
        else
            layer = nn::QuantizedLinear4Bit::from_float(fl, group_size);
        QLinearTree t = wrap(layer, child);
        save_tree(*t.root, format, path);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Builds a fresh reference module of the given shape (random weights), loads
// the file into it with the strict load_module, and runs its forward on
// x[M, K] into y[M, N]: the reference consuming a checkpoint written
// elsewhere.  Returns 0, or -1 on error (a missing key, a shape mismatch, a
// malformed file).
int ref_load_qlinear_forward(int format, const char* path, int bits, int64_t K, int64_t N, int64_t group_size,
                             const char* child, const float* x, int64_t M, float* y) {
    try {
        std::shared_ptr<nn::Module> layer;
        std::shared_ptr<nn::QuantizedLinear> q8;
        std::shared_ptr<nn::QuantizedLinear4Bit> q4;
        if (bits == 8)
            layer = q8 = std::make_shared<nn::QuantizedLinear>(K, N, Device::CPU);
        else
            layer = q4 = std::make_shared<nn::QuantizedLinear4Bit>(K, N, group_size, Device::CPU);
        QLinearTree t = wrap(layer, child);
        load_tree(*t.root, format, path);
        Tensor tx = from_host(x, {M, K});
        to_host(bits == 8 ? q8->forward(tx) : q4->forward(tx), y);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Reads one entry of a checkpoint with the reference's loader.  Writes up to
// cap floats into out and the shape into shape[8]/rank; returns the entry's
// element count, -2 when the name is absent, -1 on error.
int64_t ref_read_entry(int format, const char* path, const char* name, float* out, int64_t cap, int64_t* shape,
                       int* rank) {
    try {
        auto sd = format == 0 ? serialization::load_checkpoint(path) : safetensors::load_file(path);
        auto it = sd.find(name);
        if (it == sd.end()) return -2;
        const Tensor& t = it->second;
        *rank = (int)t.shape().size();
        for (int i = 0; i < *rank && i < 8; ++i) shape[i] = t.shape()[i];
        const int64_t n = t.numel();
        if (n <= cap) to_host(t, out);
        return n;
    } catch (const std::exception&) {
        return -1;
    }
}

// Saves n tensors (names[i], data[i] with shape shapes[i][0..ranks[i]-1])
// with serialization::save_checkpoint (format 0, src/serialization.cpp:14-47)
// or safetensors::save_file (format 1, src/safetensors.cpp:174-234).
int ref_save_entries(int format, const char* path, int n, const char* const* names, const float* const* data,
                     const int64_t* const* shapes, const int* ranks) {
    try {
        std::unordered_map<std::string, Tensor> sd;
        for (int i = 0; i < n; ++i) {
            std::vector<int64_t> shape(shapes[i], shapes[i] + ranks[i]);
            sd[names[i]] = from_host(data[i], shape);
        }
        if (format == 0)
            serialization::save_checkpoint(sd, path);
        else
            safetensors::save_file(sd, path);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Number of entries and their names, '\n'-separated, into names[cap].
int64_t ref_list_entries(int format, const char* path, char* names, int64_t cap) {
    try {
        auto sd = format == 0 ? serialization::load_checkpoint(path) : safetensors::load_file(path);
        std::string all;
        for (const auto& kv : sd) all += kv.first + "\n";
        if ((int64_t)all.size() + 1 > cap) return -1;
        std::memcpy(names, all.c_str(), all.size() + 1);
        return (int64_t)sd.size();
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
