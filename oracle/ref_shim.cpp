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
#include "sovereigngrad/quantization.hpp"
#include "sovereigngrad/ops.hpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
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

int ref_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
