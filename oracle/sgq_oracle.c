/*
 * sgq_oracle.c -- CPU restatement of SovereignGrad's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU path is compared
 * against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library (libsgq.so) never links or calls it.
 *
 * Every function restates one piece of the reference, cited file:line
 * (paths relative to the reference checkout):
 *
 *   oracle_quantize_int8_per_tensor   src/quantization.cpp:22-41
 *   oracle_quantize_int8_per_channel  src/quantization.cpp:42-75
 *   oracle_dequantize_int8            src/quantization.cpp:80-111
 *   oracle_quantize_int4              src/quantization.cpp:113-159
 *   oracle_dequantize_int4            src/quantization.cpp:161-187
 *   oracle_matmul                     src/ops.cpp:378-455 with
 *                                     include/sovereigngrad/simd.hpp:152-221
 *   oracle_add_row_bias               src/ops.cpp:132-171
 *   oracle_quantized_matmul_int8      src/quantization.cpp:189-197
 *   oracle_quantized_matmul_int4      src/quantization.cpp:199-206
 *   oracle_silu                       src/ops.cpp:561-575 with
 *                                     include/sovereigngrad/simd.hpp:103-108
 *   oracle_mul                        src/ops.cpp:239-253 with
 *                                     include/sovereigngrad/simd.hpp:31-44
 *   oracle_swiglu_int8 / _int4        include/sovereigngrad/nn.hpp:151-154 (the
 *                                     gate/up half of SwiGLU::forward) on
 *                                     quantized weights
 *   oracle_rms_norm                   src/ops.cpp:1532-1556
 *   oracle_softmax_rows               src/ops.cpp:2101-2140 (last dimension)
 *   oracle_embedding                  src/ops.cpp:2624-2650
 *   oracle_causal_attention           include/sovereigngrad/nn.hpp:533-553 (the
 *                                     non-flash branch of CausalSelfAttention)
 *   oracle_qllama_block_int4          include/sovereigngrad/models.hpp:217-222
 *                                     (LLaMABlock::forward) with every
 *                                     projection a QuantizedLinear4Bit
 *                                     (nn.hpp:994-996)
 *
 * Floating-point contract.  The reference is built with GCC -O3 -mavx2 -mfma
 * in gnu++17 mode, where -ffp-contract=fast is the default, so every
 * `c += a * b` in its matmul becomes one fused multiply-add.  This file is
 * compiled with -ffp-contract=off and spells each fused operation out as
 * fmaf(); every other operation is a single IEEE op.  Parity of every function
 * here is pinned by tests/test_oracle.py against the compiled reference
 * (oracle/_ref) through the golden fixtures in tests/golden/, and by closed
 * forms and special cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* std::max(lo, std::min(hi, v)) exactly as <algorithm> defines them:
 * std::min(a, b) = (b < a) ? b : a;  std::max(a, b) = (a < b) ? b : a.
 * A NaN v therefore yields hi (src/quantization.cpp:37,69,152). */
static inline float ref_clamp(float v, float lo, float hi) {
    float m = (v < hi) ? v : hi;
    return (lo < m) ? m : lo;
}

/* max_abs starts at 1e-8f and is replaced only when fabs(x) > max_abs, so a
 * NaN never wins (src/quantization.cpp:23-27, 57-61, 140-144). */
static inline float ref_absmax(const float* x, int64_t n) {
    float m = 1e-8f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > m) m = a;
    }
    return m;
}

/* src/quantization.cpp:22-41 */
void oracle_quantize_int8_per_tensor(const float* x, int64_t total, float* q, float* scale_out) {
    float max_abs = ref_absmax(x, total);
    float scale = max_abs / 127.0f;
    float inv_scale = 127.0f / max_abs;
    for (int64_t i = 0; i < total; ++i) {
        float v = roundf(x[i] * inv_scale);
        q[i] = ref_clamp(v, -127.0f, 127.0f);
    }
    scale_out[0] = scale;
}

/* src/quantization.cpp:42-75: one scale per row r of x viewed as [rows, total/rows]. */
void oracle_quantize_int8_per_channel(const float* x, int64_t rows, int64_t cols, float* q, float* scales) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float max_abs = ref_absmax(xr, cols);
        float scale = max_abs / 127.0f;
        float inv_scale = 127.0f / max_abs;
        scales[r] = scale;
        for (int64_t c = 0; c < cols; ++c) {
            float v = roundf(xr[c] * inv_scale);
            q[r * cols + c] = ref_clamp(v, -127.0f, 127.0f);
        }
    }
}

/* src/quantization.cpp:80-111.  per_tensor mirrors the branch condition
 * `scheme == PerTensorSymmetric || scales.numel() == 1` (:90). */
void oracle_dequantize_int8(const float* q, const float* scales, int64_t rows, int64_t cols,
                            int per_tensor, float* out) {
    int64_t total = rows * cols;
    if (per_tensor) {
        float s = scales[0];
        for (int64_t i = 0; i < total; ++i) out[i] = q[i] * s;
    } else {
        for (int64_t r = 0; r < rows; ++r) {
            float s = scales[r];
            for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = q[r * cols + c] * s;
        }
    }
}

/* src/quantization.cpp:113-159: groups of group_size contiguous elements of
 * the flattened tensor; group_size <= 0 means 32 (:118); last group partial. */
int64_t oracle_int4_num_groups(int64_t total, int64_t group_size) {
    if (group_size <= 0) group_size = 32;
    return (total + group_size - 1) / group_size;
}

void oracle_quantize_int4(const float* x, int64_t total, int64_t group_size, float* q, float* scales) {
    if (group_size <= 0) group_size = 32;
    int64_t num_groups = (total + group_size - 1) / group_size;
    for (int64_t g = 0; g < num_groups; ++g) {
        int64_t g_start = g * group_size;
        int64_t g_end = g_start + group_size < total ? g_start + group_size : total;
        float max_abs = ref_absmax(x + g_start, g_end - g_start);
        float scale = max_abs / 7.0f;
        float inv_scale = 7.0f / max_abs;
        scales[g] = scale;
        for (int64_t i = g_start; i < g_end; ++i) {
            float v = roundf(x[i] * inv_scale);
            q[i] = ref_clamp(v, -8.0f, 7.0f);
        }
    }
}

/* src/quantization.cpp:161-187 */
void oracle_dequantize_int4(const float* q, const float* scales, int64_t total, int64_t group_size,
                            int64_t num_groups, float* out) {
    for (int64_t g = 0; g < num_groups; ++g) {
        int64_t g_start = g * group_size;
        int64_t g_end = g_start + group_size < total ? g_start + group_size : total;
        float s = scales[g];
        for (int64_t i = g_start; i < g_end; ++i) out[i] = q[i] * s;
    }
}

/* src/ops.cpp:378-455.  Output zero-filled (:393,:399); tiles of 32 rows x 64
 * columns, k-blocks of 128 visited in order (:401-403,:411-413).  Inside a
 * tile: full 8-row x 8-column blocks run the AVX2 micro-kernel, which loads
 * C, adds one fused multiply-add per k in order and stores C back
 * (simd.hpp:152-221); the column tail of an 8-row group sums its k-block into
 * a zero-started local accumulator (contracted to FMA) and then adds it to C
 * with a plain add (:426-434); rows left over after the 8-row groups take
 * `c += a*b` per k in order, contracted to FMA (:436-443).  Tiles are
 * independent, so the OpenMP schedule does not change any result. */
void oracle_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N) {
    const int64_t BLOCK_M = 32, BLOCK_N = 64, BLOCK_K = 128;
    memset(C, 0, (size_t)(M * N) * sizeof(float));
    for (int64_t i0 = 0; i0 < M; i0 += BLOCK_M) {
        for (int64_t j0 = 0; j0 < N; j0 += BLOCK_N) {
            int64_t i_max = i0 + BLOCK_M < M ? i0 + BLOCK_M : M;
            int64_t j_max = j0 + BLOCK_N < N ? j0 + BLOCK_N : N;
            for (int64_t k0 = 0; k0 < K; k0 += BLOCK_K) {
                int64_t k_max = k0 + BLOCK_K < K ? k0 + BLOCK_K : K;
                int64_t i = i0;
                for (; i + 8 <= i_max; i += 8) {
                    int64_t j = j0;
                    for (; j + 8 <= j_max; j += 8) {
                        for (int64_t r = 0; r < 8; ++r) {
                            for (int64_t c = 0; c < 8; ++c) {
                                float acc = C[(i + r) * N + j + c];
                                for (int64_t k = k0; k < k_max; ++k)
                                    acc = fmaf(A[(i + r) * K + k], B[k * N + j + c], acc);
                                C[(i + r) * N + j + c] = acc;
                            }
                        }
                    }
                    for (; j < j_max; ++j) {
                        for (int64_t r = 0; r < 8; ++r) {
                            float acc = 0.0f;
                            for (int64_t k = k0; k < k_max; ++k)
                                acc = fmaf(A[(i + r) * K + k], B[k * N + j], acc);
                            C[(i + r) * N + j] += acc;
                        }
                    }
                }
                for (; i < i_max; ++i) {
                    for (int64_t k = k0; k < k_max; ++k) {
                        float a_ik = A[i * K + k];
                        for (int64_t j = j0; j < j_max; ++j)
                            C[i * N + j] = fmaf(a_ik, B[k * N + j], C[i * N + j]);
                    }
                }
            }
        }
    }
}

/* src/ops.cpp:132-171 for out[M,N] + bias[1,N]: the broadcast branch computes
 * va + vb per element (:149-165); the equal-shape branch (M == 1) is
 * simd::vec_add, the same single addition per element (simd.hpp:15-28). */
void oracle_add_row_bias(float* out, const float* bias, int64_t M, int64_t N) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) out[i * N + j] = out[i * N + j] + bias[j];
}

/* src/quantization.cpp:189-197: dequantize, matmul, optional bias. */
void oracle_quantized_matmul_int8(const float* x, int64_t M, int64_t K, int64_t N, const float* q,
                                  const float* scales, int per_tensor, const float* bias, float* out) {
    float* w = (float*)malloc((size_t)(K * N > 0 ? K * N : 1) * sizeof(float));
    oracle_dequantize_int8(q, scales, K, N, per_tensor, w);
    oracle_matmul(x, w, out, M, K, N);
    if (bias) oracle_add_row_bias(out, bias, M, N);
    free(w);
}

/* src/quantization.cpp:199-206 */
void oracle_quantized_matmul_int4(const float* x, int64_t M, int64_t K, int64_t N, const float* q,
                                  const float* scales, int64_t group_size, const float* bias, float* out) {
    if (group_size <= 0) group_size = 32;
    int64_t total = K * N;
    float* w = (float*)malloc((size_t)(total > 0 ? total : 1) * sizeof(float));
    oracle_dequantize_int4(q, scales, total, group_size, oracle_int4_num_groups(total, group_size), w);
    oracle_matmul(x, w, out, M, K, N);
    if (bias) oracle_add_row_bias(out, bias, M, N);
    free(w);
}

/* simd::vec_silu (simd.hpp:103-108), the CPU branch of silu (ops.cpp:561-575):
 * x / (1 + exp(-x)) with std::exp on float, i.e. libm's expf, one element at a
 * time (the loop calls a library function, so GCC keeps it scalar). */
void oracle_silu(const float* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        out[i] = v / (1.0f + expf(-v));
    }
}

/* mul (ops.cpp:239-253) for equal contiguous shapes: simd::vec_mul
 * (simd.hpp:31-44), one IEEE multiply per element. */
void oracle_mul(const float* a, const float* b, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* SwiGLU::forward up to the down projection (nn.hpp:151-154):
 *   gate = silu(w_gate(x)); up = w_up(x); hidden = gate * up
 * with both projections quantized linears (bias may be NULL). */
static void swiglu_finish(float* gate, const float* up, int64_t n, float* out) {
    oracle_silu(gate, n, gate);
    oracle_mul(gate, up, n, out);
}

void oracle_swiglu_int8(const float* x, int64_t M, int64_t K, int64_t N, const float* qg, const float* sg,
                        const float* bg, const float* qu, const float* su, const float* bu, int per_tensor,
                        float* out) {
    const size_t n = (size_t)(M * N > 0 ? M * N : 1);
    float* gate = (float*)malloc(n * sizeof(float));
    float* up = (float*)malloc(n * sizeof(float));
    oracle_quantized_matmul_int8(x, M, K, N, qg, sg, per_tensor, bg, gate);
    oracle_quantized_matmul_int8(x, M, K, N, qu, su, per_tensor, bu, up);
    swiglu_finish(gate, up, M * N, out);
    free(gate);
    free(up);
}

void oracle_swiglu_int4(const float* x, int64_t M, int64_t K, int64_t N, const float* qg, const float* sg,
                        const float* bg, const float* qu, const float* su, const float* bu, int64_t group_size,
                        float* out) {
    const size_t n = (size_t)(M * N > 0 ? M * N : 1);
    float* gate = (float*)malloc(n * sizeof(float));
    float* up = (float*)malloc(n * sizeof(float));
    oracle_quantized_matmul_int4(x, M, K, N, qg, sg, group_size, bg, gate);
    oracle_quantized_matmul_int4(x, M, K, N, qu, su, group_size, bu, up);
    swiglu_finish(gate, up, M * N, out);
    free(gate);
    free(up);
}

/* rms_norm, CPU branch (src/ops.cpp:1532-1556), rows of [B, D]:
 * inv_rms = 1 / sqrt(sum_sq / D + eps) with IEEE divide and sqrt, and
 * out = x * inv_rms * g as two multiplies, left to right.
 *
 * sum_sq is `sum_sq += v * v` over d in order.  With the reference's flags
 * (-O3 -mavx2 -mfma, no fast-math) GCC vectorises this loop as an in-order
 * reduction: whole blocks of 8, then one block of 4 if at least 4 remain, take
 * the products as separate multiplies and add them one at a time in order;
 * the last 0-3 elements run the scalar loop, which is contracted to FMA.  The
 * golden fixtures pin this against the compiled reference. */
static float rms_sum_squares(const float* x, int64_t D) {
    float ss = 0.0f;
    int64_t d = 0;
    if (D >= 8)
        for (; d + 8 <= D; d += 8)
            for (int64_t l = 0; l < 8; ++l) ss = ss + x[d + l] * x[d + l];
    if (D - d >= 4) {
        for (int64_t l = 0; l < 4; ++l) ss = ss + x[d + l] * x[d + l];
        d += 4;
    }
    for (; d < D; ++d) ss = fmaf(x[d], x[d], ss);
    return ss;
}

void oracle_rms_norm(const float* x, int64_t B, int64_t D, const float* g, float eps, float* out) {
    for (int64_t i = 0; i < B; ++i) {
        const float* xi = x + i * D;
        const float inv = 1.0f / sqrtf(rms_sum_squares(xi, D) / (float)D + eps);
        for (int64_t d = 0; d < D; ++d) out[i * D + d] = (xi[d] * inv) * g[d];
    }
}

/* softmax over the last dimension (src/ops.cpp:2101-2140 with inner_size 1):
 * the maximum starts at element 0 and is replaced on `>`; the sum of
 * exp(x - max) runs in order; out = exp(x - max) / sum, exp being libm's expf. */
void oracle_softmax_rows(const float* x, int64_t R, int64_t C, float* out) {
    for (int64_t r = 0; r < R; ++r) {
        const float* xr = x + r * C;
        float mx = xr[0];
        for (int64_t d = 1; d < C; ++d)
            if (xr[d] > mx) mx = xr[d];
        float sum = 0.0f;
        for (int64_t d = 0; d < C; ++d) sum += expf(xr[d] - mx);
        for (int64_t d = 0; d < C; ++d) out[r * C + d] = expf(xr[d] - mx) / sum;
    }
}

/* embedding (src/ops.cpp:2624-2650): token id = (int)index (truncation); ids
 * outside [0, V) give a zero row. */
void oracle_embedding(const float* idx, int64_t n, const float* w, int64_t V, int64_t E, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const int id = (int)idx[i];
        if (id >= 0 && id < V)
            memcpy(out + i * E, w + (int64_t)id * E, (size_t)E * sizeof(float));
        else
            memset(out + i * E, 0, (size_t)E * sizeof(float));
    }
}

/* CausalSelfAttention::forward after the projections (nn.hpp:545-552):
 * scores = Q . K^T (the reference matmul on the contiguous transpose), times
 * scale (one multiply each), masked_fill of the strict upper triangle
 * (Tensor::triu(..., 1), tensor.cpp:205-222) with -1e9, softmax over the last
 * dimension, then weights . V.  One attention over the full width D. */
void oracle_causal_attention(const float* Q, const float* K, const float* V, int64_t L, int64_t D, float scale,
                             float* ctx) {
    const size_t ll = (size_t)(L * L > 0 ? L * L : 1);
    float* kt = (float*)calloc((size_t)(L * D > 0 ? L * D : 1), sizeof(float));
    float* sc = (float*)malloc(ll * sizeof(float));
    float* w = (float*)malloc(ll * sizeof(float));
    for (int64_t j = 0; j < L; ++j)
        for (int64_t d = 0; d < D; ++d) kt[d * L + j] = K[j * D + d];
    oracle_matmul(Q, kt, sc, L, D, L);
    for (int64_t r = 0; r < L; ++r)
        for (int64_t c = 0; c < L; ++c) {
            const float v = sc[r * L + c] * scale;
            sc[r * L + c] = (c >= r + 1) ? -1e9f : v;
        }
    oracle_softmax_rows(sc, L, L, w);
    oracle_matmul(w, V, ctx, L, L, D);
    free(kt);
    free(sc);
    free(w);
}

/* LLaMABlock::forward (models.hpp:217-222) on x[L, D] with every projection a
 * QuantizedLinear4Bit (quantized_matmul_int4 with its [1, N] bias):
 *   h   = x + out_proj(attention(q_proj(n1), k_proj(n1), v_proj(n1))),  n1 = rms_norm(x, g1)
 *   out = h + w_down(silu(w_gate(n2)) * w_up(n2)),                      n2 = rms_norm(h, g2)
 * Projections p = 0..6 are q, k, v, out ([D, D]), gate, up ([D, H]) and down
 * ([H, D]); codes[p] are fp32 INT4 codes in the weight's [K, N] shape,
 * scales[p] their group scales, bias[p] a row of N floats or NULL.  The two
 * residual adds are equal-shape vec_add (one addition per element). */
void oracle_qllama_block_int4(const float* x, int64_t L, int64_t D, int64_t H, const float* const* codes,
                              const float* const* scales, const float* const* bias, const float* g1,
                              const float* g2, float eps, float attn_scale, int64_t group_size, float* out) {
    const size_t ld = (size_t)(L * D > 0 ? L * D : 1), lh = (size_t)(L * H > 0 ? L * H : 1);
    float* n1 = (float*)malloc(ld * sizeof(float));
    float* q = (float*)malloc(ld * sizeof(float));
    float* k = (float*)malloc(ld * sizeof(float));
    float* v = (float*)malloc(ld * sizeof(float));
    float* ctx = (float*)malloc(ld * sizeof(float));
    float* h = (float*)malloc(ld * sizeof(float));
    float* gate = (float*)malloc(lh * sizeof(float));
    float* up = (float*)malloc(lh * sizeof(float));
    oracle_rms_norm(x, L, D, g1, eps, n1);
    oracle_quantized_matmul_int4(n1, L, D, D, codes[0], scales[0], group_size, bias[0], q);
    oracle_quantized_matmul_int4(n1, L, D, D, codes[1], scales[1], group_size, bias[1], k);
    oracle_quantized_matmul_int4(n1, L, D, D, codes[2], scales[2], group_size, bias[2], v);
    oracle_causal_attention(q, k, v, L, D, attn_scale, ctx);
    oracle_quantized_matmul_int4(ctx, L, D, D, codes[3], scales[3], group_size, bias[3], h);
    for (int64_t i = 0; i < L * D; ++i) h[i] = x[i] + h[i];
    oracle_rms_norm(h, L, D, g2, eps, n1);
    oracle_quantized_matmul_int4(n1, L, D, H, codes[4], scales[4], group_size, bias[4], gate);
    oracle_quantized_matmul_int4(n1, L, D, H, codes[5], scales[5], group_size, bias[5], up);
    swiglu_finish(gate, up, L * H, gate);
    oracle_quantized_matmul_int4(gate, L, H, D, codes[6], scales[6], group_size, bias[6], out);
    for (int64_t i = 0; i < L * D; ++i) out[i] = h[i] + out[i];
    free(n1);
    free(q);
    free(k);
    free(v);
    free(ctx);
    free(h);
    free(gate);
    free(up);
}

/* fp64 reference dot products for tolerance pinning: out[m,n] = sum_k x[m,k]*w[k,n]
 * in double, plus the magnitude sum_k |x||w| used for error floors. */
void oracle_matmul_f64(const float* A, const float* B, double* C, double* Cabs, int64_t M, int64_t K, int64_t N) {
    for (int64_t i = 0; i < M; ++i) {
        for (int64_t j = 0; j < N; ++j) { C[i * N + j] = 0.0; Cabs[i * N + j] = 0.0; }
        for (int64_t k = 0; k < K; ++k) {
            double a = A[i * K + k];
            for (int64_t j = 0; j < N; ++j) {
                double b = B[k * N + j];
                C[i * N + j] += a * b;
                Cabs[i * N + j] += fabs(a * b);
            }
        }
    }
}
