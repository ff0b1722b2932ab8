// sgq_linear.hip -- fused dequantize + matmul kernels for gfx950:
//   y[M,N] = x[M,K] . (codes * scales) (+ bias)        fp32 accumulate
// which the reference computes as dequantize_int8/int4, then a blocked fp32
// matmul, then a bias add (src/quantization.cpp:189-206, src/ops.cpp:378-455,
// src/ops.cpp:132-171).
//
// Decode path (M <= 16): one wavefront streams one 1 KiB super-tile per
// 128-bit load (lane = chunk), unpacks codes in registers, folds the scale
// into the activation (xs = x * s, one multiply per row and lane) and
// accumulates code * xs with FMAs.  Lanes of the four bands are combined with
// cross-lane shuffles, the four waves of a workgroup through LDS, and the
// split-K workgroups of one column block by the last one to finish, which sums
// the partials in a fixed order (deterministic; no output pre-fill needed).
//
// Prefill path (M > 16): 128x128 output tiles, K staged through LDS 16 rows at
// a time; codes are dequantized on the way into LDS (code * scale, the
// reference's own product) and fed to v_mfma_f32_16x16x4_f32.
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kThreads = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of packed codes (read once; non-temporal hint).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte b of w read as a signed int8 and converted to fp32 in one VALU op
// (v_cvt_f32_i32 with an SDWA sign-extended byte select).  For INT4, a byte
// holding a code in its high nibble and zero below reads as 16*q exactly.
template <int B>
__device__ __forceinline__ float cvt_sbyte(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

__device__ __forceinline__ float i8_byte(uint32_t w, int b) {
    return b == 0 ? cvt_sbyte<0>(w) : (b == 1 ? cvt_sbyte<1>(w) : (b == 2 ? cvt_sbyte<2>(w) : cvt_sbyte<3>(w)));
}

// ---------------------------------------------------------------------------
// Shared epilogue of the GEMV kernels: wave results are in red[wave][m][col].
// Sums the four waves, then either writes y (ksplit == 1) or stores a partial
// and lets the last workgroup of the column block reduce all partials.
// ---------------------------------------------------------------------------
template <int MT, int TN>
__device__ __forceinline__ void gemv_finish(float (*red)[MT][TN], int M, int N, int n_base, int Npad, float post,
                                            const float* __restrict__ bias, float* __restrict__ y,
                                            float* __restrict__ part, unsigned* __restrict__ cnt, int cb, int ks,
                                            int ksplit, unsigned* s_last) {
    const int tid = threadIdx.x;
    if (ksplit == 1) {
        for (int o = tid; o < MT * TN; o += kThreads) {
            const int m = o / TN, i = o - m * TN;
            const int n = n_base + i;
            if (m < M && n < N) {
                float v = (red[0][m][i] + red[1][m][i]) + (red[2][m][i] + red[3][m][i]);
                v = v * post;
                if (bias) v = v + bias[n];
                y[(int64_t)m * N + n] = v;
            }
        }
        return;
    }
    for (int o = tid; o < MT * TN; o += kThreads) {
        const int m = o / TN, i = o - m * TN;
        if (m < M) {
            const float v = (red[0][m][i] + red[1][m][i]) + (red[2][m][i] + red[3][m][i]);
            part[((int64_t)ks * M + m) * Npad + n_base + i] = v;
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&cnt[cb], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        *s_last = (prev == (unsigned)(ksplit - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (*s_last == 0u) return;
    __threadfence();
    for (int o = tid; o < MT * TN; o += kThreads) {
        const int m = o / TN, i = o - m * TN;
        const int n = n_base + i;
        if (m < M && n < N) {
            float v = 0.0f;
            for (int s = 0; s < ksplit; ++s) v += part[((int64_t)s * M + m) * Npad + n];
            v = v * post;
            if (bias) v = v + bias[n];
            y[(int64_t)m * N + n] = v;
        }
    }
    if (tid == 0) __hip_atomic_store(&cnt[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads x[m][k0..k0+3] (zero past K and past M).
template <bool KALIGN4>
__device__ __forceinline__ float4 load_x4(const float* __restrict__ x, int m, int M, int K, int k0) {
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m >= M) return r;
    const float* p = x + (int64_t)m * K + k0;
    if (KALIGN4) {
        if (k0 < K) r = *(const float4*)p;
    } else {
        if (k0 + 0 < K) r.x = p[0];
        if (k0 + 1 < K) r.y = p[1];
        if (k0 + 2 < K) r.z = p[2];
        if (k0 + 3 < K) r.w = p[3];
    }
    return r;
}

__device__ __forceinline__ float f4get(const float4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// ---------------------------------------------------------------------------
// INT4 GEMV / skinny GEMM.  grid = NCB * ksplit workgroups of 256 threads.
// ---------------------------------------------------------------------------
template <int MT, bool KALIGN4>
__global__ __launch_bounds__(kThreads) void k_gemv_i4(const float* __restrict__ x, int M, int K, int N,
                                                      const uint4* __restrict__ W, const float* __restrict__ S,
                                                      int spc, int Kpad, int KT, const float* __restrict__ bias,
                                                      float* __restrict__ y, float* __restrict__ part,
                                                      unsigned* __restrict__ cnt, int ksplit, int tps) {
    __shared__ float red[4][MT][128];
    __shared__ unsigned s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cb = blockIdx.x / ksplit, ks = blockIdx.x - cb * ksplit;
    const int band = lane >> 4, strip = lane & 15;
    const int t0 = ks * tps;
    const int t1 = min(KT, t0 + tps);
    const float* __restrict__ Sc = S + (int64_t)((cb * 16 + strip) / spc) * Kpad;
    const uint4* __restrict__ Wb = W + (int64_t)cb * KT * 64 + lane;

    float acc[MT][8];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;

    constexpr int U = (MT <= 2) ? 4 : 2;
    for (int tb = t0 + wave; tb < t1; tb += 4 * U) {
        uint4 w[U];
        float4 s4[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + 4 * u;
            if (t < t1) {
                w[u] = load_stream(Wb + (int64_t)t * 64);
                s4[u] = *(const float4*)(Sc + t * 16 + band * 4);
            } else {
                w[u] = make_uint4(0u, 0u, 0u, 0u);
                s4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + 4 * u;
            if (t >= t1) break;
            const int k0 = t * 16 + band * 4;
            const uint32_t dw[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float4 xv = load_x4<KALIGN4>(x, m, M, K, k0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float xs = f4get(xv, r) * f4get(s4[u], r);
                    const uint32_t hi = dw[r] & 0xF0F0F0F0u;
                    const uint32_t lo = (dw[r] << 4) & 0xF0F0F0F0u;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        acc[m][2 * b] = fmaf(i8_byte(lo, b), xs, acc[m][2 * b]);
                        acc[m][2 * b + 1] = fmaf(i8_byte(hi, b), xs, acc[m][2 * b + 1]);
                    }
                }
            }
        }
    }

    // Combine the four bands (lanes l, l^16, l^32, l^48 share columns).
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[m][e];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[m][e] = v;
        }
    if (band == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int e = 0; e < 8; ++e) red[wave][m][strip * 8 + e] = acc[m][e];
    }
    __syncthreads();
    // Codes were read as 16*q: scale the sum back by 1/16 (exact).
    gemv_finish<MT, 128>(red, M, N, cb * 128, (int)round_up(N, kI4TileN), 0.0625f, bias, y, part, cnt, cb, ks,
                         ksplit, &s_last);
}

// ---------------------------------------------------------------------------
// INT8 GEMV / skinny GEMM.  Scales: per-tensor scales[0] or per-row scales[k].
// ---------------------------------------------------------------------------
template <int MT, bool KALIGN4>
__global__ __launch_bounds__(kThreads) void k_gemv_i8(const float* __restrict__ x, int M, int K, int N,
                                                      const uint4* __restrict__ W, const float* __restrict__ S,
                                                      int per_tensor, int KT, const float* __restrict__ bias,
                                                      float* __restrict__ y, float* __restrict__ part,
                                                      unsigned* __restrict__ cnt, int ksplit, int tps) {
    __shared__ float red[4][MT][64];
    __shared__ unsigned s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cb = blockIdx.x / ksplit, ks = blockIdx.x - cb * ksplit;
    const int band = lane >> 4, strip = lane & 15;
    const int t0 = ks * tps;
    const int t1 = min(KT, t0 + tps);
    const uint4* __restrict__ Wb = W + (int64_t)cb * KT * 64 + lane;
    const float s_all = per_tensor ? S[0] : 0.0f;

    float acc[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[m][d] = 0.0f;

    constexpr int U = (MT <= 2) ? 4 : 2;
    for (int tb = t0 + wave; tb < t1; tb += 4 * U) {
        uint4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + 4 * u;
            w[u] = (t < t1) ? load_stream(Wb + (int64_t)t * 64) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + 4 * u;
            if (t >= t1) break;
            const int k0 = t * 16 + band * 4;
            float s[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = per_tensor ? s_all : ((k0 + r < K) ? S[k0 + r] : 0.0f);
            const uint32_t dw[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float4 xv = load_x4<KALIGN4>(x, m, M, K, k0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float xs = f4get(xv, r) * s[r];
#pragma unroll
                    for (int d = 0; d < 4; ++d) acc[m][d] = fmaf(i8_byte(dw[d], r), xs, acc[m][d]);
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            float v = acc[m][d];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[m][d] = v;
        }
    if (band == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int d = 0; d < 4; ++d) red[wave][m][strip * 4 + d] = acc[m][d];
    }
    __syncthreads();
    gemv_finish<MT, 64>(red, M, N, cb * 64, (int)round_up(N, kI8TileN), 1.0f, bias, y, part, cnt, cb, ks, ksplit,
                        &s_last);
}

// ---------------------------------------------------------------------------
// MFMA GEMM: 128x128 tile per workgroup, four waves in 2x2, each 64x64 made of
// 4x4 blocks of v_mfma_f32_16x16x4_f32.  LDS holds A as [m][k] and the
// dequantized B as [n][k] (k contiguous), 16 k per stage, double buffered.
// Within a stage lane l supplies k = 4*(l/16) + kk to the kk-th MFMA, so one
// 128-bit LDS read per operand block feeds four MFMAs; A and B use the same
// k assignment, so every product pairs matching k.
// ---------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 16, kLdsStride = kBK + 4;

template <int BITS, bool KALIGN4>
__global__ __launch_bounds__(kThreads) void k_gemm(const float* __restrict__ x, int M, int K, int N,
                                                   const uint4* __restrict__ W, const float* __restrict__ S,
                                                   int mode, int Kpad, int KT, const float* __restrict__ bias,
                                                   float* __restrict__ y) {
    // mode: INT8 -> per_tensor flag; INT4 -> strips per scale column (spc).
    __shared__ __attribute__((aligned(16))) float As[2][kBM][kLdsStride];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBN][kLdsStride];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ntn = (N + kBN - 1) / kBN;
    const int tm = blockIdx.x / ntn, tn = blockIdx.x - tm * ntn;
    const int m0 = tm * kBM, n0 = tn * kBN;

    // ---- global -> register staging -------------------------------------
    float4 ra[2];
    uint4 rb;
    auto load_a = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kThreads * i;
            const int row = idx >> 2, kq = idx & 3;
            const int m = m0 + row, k = kt * kBK + kq * 4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < M) {
                const float* p = x + (int64_t)m * K + k;
                if (KALIGN4) {
                    if (k < K) v = *(const float4*)p;
                } else {
                    if (k + 0 < K) v.x = p[0];
                    if (k + 1 < K) v.y = p[1];
                    if (k + 2 < K) v.z = p[2];
                    if (k + 3 < K) v.w = p[3];
                }
            }
            ra[i] = v;
        }
    };
    // INT8: 128 columns = two 64-column blocks -> threads 0..127 take one chunk each.
    // INT4: 128 columns = one 128-column block -> threads 0..63 take one chunk each.
    constexpr int kBChunks = (BITS == 8) ? 128 : 64;
    auto load_b = [&](int kt) {
        if (tid < kBChunks) {
            const int cbl = tid >> 6, ch = tid & 63;
            const int64_t cb = (BITS == 8) ? (int64_t)(n0 / 64 + cbl) : (int64_t)(n0 / 128);
            // INT8 pads N to 64 only: the second half of the last tile may not exist.
            rb = (BITS == 4 || cb < (N + 63) / 64) ? W[(cb * KT + kt) * 64 + ch] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kThreads * i;
            const int row = idx >> 2, kq = idx & 3;
            *(float4*)&As[buf][row][kq * 4] = ra[i];
        }
    };
    auto store_b = [&](int buf, int kt) {
        if (tid >= kBChunks) return;
        const int ch = tid & 63, band = ch >> 4, strip = ch & 15;
        const int kl = band * 4;
        const int k = kt * kBK + kl;
        const uint32_t dw[4] = {rb.x, rb.y, rb.z, rb.w};
        if (BITS == 8) {
            float s[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = mode ? S[0] : ((k + r < K) ? S[k + r] : 0.0f);
            const int nl = (tid >> 6) * 64 + strip * 4;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                float4 v;
                v.x = i8_byte(dw[d], 0) * s[0];
                v.y = i8_byte(dw[d], 1) * s[1];
                v.z = i8_byte(dw[d], 2) * s[2];
                v.w = i8_byte(dw[d], 3) * s[3];
                *(float4*)&Bs[buf][nl + d][kl] = v;
            }
        } else {
            const float4 s = *(const float4*)(S + (int64_t)((n0 / 8 + strip) / mode) * Kpad + k);
            const int nl = strip * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float4 v;
                v.x = (float)(((int)(dw[0] << (28 - 4 * e))) >> 28) * s.x;
                v.y = (float)(((int)(dw[1] << (28 - 4 * e))) >> 28) * s.y;
                v.z = (float)(((int)(dw[2] << (28 - 4 * e))) >> 28) * s.z;
                v.w = (float)(((int)(dw[3] << (28 - 4 * e))) >> 28) * s.w;
                *(float4*)&Bs[buf][nl + e][kl] = v;
            }
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    load_a(0);
    load_b(0);
    store_a(0);
    store_b(0, 0);
    __syncthreads();

    const int lr = lane & 15, lk = (lane >> 4) * 4;
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        const bool more = (kt + 1 < KT);
        if (more) {
            load_a(kt + 1);
            load_b(kt + 1);
        }
        float4 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *(const float4*)&As[buf][wm * 64 + i * 16 + lr][lk];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *(const float4*)&Bs[buf][wn * 64 + j * 16 + lr][lk];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(a[i], kk), f4get(b[j], kk), acc[i][j],
                                                                     0, 0, 0);
        if (more) {
            store_a(buf ^ 1);
            store_b(buf ^ 1, kt + 1);
        }
        __syncthreads();
    }

    // D layout of 16x16x4: lane l, element r -> row 4*(l/16) + r, column l%16.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + lr;
            if (n >= N) continue;
            const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) {
                    const float v = acc[i][j][r];
                    y[(int64_t)m * N + n] = bias ? v + bv : v;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Generic INT4 forward over the flat layout (shapes the tiled layout cannot
// hold).  One thread per output; per-element scale index, the reference's own
// product code*scale, FMA accumulation in k order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_linear_i4_flat(const float* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t N, const unsigned char* __restrict__ P,
                                                             const float* __restrict__ S, int64_t G,
                                                             const float* __restrict__ bias, float* __restrict__ y) {
    for (int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; o < M * N;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = o / N, n = o - m * N;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const int64_t i = k * N + n;
            const uint32_t byte = P[i >> 1];
            const float q = (float)(((int)(byte << (28 - 4 * (int)(i & 1)))) >> 28);
            acc = fmaf(x[m * K + k], q * S[i / G], acc);
        }
        y[o] = bias ? acc + bias[n] : acc;
    }
}

template <int MT>
hipError_t gemv_i4_dispatch(const float* x, int M, int K, int N, const void* packed, const float* devscales,
                            const I4Geom& g, const float* bias, float* y, float* partial, unsigned* counters,
                            hipStream_t s) {
    const GemvPlan p = gemv_plan(g.KT, g.NCB);
    const dim3 grid((unsigned)(g.NCB * p.ksplit));
    if (K % 4 == 0 && (((uintptr_t)x) & 15) == 0)
        k_gemv_i4<MT, true><<<grid, kThreads, 0, s>>>(x, M, K, N, (const uint4*)packed, devscales, (int)g.spc,
                                                      (int)g.Kpad, (int)g.KT, bias, y, partial, counters, p.ksplit,
                                                      p.tps);
    else
        k_gemv_i4<MT, false><<<grid, kThreads, 0, s>>>(x, M, K, N, (const uint4*)packed, devscales, (int)g.spc,
                                                       (int)g.Kpad, (int)g.KT, bias, y, partial, counters,
                                                       p.ksplit, p.tps);
    return hipGetLastError();
}

template <int MT>
hipError_t gemv_i8_dispatch(const float* x, int M, int K, int N, const void* packed, const float* scales,
                            bool per_tensor, const float* bias, float* y, float* partial, unsigned* counters,
                            hipStream_t s) {
    I8Geom g(K, N);
    const GemvPlan p = gemv_plan(g.KT, g.NCB);
    const dim3 grid((unsigned)(g.NCB * p.ksplit));
    if (K % 4 == 0 && (((uintptr_t)x) & 15) == 0)
        k_gemv_i8<MT, true><<<grid, kThreads, 0, s>>>(x, M, K, N, (const uint4*)packed, scales, per_tensor ? 1 : 0,
                                                      (int)g.KT, bias, y, partial, counters, p.ksplit, p.tps);
    else
        k_gemv_i8<MT, false><<<grid, kThreads, 0, s>>>(x, M, K, N, (const uint4*)packed, scales,
                                                       per_tensor ? 1 : 0, (int)g.KT, bias, y, partial, counters,
                                                       p.ksplit, p.tps);
    return hipGetLastError();
}

}  // namespace

GemvPlan gemv_plan(int64_t KT, int64_t NCB) {
    // Aim for ~1024 workgroups (4 per CU) with at least 8 super-tiles
    // (two per wave) in every k-range.
    int64_t ksplit = 1024 / (NCB > 0 ? NCB : 1);
    int64_t max_split = KT / 8;
    if (ksplit > max_split) ksplit = max_split;
    if (ksplit < 1) ksplit = 1;
    int64_t tps = ceil_div(KT, ksplit);
    ksplit = ceil_div(KT, tps);  // drop empty ranges
    if (ksplit < 1) ksplit = 1;
    return GemvPlan{(int)ksplit, (int)tps};
}

hipError_t launch_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, float* partial,
                          unsigned* counters, hipStream_t s) {
    const int m = (int)M, k = (int)K, n = (int)N;
    if (M <= 1) return gemv_i4_dispatch<1>(x, m, k, n, packed, devscales, g, bias, y, partial, counters, s);
    if (M <= 2) return gemv_i4_dispatch<2>(x, m, k, n, packed, devscales, g, bias, y, partial, counters, s);
    if (M <= 4) return gemv_i4_dispatch<4>(x, m, k, n, packed, devscales, g, bias, y, partial, counters, s);
    if (M <= 8) return gemv_i4_dispatch<8>(x, m, k, n, packed, devscales, g, bias, y, partial, counters, s);
    return gemv_i4_dispatch<16>(x, m, k, n, packed, devscales, g, bias, y, partial, counters, s);
}

hipError_t launch_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, float* partial, unsigned* counters,
                          hipStream_t s) {
    const int m = (int)M, k = (int)K, n = (int)N;
    if (M <= 1) return gemv_i8_dispatch<1>(x, m, k, n, packed, scales, per_tensor, bias, y, partial, counters, s);
    if (M <= 2) return gemv_i8_dispatch<2>(x, m, k, n, packed, scales, per_tensor, bias, y, partial, counters, s);
    if (M <= 4) return gemv_i8_dispatch<4>(x, m, k, n, packed, scales, per_tensor, bias, y, partial, counters, s);
    if (M <= 8) return gemv_i8_dispatch<8>(x, m, k, n, packed, scales, per_tensor, bias, y, partial, counters, s);
    return gemv_i8_dispatch<16>(x, m, k, n, packed, scales, per_tensor, bias, y, partial, counters, s);
}

hipError_t launch_gemm_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, hipStream_t s) {
    I8Geom g(K, N);
    const dim3 grid((unsigned)(ceil_div(M, kBM) * ceil_div(N, kBN)));
    if (K % 4 == 0 && (((uintptr_t)x) & 15) == 0)
        k_gemm<8, true><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, scales,
                                                  per_tensor ? 1 : 0, (int)g.Kpad, (int)g.KT, bias, y);
    else
        k_gemm<8, false><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, scales,
                                                   per_tensor ? 1 : 0, (int)g.Kpad, (int)g.KT, bias, y);
    return hipGetLastError();
}

hipError_t launch_gemm_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, hipStream_t s) {
    const dim3 grid((unsigned)(ceil_div(M, kBM) * ceil_div(N, kBN)));
    if (K % 4 == 0 && (((uintptr_t)x) & 15) == 0)
        k_gemm<4, true><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, devscales,
                                                  (int)g.spc, (int)g.Kpad, (int)g.KT, bias, y);
    else
        k_gemm<4, false><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, devscales,
                                                   (int)g.spc, (int)g.Kpad, (int)g.KT, bias, y);
    return hipGetLastError();
}

hipError_t launch_linear_i4_flat(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                                 const float* scales, int64_t G, const float* bias, float* y, hipStream_t s) {
    int64_t blocks = ceil_div(M * N, kThreads);
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    k_linear_i4_flat<<<(unsigned)blocks, kThreads, 0, s>>>(x, M, K, N, (const unsigned char*)packed, scales, G,
                                                            bias, y);
    return hipGetLastError();
}

}  // namespace sgq
