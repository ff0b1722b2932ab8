// sgq_quant.hip -- quantize / pack / unpack / dequantize kernels for gfx950.
//
// Bit-exactness contract with the reference quantizer (src/quantization.cpp):
//   max_abs  starts at 1e-8f and takes |x| only when |x| > max_abs, so NaN never
//            wins (:23-27, :57-61, :140-144).  A maximum is order-independent,
//            so the parallel reductions below give the serial loop's value.
//   scale    = max_abs / qmax and inv = qmax / max_abs, two correctly rounded
//            IEEE divisions (:29-30, :63-64, :146-147).
//   code     = max(lo, min(hi, round(x * inv))) with round half away from zero
//            and std::min/std::max operand order, so NaN gives hi (:36-37, :68-69, :151-152).
// Nothing in this file may be contracted into FMAs.
#include "sgq_internal.h"

#pragma clang fp contract(off)

namespace sgq {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float ref_code(float x, float inv, float lo, float hi) {
    float v = roundf(x * inv);
    float m = (v < hi) ? v : hi;  // std::min(hi, v)
    return (lo < m) ? m : lo;     // std::max(lo, m)
}

__device__ __forceinline__ float ref_max(float m, float a) { return (a > m) ? a : m; }

__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = ref_max(m, __shfl_xor(m, off));
    return m;
}

__device__ __forceinline__ bool valid_code(float v, float lo, float hi) {
    return v == truncf(v) && v >= lo && v <= hi;  // false for NaN and +-inf
}

__global__ void k_fill_zero(uint4* __restrict__ p, int64_t n16, unsigned char* __restrict__ tail, int ntail) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n16; i += stride) p[i] = make_uint4(0u, 0u, 0u, 0u);
    if (blockIdx.x == 0 && (int)threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

__global__ void k_fill_bias(float* __restrict__ y, int64_t M, int64_t N, const float* __restrict__ bias) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < M * N; i += stride) y[i] = bias ? bias[i % N] : 0.0f;
}

// One wavefront per group of G consecutive elements.
__global__ void k_group_scales(const float* __restrict__ x, int64_t total, int64_t G, int64_t ngroups, float qmax,
                               float* __restrict__ scales, float* __restrict__ inv) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t g = wave; g < ngroups; g += nwaves) {
        const int64_t b = g * G;
        const int64_t e = (b + G < total) ? b + G : total;
        float m = 1e-8f;
        for (int64_t i = b + lane; i < e; i += 64) m = ref_max(m, fabsf(x[i]));
        m = wave_max(m);
        if (lane == 0) {
            scales[g] = m / qmax;
            if (inv) inv[g] = qmax / m;
        }
    }
}

__global__ void k_absmax_partial(const float* __restrict__ x, int64_t total, float* __restrict__ partial) {
    __shared__ float sm[kBlock / 64];
    float m = 1e-8f;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < total; i += stride) m = ref_max(m, fabsf(x[i]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = sm[0];
        for (int w = 1; w < kBlock / 64; ++w) r = ref_max(r, sm[w]);
        partial[blockIdx.x] = r;
    }
}

// INT8 strip-major pack: one thread per 16-byte chunk (4 columns x 4 rows).
__global__ void k_pack_i8_tiled(const float* __restrict__ src, int from_codes, int64_t K, int64_t N, int64_t RQ,
                                int64_t NS, int64_t nchunks, const float* __restrict__ inv, int per_tensor,
                                uint4* __restrict__ packed, float* __restrict__ qdata, int* __restrict__ bad) {
    for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < nchunks;
         c += (int64_t)gridDim.x * blockDim.x) {
    // Consecutive threads take consecutive strips of the same rows, so the
    // reads of x (or qdata) are coalesced; each thread writes chunk j*RQ + rq.
    const int64_t rq = c / NS, j = c - rq * NS;
    const int64_t k0 = rq * 4;
    const int64_t n0 = j * 4;
    uint32_t dw[4];
    int badflag = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int64_t n = n0 + d;
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t k = k0 + r;
            int code = 0;
            if (k < K && n < N) {
                float v;
                if (from_codes) {
                    v = src[k * N + n];
                    if (!valid_code(v, -128.0f, 127.0f)) {
                        badflag = 1;
                        v = 0.0f;
                    }
                } else {
                    v = ref_code(src[k * N + n], per_tensor ? inv[0] : inv[k], -127.0f, 127.0f);
                    if (qdata) qdata[k * N + n] = v;
                }
                code = (int)v;
            }
            word |= ((uint32_t)code & 0xFFu) << (8 * r);
        }
        dw[d] = word;
    }
    if (packed) packed[j * RQ + rq] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    if (badflag) atomicOr(bad, 1);
    }
}

// INT4 strip-major pack: one thread per 16-byte chunk (4 rows x 8 columns).
__global__ void k_pack_i4_tiled(const float* __restrict__ src, int from_codes, int64_t K, int64_t N, int64_t G,
                                int64_t RQ, int64_t NS, int64_t nchunks, const float* __restrict__ inv,
                                uint4* __restrict__ packed, float* __restrict__ qdata, int* __restrict__ bad) {
    for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < nchunks;
         c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rq = c / NS, j = c - rq * NS;
    const int64_t k0 = rq * 4;
    const int64_t n0 = j * 8;
    uint32_t dw[4];
    int badflag = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t k = k0 + r;
        uint32_t word = 0;
        if (k < K) {
            // The strip layout requires N % 8 == 0 and G % 8 == 0, so the 8
            // columns of this row of the strip lie in one group.
            const int64_t i0 = k * N + n0;
            const float iv = from_codes ? 0.0f : inv[i0 / G];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t i = i0 + e;
                float v;
                if (from_codes) {
                    v = src[i];
                    if (!valid_code(v, -8.0f, 7.0f)) {
                        badflag = 1;
                        v = 0.0f;
                    }
                } else {
                    v = ref_code(src[i], iv, -8.0f, 7.0f);
                    if (qdata) qdata[i] = v;
                }
                word |= ((uint32_t)(int)v & 0xFu) << (4 * e);
            }
        }
        dw[r] = word;
    }
    if (packed) packed[j * RQ + rq] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    if (badflag) atomicOr(bad, 1);
    }
}

// The k-octet copy of an INT4 strip-major weight, built from its strips: one
// thread per dword t of block (cb, kb), column 16 cb + (t & 15), rows
// 32 kb + 8 (t >> 4) .. + 7 in nibbles 0..7.  Strip dword (j, row k) is dword
// 4 * (j * RQ + k / 4) + k % 4, column n of it nibble n % 8.  The first ngap
// threads also zero the ngap dwords between the strips and the copy, so that
// the whole buffer is a function of the codes.
__global__ void k_koct_i4(const uint32_t* __restrict__ strips, int64_t N, int64_t Kpad, int64_t RQ, int64_t KB,
                          int64_t ndw, uint32_t* __restrict__ koct, uint32_t* __restrict__ gap, int ngap) {
    const int64_t t0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t0 < ngap) gap[t0] = 0u;
    for (int64_t d = t0; d < ndw; d += (int64_t)gridDim.x * blockDim.x) {
        const int64_t blk = d >> 6, t = d & 63;
        const int64_t cb = blk / KB, kb = blk - cb * KB;
        const int64_t n = 16 * cb + (t & 15), j = n >> 3;
        const int e = (int)(n & 7);
        const int64_t k0 = 32 * kb + 8 * (t >> 4);
        uint32_t word = 0;
        if (n < N) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t k = k0 + i;
                if (k < Kpad) word |= ((strips[4 * (j * RQ + (k >> 2)) + (k & 3)] >> (4 * e)) & 0xFu) << (4 * i);
            }
        }
        koct[d] = word;
    }
}

// INT4 flat pack: one thread per byte (elements 2b, 2b+1 of the flattened tensor).
__global__ void k_pack_i4_flat(const float* __restrict__ src, int from_codes, int64_t total, int64_t G,
                               const float* __restrict__ inv, unsigned char* __restrict__ packed,
                               float* __restrict__ qdata, int* __restrict__ bad) {
    for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; 2 * b < total;
         b += (int64_t)gridDim.x * blockDim.x) {
    uint32_t byte = 0;
    int badflag = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t i = 2 * b + h;
        if (i >= total) break;
        float v;
        if (from_codes) {
            v = src[i];
            if (!valid_code(v, -8.0f, 7.0f)) {
                badflag = 1;
                v = 0.0f;
            }
        } else {
            v = ref_code(src[i], inv[i / G], -8.0f, 7.0f);
            if (qdata) qdata[i] = v;
        }
        byte |= ((uint32_t)(int)v & 0xFu) << (4 * h);
    }
    if (packed) packed[b] = (unsigned char)byte;
    if (badflag) atomicOr(bad, 1);
    }
}

// devscales[sc][k] = scale of the first strip of scale column sc in row k.
__global__ void k_devscales_i4(const float* __restrict__ scales, int64_t K, int64_t N, int64_t G, int64_t Kpad,
                               int64_t spc, int64_t nsc, float* __restrict__ devscales) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nsc * Kpad;
         i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t sc = i / Kpad, k = i - sc * Kpad;
    const int64_t n = sc * spc * 8;
    devscales[i] = (k < K && n < N) ? scales[(k * N + n) / G] : 0.0f;
    }
}

__global__ void k_unpack_i8_tiled(const uint4* __restrict__ packed, int64_t K, int64_t N, int64_t RQ,
                                  int64_t NS, int64_t nchunks, const float* __restrict__ scales, int per_tensor,
                                  float* __restrict__ out) {
    for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < nchunks;
         c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rq = c / NS, j = c - rq * NS;  // strip fastest: coalesced writes of out
    const int64_t k0 = rq * 4;
    const int64_t n0 = j * 4;
    const uint4 w = packed[j * RQ + rq];
    const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int64_t n = n0 + d;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t k = k0 + r;
            if (k < K && n < N) {
                const float q = (float)(int)(signed char)(dw[d] >> (8 * r));
                out[k * N + n] = scales ? q * (per_tensor ? scales[0] : scales[k]) : q;
            }
        }
    }
    }
}

__global__ void k_unpack_i4_tiled(const uint4* __restrict__ packed, int64_t K, int64_t N, int64_t G, int64_t RQ,
                                  int64_t NS, int64_t nchunks, const float* __restrict__ scales,
                                  float* __restrict__ out) {
    for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < nchunks;
         c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rq = c / NS, j = c - rq * NS;  // strip fastest: coalesced writes of out
    const int64_t k0 = rq * 4;
    const int64_t n0 = j * 8;
    const uint4 w = packed[j * RQ + rq];
    const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t k = k0 + r;
        if (k >= K) continue;
        const int64_t i0 = k * N + n0;
        const float s = scales ? scales[i0 / G] : 1.0f;  // one group per strip row (N % 8 == 0, G % 8 == 0)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float q = (float)(((int)(dw[r] << (28 - 4 * e))) >> 28);
            out[i0 + e] = scales ? q * s : q;
        }
    }
    }
}

__global__ void k_unpack_i4_flat(const unsigned char* __restrict__ packed, int64_t total, int64_t G,
                                 const float* __restrict__ scales, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t byte = packed[i >> 1];
    const float q = (float)(((int)(byte << (28 - 4 * (int)(i & 1)))) >> 28);
    out[i] = scales ? q * scales[i / G] : q;
    }
}

__global__ void k_dequant_codes(const float* __restrict__ q, const float* __restrict__ scales, int64_t total,
                                int mode, int64_t div, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = q[i] * (mode == 0 ? scales[0] : scales[i / div]);
}

inline unsigned grid_for(int64_t n, int64_t cap = 1 << 16) {
    int64_t g = ceil_div(n, kBlock);
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace

hipError_t launch_fill_zero(void* p, int64_t bytes, hipStream_t s) {
    if (bytes <= 0) return hipSuccess;
    const int64_t n16 = bytes / 16;
    const int ntail = (int)(bytes - n16 * 16);
    k_fill_zero<<<grid_for(n16 > 0 ? n16 : 1, 4096), kBlock, 0, s>>>(
        (uint4*)p, n16, (unsigned char*)p + n16 * 16, ntail);
    return hipGetLastError();
}

hipError_t launch_fill_bias(float* y, int64_t M, int64_t N, const float* bias, hipStream_t s) {
    if (M * N <= 0) return hipSuccess;
    k_fill_bias<<<grid_for(M * N, 4096), kBlock, 0, s>>>(y, M, N, bias);
    return hipGetLastError();
}

hipError_t launch_group_scales(const float* x, int64_t total, int64_t G, int64_t ngroups, float qmax, float* scales,
                               float* inv, hipStream_t s) {
    if (ngroups <= 0) return hipSuccess;
    const int64_t waves_per_block = kBlock / 64;
    k_group_scales<<<grid_for(ngroups * 64, 1 << 16), kBlock, 0, s>>>(x, total, G, ngroups, qmax, scales, inv);
    (void)waves_per_block;
    return hipGetLastError();
}

int64_t absmax_partial_count(int64_t total) {
    int64_t n = ceil_div(total, kBlock * 16);
    if (n < 1) n = 1;
    if (n > 1024) n = 1024;
    return n;
}

hipError_t launch_absmax_partial(const float* x, int64_t total, float* partial, int64_t nparts, hipStream_t s) {
    k_absmax_partial<<<(unsigned)nparts, kBlock, 0, s>>>(x, total, partial);
    return hipGetLastError();
}

hipError_t launch_pack_i8_tiled(const float* src, bool from_codes, int64_t K, int64_t N, const float* inv,
                                bool per_tensor, void* packed, float* qdata, int* bad, hipStream_t s) {
    I8Geom g(K, N);
    const int64_t nchunks = g.chunks();
    if (nchunks <= 0) return hipSuccess;
    k_pack_i8_tiled<<<grid_for(nchunks), kBlock, 0, s>>>(src, from_codes, K, N, g.RQ, g.NS, nchunks, inv, per_tensor,
                                                         (uint4*)packed, qdata, bad);
    return hipGetLastError();
}

hipError_t launch_pack_i4_tiled(const float* src, bool from_codes, int64_t K, int64_t N, int64_t G,
                                const float* inv, void* packed, float* qdata, int* bad, hipStream_t s) {
    I4Geom g(K, N, G);
    const int64_t nchunks = g.chunks();
    if (nchunks <= 0) return hipSuccess;
    k_pack_i4_tiled<<<grid_for(nchunks), kBlock, 0, s>>>(src, from_codes, K, N, g.G, g.RQ, g.NS, nchunks, inv,
                                                         (uint4*)packed, qdata, bad);
    if (packed) {
        const int64_t ndw = g.koct_bytes() / 4;
        const int64_t strip_bytes = g.chunks() * 16;
        k_koct_i4<<<grid_for(ndw), kBlock, 0, s>>>((const uint32_t*)packed, N, g.Kpad, g.RQ, g.KB(), ndw,
                                                   (uint32_t*)((char*)packed + g.koct_off()),
                                                   (uint32_t*)((char*)packed + strip_bytes),
                                                   (int)((g.koct_off() - strip_bytes) / 4));
    }
    return hipGetLastError();
}

hipError_t launch_pack_i4_flat(const float* src, bool from_codes, int64_t total, int64_t G, const float* inv,
                               void* packed, float* qdata, int* bad, hipStream_t s) {
    const int64_t nbytes = ceil_div(total, 2);
    if (nbytes <= 0) return hipSuccess;
    k_pack_i4_flat<<<grid_for(nbytes), kBlock, 0, s>>>(src, from_codes, total, G, inv, (unsigned char*)packed,
                                                       qdata, bad);
    return hipGetLastError();
}

hipError_t launch_devscales_i4(const float* scales, const I4Geom& g, float* devscales, hipStream_t s) {
    const int64_t n = g.devscale_count();
    if (n <= 0) return hipSuccess;
    k_devscales_i4<<<grid_for(n), kBlock, 0, s>>>(scales, g.K, g.N, g.G, g.Kpad, g.spc, g.nsc, devscales);
    return hipGetLastError();
}

hipError_t launch_unpack_i8_tiled(const void* packed, int64_t K, int64_t N, const float* scales, bool per_tensor,
                                  float* out, hipStream_t s) {
    I8Geom g(K, N);
    const int64_t nchunks = g.chunks();
    if (nchunks <= 0 || K * N <= 0) return hipSuccess;
    k_unpack_i8_tiled<<<grid_for(nchunks), kBlock, 0, s>>>((const uint4*)packed, K, N, g.RQ, g.NS, nchunks, scales,
                                                           per_tensor, out);
    return hipGetLastError();
}

hipError_t launch_unpack_i4_tiled(const void* packed, int64_t K, int64_t N, int64_t G, const float* scales,
                                  float* out, hipStream_t s) {
    I4Geom g(K, N, G);
    const int64_t nchunks = g.chunks();
    if (nchunks <= 0 || K * N <= 0) return hipSuccess;
    k_unpack_i4_tiled<<<grid_for(nchunks), kBlock, 0, s>>>((const uint4*)packed, K, N, g.G, g.RQ, g.NS, nchunks, scales,
                                                           out);
    return hipGetLastError();
}

hipError_t launch_unpack_i4_flat(const void* packed, int64_t total, int64_t G, const float* scales, float* out,
                                 hipStream_t s) {
    if (total <= 0) return hipSuccess;
    k_unpack_i4_flat<<<grid_for(total), kBlock, 0, s>>>((const unsigned char*)packed, total, G, scales, out);
    return hipGetLastError();
}

hipError_t launch_dequant_codes(const float* q, const float* scales, int64_t total, int mode, int64_t div, float* out,
                                hipStream_t s) {
    if (total <= 0) return hipSuccess;
    k_dequant_codes<<<grid_for(total), kBlock, 0, s>>>(q, scales, total, mode, div, out);
    return hipGetLastError();
}

}  // namespace sgq
