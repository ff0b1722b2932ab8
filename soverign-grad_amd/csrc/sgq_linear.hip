// sgq_linear.hip -- fused dequantize + matmul kernels for gfx950:
//   y[M,N] = x[M,K] . (codes * scales) (+ bias)        fp32 accumulate
// which the reference computes as dequantize_int8/int4, then a blocked fp32
// matmul, then a bias add (src/quantization.cpp:189-206, src/ops.cpp:378-455,
// src/ops.cpp:132-171).
//
// Decode path (M <= 16): a workgroup owns S strips (whole columns over all of
// K), so no workgroup ever needs another's result.  Its four wavefronts split
// K; within a wavefront 64/S lanes take consecutive row quads of one strip, so
// every 128-bit load of packed codes is part of a contiguous run.  All loads
// of a batch of row quads are issued before any is consumed.  Codes are
// unpacked in registers, the scale is folded into the activation (xs = x * s,
// one multiply per row and lane) and code * xs is accumulated with FMAs.  Lanes
// of a strip are combined by a butterfly that halves the values each lane
// carries at every step, the four wavefronts through LDS.
//
// Prefill path (M > 16): output tiles of 128 rows, K staged through LDS 32
// rows at a time.  k_gemm3 runs the fp32 products on the bf16 matrix cores as
// three exact bf16 products each (x * s split into three bf16 terms, codes
// exact in bf16, fp32 accumulation); k_gemm (INT4 groups that are not a
// multiple of 128) dequantizes codes on the way into LDS (code * scale, the
// reference's own product) and feeds v_mfma_f32_16x16x4_f32.
#include <atomic>
#include <type_traits>

#include "sgq_internal.h"
#include "sgq_lanes.h"

namespace sgq {
namespace {

constexpr int kThreads = 256;

// Batches of up to this many rows decode INT4 with the offset-binary fma_mix
// form; larger batches share one convert per code over their rows instead.
#ifndef SGQ_GEMV_MIX_MAXMT
#define SGQ_GEMV_MIX_MAXMT 2
#endif
constexpr int kGemvMixMaxRows = SGQ_GEMV_MIX_MAXMT;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Byte B of w read as a signed int8 and converted to fp32: the compiler emits
// one v_cvt_f32_i32 with an SDWA sign-extended byte select.  For INT4, a byte
// holding a code in its high nibble and zero below reads as 16*q exactly.
// Plain C++ rather than inline asm: the hazard recognizer does not track
// registers written inside inline asm, so an instruction that reads such a
// register too soon after it is written (an MFMA operand, for one) would get
// no wait states.
template <int B>
__device__ __forceinline__ float cvt_sbyte(uint32_t w) {
    return (float)(signed char)(w >> (8 * B));
}

__device__ __forceinline__ float i8_byte(uint32_t w, int b) {
    return b == 0 ? cvt_sbyte<0>(w) : (b == 1 ? cvt_sbyte<1>(w) : (b == 2 ? cvt_sbyte<2>(w) : cvt_sbyte<3>(w)));
}

// INT4 decode of the GEMV.  A two's-complement nibble q in [-8, 7] XOR 8 is
// its offset-binary form u = q + 8 in [0, 15].  Masked into the low bits of a
// 16-bit half with the exponent bits clear, u reads as the fp16 subnormal
// u * 2^-24 (u at bits 4-7: u * 2^-20), exactly.  fmaf on the half converted
// to float compiles to one v_fma_mix_f32 (the fp16 operand is converted
// inside the FMA, op_sel picks the half), so a code costs one VALU op plus
// 6/8 op of masking, against a convert plus an FMA otherwise.  The kernel
// accumulates sum(u * xs) and undoes the offset with -8 * sum(xs) at the end.
__device__ __forceinline__ float half_lo(uint32_t p) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(p & 0xFFFFu));
}
__device__ __forceinline__ float half_hi(uint32_t p) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(p >> 16));
}

// One INT4 output summed in k order over rows [k0, k1) as code * (x * s)
// (NORM: x * (gamma * s)), reading strip j of the strip-major layout, whose
// dword k is row k.  The GEMV falls back to this when its offset-corrected
// sum is not finite (an infinite or NaN input, or an overflow), so that
// infinities and NaNs come out as in the reference's x . (q * s) rather than
// as inf - inf; the skinny MFMA kernel likewise over its K range.
template <bool NORM>
__device__ float i4_column_exact(const uint4* W, const float* SC, int j, int e, int spc, int Kpad, int RQ,
                                 const float* xrow, const float* gamma, int k0, int k1) {
    const uint32_t* wd = reinterpret_cast<const uint32_t*>(W + (int64_t)j * RQ);
    const float* sc = SC + (int64_t)(j / spc) * Kpad;
    float acc = 0.0f;
    for (int k = k0; k < k1; ++k) {
        const int q = ((int)(wd[k] << (28 - 4 * e))) >> 28;
        const float s = NORM ? gamma[k] * sc[k] : sc[k];
        acc = fmaf((float)q, xrow[k] * s, acc);
    }
    return acc;
}

__device__ __forceinline__ float f4get(const float4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Raw buffer resource over [p, p + bytes): loads through it take a 32-bit
// lane offset plus a wave-uniform SGPR offset (no per-load 64-bit address
// math), and every dword past `bytes` reads as 0 -- which is how rows past K
// and row quads past the strip end contribute nothing.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

constexpr int kOobOff = 0x40000000;  // a lane offset past every buffer the forward kernels read

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads of weight codes that a launch reads once (the GEMV with one row
// group, the INT4 skinny kernels: their workgroups partition the columns and
// K ranges) carry the non-temporal cache policy (`nt`): the stream does not
// displace x and the scales, which every workgroup of a scale column reads
// again.  Kernels whose workgroups read a code again (row groups, GEMM row
// tiles) keep the default policy.  Measured on MI355X (INT4
// g128, M = 1, graphs of 100 calls): 4096->4096 4.42 -> 4.03 us, 4096->11008
// 7.33 -> 6.85, 11008->4096 8.15 -> 7.26, 8192->8192 9.75 -> 8.27.
constexpr int kStreamPolicy = 2;  // buffer-instruction cache policy bit nt (gfx940+)
__device__ __forceinline__ uint4 buf_load16_stream(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kStreamPolicy);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t buf_load4_stream(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kStreamPolicy);
}

// Four floats at byte offset voff + soff (zero past the end).  ALIGN4: the
// buffer holds a multiple of four floats, so a quad is entirely in or out and
// one 128-bit load serves; otherwise four 32-bit loads.
template <bool ALIGN4>
__device__ __forceinline__ float4 buf_load4f(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    if (ALIGN4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    } else {
        return make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff + 0, soff, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff + 4, soff, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff + 8, soff, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff + 12, soff, 0)));
    }
}

// silu(v) = v / (1 + exp(-v)), as simd::vec_silu (simd.hpp:103-108); the
// device expf differs from libm's by at most a few ulp, the division is
// correctly rounded.
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

// Workgroups are dispatched round-robin over the device's X = 2^xlog XCDs
// (workgroup b runs on XCD b % X; a full MI355X has 8, its partitions 4, 2 or
// 1, read per device as device_xcds), and each XCD has its own L2.  Strips
// that share a scale column (and, for the MFMA GEMM, tiles that share
// operands) should run on the same XCD, so the first X*(n/X) workgroup ids are
// permuted to give XCD x the contiguous range [x*(n/X), (x+1)*(n/X)); the
// remaining ids map to themselves.  A bijection on [0, n) for any xlog (0: the
// identity), so the XCD count only affects speed.
__device__ __forceinline__ int xcd_swizzle(int b, int n, int xlog) {
    const int per = n >> xlog;
    const int sw = (b & ((1 << xlog) - 1)) * per + (b >> xlog);
    return b >= (per << xlog) ? b : sw;  // a select, not a branch, ahead of the first loads
}

// Workgroup barrier ordering LDS accesses only: waits for this wave's LDS
// operations, not for its global loads.  __syncthreads() is a release fence
// as well, and gfx950 counts loads and stores on one counter (vmcnt), so it
// waits for every load in flight -- prefetched data included.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Arguments of one GEMV launch (passed by value in the kernel arguments).
struct GemvArgs {
    const float* x;  // [M, K] rows of this pass
    int M, K, N;     // N: columns of one weight
    const uint4* W[3];
    const float* SC[3];
    const float* bias[3];
    int mode, Kpad, RQ, NS;  // NS: strips of one weight
    const float* res;        // added to the output (same indexing), or null
    float* y;
    int ldy;                 // row stride of y and res
    const float* gamma;      // RMSNorm weight [K]: the input is rms_norm(x, gamma, eps)
    float eps;
    int Plog;                // row groups: M rows in 2^Plog groups of MT (one workgroup each; a
                             // group past M reads zeros for x and writes nothing)
    FastDiv spc;             // INT4: division by mode (strips per scale column)
    int nblk;                // grid x (passed here: reading the hidden gridDim argument cost a second
                             // dependent round of kernel-argument loads ahead of the first data load)
    int cus;                 // compute units of the launch's device (host-side heuristics only)
    int xlog;                // log2 of the device's XCD count (xcd_swizzle)
};

// What k_gemv's prologue needs before its first load travels ahead of the
// GemvArgs copy as plain scalar arguments, which gfx950 preloads into SGPRs
// (the build's -amdgpu-kernarg-preload-count=16: 14 dwords after the
// kernel-argument pointer; a by-value struct is never preloaded).  A wave
// then issues its first loads without waiting for a kernel-argument load.
// Measured on MI355X (graphs of 100 calls, us): C2 4.15-4.26 -> 3.98-4.00,
// 4096->11008 at one row 6.88 -> 6.62-6.67, 2048->2048 at 8 rows 4.25-4.43 ->
// 3.95-3.97.  Kpad is 4 * RQ; pk packs Plog (bits 0-7), xlog (8-15), the
// scale-column divider's shift (16-23) and the INT8 per-tensor flag (24).
struct GemvHot {
    const float* x;
    const uint4* W0;
    const float* S0;
    int K, RQ, NS, M, nblk, pk;
    uint32_t spcm;
};
inline GemvHot gemv_hot(const GemvArgs& a, int bits) {
    GemvHot h;
    h.x = a.x, h.W0 = a.W[0], h.S0 = a.SC[0];
    h.K = a.K, h.RQ = a.RQ, h.NS = a.NS, h.M = a.M, h.nblk = a.nblk;
    h.pk = a.Plog | (a.xlog << 8) | (a.spc.l << 16) | ((bits == 8 && a.mode) ? 1 << 24 : 0);
    h.spcm = a.spc.m;
    return h;
}

// ---------------------------------------------------------------------------
// GEMV / skinny GEMM for M <= 8 rows per pass.  One workgroup of NW
// wavefronts per strip (all K rows of SW columns): BITS 4 -> 8 columns,
// scales devscales[j / spc][k]; BITS 8 -> 4 columns, scales[0] (per-tensor)
// or scales[k] (per-row).  Thread t takes row quads rq = 64*NW*it + t, U of
// them in flight at once.  The codes, the
// scales and x of one row quad all sit at byte 16*rq of their buffers, so the
// four loads share one lane offset and one SGPR iteration offset.
// ---------------------------------------------------------------------------
//
// NG == 2 is the gated MLP (SwiGLU::forward up to the down projection,
// include/sovereigngrad/nn.hpp:151-154): the workgroup runs NW wavefronts on
// strip j of the gate weight and NW on strip j of the up weight -- x is read
// by both groups from the same CU's caches -- and the epilogue writes
// silu(gate + bias) * (up + bias2).
//
// SPW > 1 strips per workgroup (adjacent strips j0 .. j0+SPW-1, which must
// share their INT4 scale column: spc % SPW == 0) load each x and scale quad
// once for all of them: fewer load instructions per code byte, which is what
// bounds the single-row GEMV.
//
// With NG == 1, a.nw weights of equal shape may sit side by side along the
// output (a LLaMA block's q, k and v projections of one input): workgroup
// strips run over all of them and weight w writes columns w*N .. w*N+N-1 of
// y.  a.res, when set, is added to every output (a residual connection).
//
// NORM: the input rows are first RMS-normalised (rms_norm, src/ops.cpp:
// 1532-1556: x * inv_rms * gamma, inv_rms = 1 / sqrt(sum(x^2) / K + eps)).
// inv_rms is one factor per row, so it comes out of the K sum: the workgroup
// accumulates (x * gamma * s) * q and sum(x^2) of the x rows it reads anyway
// (all of K), and multiplies by inv_rms in the epilogue.  No separate norm
// launch and no normed copy of x.
template <int BITS, int MT, int NW, int U, bool KALIGN4, int NG, int SPW, bool NORM, bool STREAM>
__global__ __launch_bounds__(NG * NW * 64) void k_gemv(const float* __restrict__ hx, const uint4* __restrict__ hW0,
                                                       const float* __restrict__ hS0, int K, int RQ, int NS, int hM,
                                                       int nblk, int pk, uint32_t spcm, const GemvArgs a) {
    static_assert(NG == 1 || SPW == 1, "the gated form takes one strip of each weight");
    // The scalar arguments (GemvHot) carry every field used ahead of the first
    // loads; the GemvArgs copy the rest (other weights, epilogue, fallback).
    const int N = a.N, Kpad = 4 * RQ, Plog = pk & 255, xlog = (pk >> 8) & 255;
    const int mode = BITS == 8 ? (pk >> 24) & 1 : a.mode;
    constexpr int SW = (BITS == 4) ? 8 : 4;  // columns per strip
    constexpr int RQ_IT = NW * 64;           // row quads per group iteration
    constexpr int CW = SPW * SW;             // columns per workgroup
    constexpr int V = MT * CW;               // accumulators per lane
    constexpr bool MIX = BITS == 4 && MT <= kGemvMixMaxRows;  // offset-binary fma_mix decode
    __shared__ float red[NG * NW][V];
    __shared__ float sqr[NORM ? NG * NW : 1][MT];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = NG == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave / NW);  // weight matrix of this wave
    const int gtid = threadIdx.x - grp * (NW * 64);                           // thread index within its group
    // Strips of a scale column share an XCD's L2.  Workgroups of one weight
    // cover (NS + SPW - 1) / SPW strip groups (x of the grid); with several
    // weights side by side (NG == 1), y of the grid selects the weight.
    // Workgroup v covers row group p = v % P of strip group v / P (P = 2^Plog):
    // the row groups of one strip are neighbours in v, so they run on one XCD
    // and the second read of the strip's codes hits its L2.  No integer
    // division on the way to the first load: every index here is a shift, a
    // mask or a grid coordinate (a runtime division costs about 30 dependent
    // instructions, all of them ahead of the loads).
    const int vg = xcd_swizzle(blockIdx.x, nblk, xlog);
    const int prow = vg & ((1 << Plog) - 1);
    const int jg = vg >> Plog;
    const int m0 = prow * MT;
    const float* __restrict__ x = hx + (int64_t)m0 * K;
    const int M = min(MT, hM - m0);  // <= 0 for a padding group: no x rows, no outputs
    const int wt = NG == 1 ? (int)blockIdx.y : 0;
    const int j0 = SPW * jg;
    const int widx = NG == 1 ? wt : grp;
    // One weight without the norm (every linear call): the preloaded pointers
    // alone, so that no select waits for the GemvArgs copy.  Several weights
    // (the norm-fused q/k/v launch, the gated MLP) select among them.
    constexpr bool ONE = NG == 1 && !NORM;
    const uint4* __restrict__ Wm = (ONE || widx == 0) ? hW0 : (widx == 1 ? a.W[1] : a.W[2]);
    const float* __restrict__ SCm = (ONE || widx == 0) ? hS0 : (widx == 1 ? a.SC[1] : a.SC[2]);
    const float* __restrict__ bias = NG == 1 ? (wt == 0 ? a.bias[0] : (wt == 1 ? a.bias[1] : a.bias[2])) : a.bias[0];
    const float* __restrict__ bias2 = a.bias[1];
    const int voff = gtid * 16;

    __amdgpu_buffer_rsrc_t rW[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s)  // a strip past the last reads zeros and is not stored
        rW[s] = make_rsrc(Wm + (int64_t)(j0 + s < NS ? j0 + s : 0) * RQ, j0 + s < NS ? (uint32_t)RQ * 16u : 0u);
    __amdgpu_buffer_rsrc_t rS;
    float s_all = 0.0f;
    if constexpr (BITS == 4) {
        FastDiv spc;
        spc.m = spcm, spc.l = (pk >> 16) & 255;
        rS = make_rsrc(SCm + (int64_t)spc.div(j0) * Kpad, (uint32_t)Kpad * 4u);
    } else {
        rS = make_rsrc(SCm, mode ? 4u : (uint32_t)K * 4u);
        if (mode) s_all = SCm[0];
    }
    __amdgpu_buffer_rsrc_t rX[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) rX[m] = make_rsrc(x + (int64_t)m * K, m < M ? (uint32_t)K * 4u : 0u);

    __amdgpu_buffer_rsrc_t rG;
    if constexpr (NORM) rG = make_rsrc(a.gamma, (uint32_t)K * 4u);
    float sq[MT];  // NORM: sum of x^2 per row
    float sx[MT];  // INT4: sum of xs per row (the offset correction)
#pragma unroll
    for (int m = 0; m < MT; ++m) sq[m] = 0.0f, sx[m] = 0.0f;

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;

    const int nit = (RQ + RQ_IT - 1) / RQ_IT;
    for (int it0 = 0; it0 < nit; it0 += U) {
        uint4 w[U][SPW];
        float4 sv[U];
        float4 gv[NORM ? U : 1];
        float4 xv[U][MT];  // x is loaded with the codes (measured 4-7% faster for M >= 4 than at use)
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // Row quads past the strip read as zero (buffer range).  No guard on
            // a partial last batch: a branch here would make the compiler wait
            // for every load before the first use instead of one batch entry at a time.
            const int soff = (it0 + u) * RQ_IT * 16;
#pragma unroll
            for (int s = 0; s < SPW; ++s)
                w[u][s] = STREAM ? buf_load16_stream(rW[s], voff, soff) : buf_load16(rW[s], voff, soff);
            if constexpr (BITS == 4) {
                sv[u] = buf_load4f<true>(rS, voff, soff);  // devscales rows are padded to 16
            } else if (!mode) {
                sv[u] = buf_load4f<KALIGN4>(rS, voff, soff);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) xv[u][m] = buf_load4f<KALIGN4>(rX[m], voff, soff);
            if constexpr (NORM) gv[u] = buf_load4f<KALIGN4>(rG, voff, soff);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k0 = 4 * ((it0 + u) * RQ_IT) + 4 * gtid;
            if constexpr (BITS == 8) {
                if (mode) {
                    // Rows past K must give exactly zero, also for a non-finite per-tensor scale.
                    sv[u].x = (k0 + 0 < K) ? s_all : 0.0f;
                    sv[u].y = (k0 + 1 < K) ? s_all : 0.0f;
                    sv[u].z = (k0 + 2 < K) ? s_all : 0.0f;
                    sv[u].w = (k0 + 3 < K) ? s_all : 0.0f;
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float4 xm = xv[u][m];
                float xs[4];
                if constexpr (NORM) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        sq[m] = fmaf(f4get(xm, r), f4get(xm, r), sq[m]);
                        xs[r] = f4get(xm, r) * (f4get(gv[u], r) * f4get(sv[u], r));
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) xs[r] = f4get(xm, r) * f4get(sv[u], r);
                }
                if constexpr (MIX) sx[m] += (xs[0] + xs[1]) + (xs[2] + xs[3]);
#pragma unroll
                for (int s = 0; s < SPW; ++s) {
                    const uint32_t dw[4] = {w[u][s].x, w[u][s].y, w[u][s].z, w[u][s].w};
                    float* a = acc + m * CW + s * SW;
                    if constexpr (MIX) {
                        // Nibble e (column e of the strip) as u * 2^-24 (even e) or
                        // u * 2^-20 (odd e); the masks are shared by all rows m.
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t ob = dw[r] ^ 0x88888888u;
                            const uint32_t p04 = ob & 0x000F000Fu, p15 = ob & 0x00F000F0u;
                            const uint32_t ob8 = ob >> 8;
                            const uint32_t p26 = ob8 & 0x000F000Fu, p37 = ob8 & 0x00F000F0u;
                            a[0] = fmaf(half_lo(p04), xs[r], a[0]);
                            a[4] = fmaf(half_hi(p04), xs[r], a[4]);
                            a[1] = fmaf(half_lo(p15), xs[r], a[1]);
                            a[5] = fmaf(half_hi(p15), xs[r], a[5]);
                            a[2] = fmaf(half_lo(p26), xs[r], a[2]);
                            a[6] = fmaf(half_hi(p26), xs[r], a[6]);
                            a[3] = fmaf(half_lo(p37), xs[r], a[3]);
                            a[7] = fmaf(half_hi(p37), xs[r], a[7]);
                        }
                    } else if constexpr (BITS == 4) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t hi = dw[r] & 0xF0F0F0F0u;         // columns 2b+1, as 16*q
                            const uint32_t lo = (dw[r] << 4) & 0xF0F0F0F0u;  // columns 2b, as 16*q
#pragma unroll
                            for (int b = 0; b < 4; ++b) {
                                a[2 * b] = fmaf(i8_byte(lo, b), xs[r], a[2 * b]);
                                a[2 * b + 1] = fmaf(i8_byte(hi, b), xs[r], a[2 * b + 1]);
                            }
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
#pragma unroll
                            for (int d = 0; d < 4; ++d) a[d] = fmaf(i8_byte(dw[d], r), xs[r], a[d]);
                    }
                }
            }
        }
    }

    if constexpr (MIX) {
        // Undo the scaling (exact) and the offset per lane: the reduction below
        // is a plain sum, so correcting each lane's partial sums before it gives
        // the corrected total with no second reduction for sum(xs).
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float off = -8.0f * sx[m];
#pragma unroll
            for (int c = 0; c < CW; ++c)
                acc[m * CW + c] = fmaf(acc[m * CW + c], (c & 1) ? 1048576.0f : 16777216.0f, off);
        }
    }

    // Combine the 64 lanes of each wavefront, then the NW wavefronts.
    int base = 0;
    lane_reduce_tail<V, 0>(acc, lane, base);
    constexpr int left = red_left(V);
    constexpr LaneSel wsel = red_tail_writer(V);
    if ((lane & wsel.mask) == wsel.value) {
#pragma unroll
        for (int i = 0; i < left; ++i) red[wave][base + i] = acc[i];
    }
    if constexpr (NORM) {
        int sbase = 0;
        lane_reduce<MT, 0>(sq, lane, sbase);
        if ((lane & red_dup_mask(MT)) == 0) {
#pragma unroll
            for (int i = 0; i < red_left(MT); ++i) sqr[wave][sbase + i] = sq[i];
        }
    }
    __syncthreads();

    // MIX: a non-finite total (an infinite or NaN input, or an overflow) takes
    // the exact k-order sum instead.  INT4 without MIX read its codes as
    // 16 * q: scale by 1/16 (exact).
    for (int v = threadIdx.x; v < V; v += NG * NW * 64) {
        const int m = v / CW, e = v - m * CW;
        const int n = j0 * SW + e;
        if (m < M && n < N) {
            const int64_t o = (int64_t)(m0 + m) * a.ldy + (int64_t)wt * N + n;
            float r = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) r += red[w][v];
            float inv = 1.0f;
            if constexpr (NORM) {  // every group read all of x: group 0's waves hold the full sum
                float ss = 0.0f;
#pragma unroll
                for (int w = 0; w < NW; ++w) ss += sqr[w][m];
                inv = 1.0f / sqrtf(ss / (float)K + a.eps);
            }
            auto i4_total = [&](float t, const uint4* Wg, const float* SCg) {
                if (!isfinite(t))
                    t = i4_column_exact<NORM>(Wg, SCg, j0 + e / SW, e % SW, mode, Kpad, RQ,
                                              hx + (int64_t)(m0 + m) * K, a.gamma, 0, K);
                return t;
            };
            if constexpr (MIX) r = i4_total(r, NG == 1 ? Wm : a.W[0], NG == 1 ? SCm : a.SC[0]);
            if constexpr (BITS == 4 && !MIX) r = r * 0.0625f;
            if constexpr (NORM) r = r * inv;
            if (bias) r = r + bias[n];
            if constexpr (NG == 2) {
                float r2 = 0.0f;
#pragma unroll
                for (int w = NW; w < 2 * NW; ++w) r2 += red[w][v];
                if constexpr (MIX) r2 = i4_total(r2, a.W[1], a.SC[1]);
                if constexpr (BITS == 4 && !MIX) r2 = r2 * 0.0625f;
                if constexpr (NORM) r2 = r2 * inv;
                if (bias2) r2 = r2 + bias2[n];
                r = silu_f32(r) * r2;
            }
            if (a.res) r = r + a.res[o];
            a.y[o] = r;
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM: 128x128 tile per workgroup, four waves in 2x2, each 64x64 made of
// 4x4 blocks of v_mfma_f32_16x16x4_f32.  LDS holds A as [m][k] and the
// dequantized B as [n][k] (k contiguous), kBK k per stage, double buffered.
// Global loads run two stages ahead in two register sets; the stage after the
// current one is dequantized into the other LDS buffer between the current
// stage's MFMA blocks (measured on MI355X, C4: 117 TFLOP/s against 105 with
// one stage ahead and the stores before the barrier).  Within each 16-k block of a stage lane l supplies
// k = 4*(l/16) + kk to the kk-th MFMA, so one 128-bit LDS read per operand
// block feeds four MFMAs; A and B use the same k assignment, so every product
// pairs matching k.  The LDS row stride kBK + 4 floats keeps the 16 lanes of
// a 128-bit read on distinct banks.
// ---------------------------------------------------------------------------
#ifndef SGQ_GEMM_BK
#define SGQ_GEMM_BK 32
#endif
#ifndef SGQ_GEMM_STORE_BLOCK
#define SGQ_GEMM_STORE_BLOCK 1
#endif
constexpr int kBM = 128, kBN = 128, kBK = SGQ_GEMM_BK, kLdsStride = kBK + 4;
constexpr int kStoreBlock = SGQ_GEMM_STORE_BLOCK;  // 16-k block of a stage before which the next stage is stored
static_assert(kBK % 16 == 0 && kBK <= 64, "stage depth is a multiple of 16");

template <int BITS, bool KALIGN4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm(const float* __restrict__ x, int M, int K, int N,
                                                   const uint4* __restrict__ W, const float* __restrict__ S,
                                                   int mode, int Kpad, int RQ, int NS, int KS, int sps,
                                                   const float* __restrict__ bias, float* __restrict__ y,
                                                   float* __restrict__ part) {
    // mode: INT8 -> per_tensor flag; INT4 -> strips per scale column (spc).
    // Workgroup b computes split b % KS (stages [kt0, kt1) of sps each) of
    // tile b / KS; with KS > 1 it writes part[split][M][N] instead of y.
    constexpr int SW = (BITS == 4) ? 8 : 4;
    constexpr int KQ = kBK / 4;                 // row quads per stage
    constexpr int kStrips = kBN / SW;           // strips per tile: 16 (INT4) or 32 (INT8)
    // INT4: B dequantized to fp32 [n][k].  INT8: B as the raw 16-byte chunks
    // (strip, row quad), each dword four consecutive k of one column -- what
    // an MFMA lane consumes -- with the strip stride padded to KQ*4 + 8 dwords
    // so the 32 lanes of a half-wave read 32 different banks.
    __shared__ __attribute__((aligned(16))) float As[2][kBM][kLdsStride];
    __shared__ __attribute__((aligned(16))) float Bs[BITS == 4 ? 2 : 1][BITS == 4 ? kBN : 1][kLdsStride];
    __shared__ __attribute__((aligned(16))) uint4 Bq[BITS == 8 ? 2 : 1][BITS == 8 ? kStrips : 1][KQ + 2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ntn = (N + kBN - 1) / kBN;
    const int tile = blockIdx.x / KS, split = blockIdx.x - tile * KS;
    const int tm = tile / ntn, tn = tile - tm * ntn;
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int KT = (Kpad + kBK - 1) / kBK;  // the last stage may reach past Kpad: masked below
    const int kt0 = split * sps, kt1 = (kt0 + sps) < KT ? (kt0 + sps) : KT;
    // Scales: INT8 per-channel scales[k] (zero past K), per-tensor scales[0];
    // INT4 devscales[sc][Kpad].
    const __amdgpu_buffer_rsrc_t rS =
        make_rsrc(S, BITS == 8 ? (mode ? 4u : (uint32_t)K * 4u) : (uint32_t)(((NS + mode - 1) / mode) * Kpad) * 4u);
    const float s_all = (BITS == 8 && mode) ? S[0] : 0.0f;

    constexpr int kBChunks = kStrips * KQ;      // chunks of B per stage
    constexpr int kAVec = kBM * kBK / 4 / kThreads;  // float4 of A per thread per stage
    constexpr int kBPer = (kBChunks + kThreads - 1) / kThreads;  // chunks of B per thread per stage
    static_assert(kBChunks % kThreads == 0 || kBChunks < kThreads, "B chunks spread evenly");
    // chunk t of a stage: strip n0/SW + t / KQ, row quad KQ*kt + t % KQ

    // Two register sets of one stage each: while stage kt is computed from
    // LDS, set A/B of stage kt+1 (loaded a whole stage earlier) is stored to
    // the other LDS buffer and the loads of stage kt+2 are in flight.
    struct Regs {
        float4 a[kAVec];
        uint4 b[kBPer];
        float4 s;  // INT8 per-channel: scales of this thread's four A columns k
    };
    // Buffer resources over this tile's rows of x and strips of W: rows past
    // M and strips past NS read as zero; k past K and row quads past RQ (which
    // would read the next row or strip) get an out-of-range lane offset.
    const int mrows = (M - m0) < kBM ? (M - m0) : kBM;
    const int nstr = (NS - n0 / SW) < kStrips ? (NS - n0 / SW) : kStrips;
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(x + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(W + (int64_t)(n0 / SW) * RQ, (uint32_t)nstr * (uint32_t)RQ * 16u);
    auto load = [&](Regs& rg, int kt) {
        const int soffA = kt * kBK * 4, soffB = kt * KQ * 16;
#pragma unroll
        for (int i = 0; i < kAVec; ++i) {
            const int idx = tid + kThreads * i;
            const int row = idx / KQ, kq = idx % KQ;
            const int k = kt * kBK + kq * 4;
            const int vo = (row * K + kq * 4) * 4;
            if (KALIGN4) {
                rg.a[i] = buf_load4f<true>(rX, k < K ? vo : kOobOff, soffA);
            } else {
                float t[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    t[r] = __uint_as_float(
                        __builtin_amdgcn_raw_buffer_load_b32(rX, k + r < K ? vo + 4 * r : kOobOff, soffA, 0));
                rg.a[i] = make_float4(t[0], t[1], t[2], t[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < kBPer; ++i) {
            const int t = tid + kThreads * i;
            const int rq = kt * KQ + t % KQ;
            const int vo = ((t / KQ) * RQ + t % KQ) * 16;
            rg.b[i] = buf_load16(rW, (t < kBChunks && rq < RQ) ? vo : kOobOff, soffB);
        }
        // Every A float4 of this thread sits at column quad tid % KQ of the stage.
        if constexpr (BITS == 8)
            if (!mode) rg.s = buf_load4f<KALIGN4>(rS, (tid % KQ) * 16, kt * kBK * 4);  // zero past K
    };
    auto store = [&](const Regs& rg, int buf, int kt) {
        // INT8: the scale of row k of W goes into column k of A, (x * s) * q
        // (the reference forms x * (q * s): the same products up to one
        // rounding); columns past K are exactly zero, also for a non-finite
        // per-tensor scale.
        float4 sa = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        if constexpr (BITS == 8) {
            if (mode) {
                const int k = kt * kBK + (tid % KQ) * 4;
                sa = make_float4(k < K ? s_all : 0.0f, k + 1 < K ? s_all : 0.0f, k + 2 < K ? s_all : 0.0f,
                                 k + 3 < K ? s_all : 0.0f);
            } else {
                sa = rg.s;
            }
        }
#pragma unroll
        for (int i = 0; i < kAVec; ++i) {
            const int idx = tid + kThreads * i;
            const int row = idx / KQ, kq = idx % KQ;
            if constexpr (BITS == 8)
                *(float4*)&As[buf][row][kq * 4] =
                    make_float4(rg.a[i].x * sa.x, rg.a[i].y * sa.y, rg.a[i].z * sa.z, rg.a[i].w * sa.w);
            else
                *(float4*)&As[buf][row][kq * 4] = rg.a[i];
        }
#pragma unroll
        for (int i = 0; i < kBPer; ++i) {
            const int t = tid + kThreads * i;
            if (t >= kBChunks) continue;
            const int jl = t / KQ, kl = (t % KQ) * 4;
            const int k = kt * kBK + kl;
            const uint32_t dw[4] = {rg.b[i].x, rg.b[i].y, rg.b[i].z, rg.b[i].w};
            if constexpr (BITS == 8) {
                (void)dw;
                (void)k;
                Bq[buf][jl][kl / 4] = rg.b[i];
            } else {
                const int bj = n0 / SW + jl;
                const int jc = bj < NS ? bj : NS - 1;
                // devscales rows stop at Kpad (codes there are zero); the
                // 1/16 turns the 16*q read of a high nibble back into q (exact)
                const float4 s4 = buf_load4f<true>(rS, k < Kpad ? ((jc / mode) * Kpad + kl) * 4 : kOobOff,
                                                   kt * kBK * 4);
                const float sc[4] = {s4.x * 0.0625f, s4.y * 0.0625f, s4.z * 0.0625f, s4.w * 0.0625f};
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    hi[r] = dw[r] & 0xF0F0F0F0u;         // byte c: column 2c+1 of row r, as 16*q
                    lo[r] = (dw[r] << 4) & 0xF0F0F0F0u;  // byte c: column 2c
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    *(float4*)&Bs[buf][jl * 8 + 2 * c][kl] =
                        make_float4(i8_byte(lo[0], c) * sc[0], i8_byte(lo[1], c) * sc[1], i8_byte(lo[2], c) * sc[2],
                                    i8_byte(lo[3], c) * sc[3]);
                    *(float4*)&Bs[buf][jl * 8 + 2 * c + 1][kl] =
                        make_float4(i8_byte(hi[0], c) * sc[0], i8_byte(hi[1], c) * sc[1], i8_byte(hi[2], c) * sc[2],
                                    i8_byte(hi[3], c) * sc[3]);
                }
            }
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int lr = lane & 15;
    // One stage: `next` holds stage kt+1 (stored to the other buffer during
    // the MFMAs), `fill` is free and receives the loads of stage kt+2.
    auto stage = [&](int kt, const Regs& next, Regs& fill) {
        const int buf = kt & 1;
        // Unconditional: past the last stage the loads read zeros (k past K,
        // row quads past RQ); a guard here would make the compiler wait for
        // these loads at the join, before the next stage's LDS store.
        load(fill, kt + 2);
#pragma unroll
        for (int sb = 0; sb < kBK / 16; ++sb) {
            if (sb == kStoreBlock && kt + 1 < kt1) store(next, buf ^ 1, kt + 1);
            const int lk = sb * 16 + (lane >> 4) * 4;
            float4 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *(const float4*)&As[buf][wm * 64 + i * 16 + lr][lk];
            if constexpr (BITS == 8) {
                // one dword: column n, rows lk .. lk+3, converted here
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int nl = wn * 64 + j * 16 + lr;
                    const uint32_t bd = ((const uint32_t*)&Bq[buf][nl >> 2][lk >> 2])[nl & 3];
                    b[j] = make_float4(cvt_sbyte<0>(bd), cvt_sbyte<1>(bd), cvt_sbyte<2>(bd), cvt_sbyte<3>(bd));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = *(const float4*)&Bs[buf][wn * 64 + j * 16 + lr][lk];
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(a[i], kk), f4get(b[j], kk), acc[i][j],
                                                                         0, 0, 0);
        }
        lds_barrier();
    };

    Regs r0, r1;
    load(r0, kt0);
    if (kt0 + 1 < kt1) load(r1, kt0 + 1);
    store(r0, kt0 & 1, kt0);
    lds_barrier();
    for (int kt = kt0; kt < kt1; kt += 2) {
        stage(kt, r1, r0);
        if (kt + 1 < kt1) stage(kt + 1, r0, r1);
    }

    // D layout of 16x16x4: lane l, element r -> row 4*(l/16) + r, column l%16.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + lr;
            if (n >= N) continue;
            const float bv = (bias && KS == 1) ? bias[n] : 0.0f;
            float* out = KS == 1 ? y : part + (int64_t)split * M * N;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) {
                    const float v = acc[i][j][r];
                    out[(int64_t)m * N + n] = (bias && KS == 1) ? v + bv : v;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Three-term bf16 MFMA GEMM (prefill).  The fp32 products of the reference's
// matmul run on the bf16 matrix cores, which gfx950 issues at 16 times the
// fp32 MFMA rate, without giving up fp32 results:
//   - every operand of the bf16 MFMAs is exact.  A code q (|q| <= 127) is a
//     bf16 integer.  The activation xs = x * s (the weight's scale folded in,
//     one rounding as in the fp32 kernels) is split as xs = h + m + l, where
//     h keeps the leading 8 significant bits of xs (truncation), m the next 8
//     of the remainder and l the rest, which is at most 8 bits: the three are
//     bf16 numbers and their sum is xs exactly;
//   - a bf16 x bf16 product is exact in fp32, and v_mfma_f32_16x16x32_bf16
//     sums into an fp32 accumulator, so acc += h.q, m.q and l.q (three MFMAs
//     per 16x16x32 block) computes sum(xs * q) with fp32 accumulation.
//     (Measured on the box: a 32-term dot product of split fp32 values and
//     codes came out within 5e-9 of fp64, against 1.6e-8 for an fp32 FMA chain.)
// An output whose total is not finite (an infinite or NaN input, or an
// overflow, where h + m + l would be inf - inf) is recomputed by its thread
// as the reference's x . (q * s) in k order, so infinities and NaNs land
// where the reference puts them.
//
// Tiles (G3Shape): INT8 128x256 with eight wavefronts in 2x4, INT4 128x128
// with four in 2x2; each wavefront owns 64x64 as 4x4 MFMA blocks.  One 32-k
// stage per LDS buffer, double-buffered, global loads two stages ahead (as
// k_gemm).  LDS entries are 16 bytes, eight consecutive k of one row (A
// planes) or one column (B): one MFMA operand.  Per-tensor INT8 puts x itself
// into A and multiplies by the scale in the epilogue.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kB3BK = 32;           // k per stage: one 16x16x32 MFMA step
constexpr int kB3KG = kB3BK / 8;    // 8-k groups per stage
constexpr int kB3RQ = kB3BK / 4;    // row quads per stage

// Upper halves (bf16 bits) of two floats in one dword, lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
__device__ __forceinline__ float trunc_bf16(float v) { return __uint_as_float(__float_as_uint(v) & 0xFFFF0000u); }

// Eight nibble codes (k order, nibble 0 first) as the bf16 values 16q of a B
// operand: high nibbles masked in place and low nibbles shifted up read as
// signed bytes 16q, converted exactly.
__device__ __forceinline__ bf16x8 nibbles_bf16x16(uint32_t t) {
    const uint32_t hi = t & 0xF0F0F0F0u, lo = (t << 4) & 0xF0F0F0F0u;
    const uint4 b = make_uint4(pack_hi16(cvt_sbyte<0>(lo), cvt_sbyte<0>(hi)), pack_hi16(cvt_sbyte<1>(lo), cvt_sbyte<1>(hi)),
                               pack_hi16(cvt_sbyte<2>(lo), cvt_sbyte<2>(hi)), pack_hi16(cvt_sbyte<3>(lo), cvt_sbyte<3>(hi)));
    return __builtin_bit_cast(bf16x8, b);
}

// Splits eight floats into the bf16 planes h, m, l (four dwords each).
__device__ __forceinline__ void split3(const float* v, uint4& h, uint4& m, uint4& l) {
    // No fma: fused with the multiply that made v (x * s), a - trunc(a)
    // would take the unrounded product, and h + m + l would miss v by up to
    // an ulp.
#pragma clang fp contract(off)
    uint32_t ph[4], pm[4], pl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = v[2 * i], b = v[2 * i + 1];
        ph[i] = pack_hi16(a, b);
        const float ra = a - trunc_bf16(a), rb = b - trunc_bf16(b);
        pm[i] = pack_hi16(ra, rb);
        pl[i] = pack_hi16(ra - trunc_bf16(ra), rb - trunc_bf16(rb));
    }
    h = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    m = make_uint4(pm[0], pm[1], pm[2], pm[3]);
    l = make_uint4(pl[0], pl[1], pl[2], pl[3]);
}

// split3 of four floats (two dwords per plane).
__device__ __forceinline__ void split3_4(const float* v, uint2& h, uint2& m, uint2& l) {
#pragma clang fp contract(off)
    uint32_t ph[2], pm[2], pl[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float a = v[2 * i], b = v[2 * i + 1];
        ph[i] = pack_hi16(a, b);
        const float ra = a - trunc_bf16(a), rb = b - trunc_bf16(b);
        pm[i] = pack_hi16(ra, rb);
        pl[i] = pack_hi16(ra - trunc_bf16(ra), rb - trunc_bf16(rb));
    }
    h = make_uint2(ph[0], ph[1]);
    m = make_uint2(pm[0], pm[1]);
    l = make_uint2(pl[0], pl[1]);
}

// One output of the forward as the reference forms it: sum over k in
// [k0, k1) of x[k] * (q[k][n] * s), in k order (the non-finite fallback).
template <int BITS>
__device__ float output_exact(const float* xrow, const uint4* W, const float* S, int mode, int Kpad, int RQ, int n,
                              int k0, int k1) {
    float acc = 0.0f;
    for (int k = k0; k < k1; ++k) {
        float q, s;
        if constexpr (BITS == 8) {
            q = (float)reinterpret_cast<const signed char*>(W)[((int64_t)(n >> 2) * RQ + (k >> 2)) * 16 + (n & 3) * 4 +
                                                                (k & 3)];
            s = mode ? S[0] : S[k];
        } else {
            const uint32_t d = reinterpret_cast<const uint32_t*>(W + (int64_t)(n >> 3) * RQ)[k];
            q = (float)(((int)(d << (28 - 4 * (n & 7)))) >> 28);
            s = S[(int64_t)((n >> 3) / mode) * Kpad + k];
        }
        acc = fmaf(xrow[k], q * s, acc);
    }
    return acc;
}

// Tile shape: WM x WN wavefronts, each RB x CB blocks of 16x16 outputs, so
// the tile is BM = 16 * RB * WM rows by BN = 16 * CB * WN columns.  A wider
// tile splits each x value once for more columns (less split work per
// MFMA); INT4 tiles are 128 columns, the width of one scale column at group
// 128.
template <int WM_, int RB_, int WN_, int CB_>
struct G3Shape {
    static constexpr int WM = WM_, RB = RB_, WN = WN_, CB = CB_;
    static constexpr int NT = 64 * WM * WN;
    static constexpr int BM = 16 * RB * WM, BN = 16 * CB * WN;
    static constexpr int WPE = RB * CB >= 16 ? 2 : 1;  // minimum waves per SIMD the register budget keeps
};
using G3Wide = G3Shape<2, 4, 4, 4>;  // 128 x 256, 8 wavefronts: INT8
using G3Tile = G3Shape<2, 4, 2, 4>;  // 128 x 128, 4 wavefronts: INT4
// Skinny batches (17..64 rows) waste most of a 128-row tile's MFMA work and
// split work: they take 32- or 64-row tiles (either code width, 128 columns).
using G3Rows32 = G3Shape<1, 2, 2, 4>;  // 32 x 128, 2 wavefronts
using G3Rows64 = G3Shape<2, 2, 2, 4>;  // 64 x 128, 4 wavefronts

// Arguments of one k_gemm3 launch, passed as one struct: the build preloads
// leading scalar kernel arguments into SGPRs, which the latency-bound GEMV and
// skinny kernels gain from and a GEMM of this length does not need.
struct Gemm3Args {
    const float* x;
    int M, K, N;
    const uint4* W;
    const float* S;
    int mode, Kpad, RQ, NS, KS, sps;
    const float* bias;
    float* y;
    float* part;
    int xr, xlog;
    int ko;  // INT4: byte offset / 256 of the k-octet copy
};

template <int BITS, bool KALIGN4, bool PT, class SH>
__global__ __launch_bounds__(SH::NT) __attribute__((amdgpu_waves_per_eu(SH::WPE))) void k_gemm3(const Gemm3Args ga) {
    const float* __restrict__ x = ga.x;
    const int M = ga.M, K = ga.K, N = ga.N;
    const uint4* __restrict__ W = ga.W;
    const float* __restrict__ S = ga.S;
    const int mode = ga.mode, Kpad = ga.Kpad, RQ = ga.RQ, NS = ga.NS, KS = ga.KS, sps = ga.sps;
    const float* __restrict__ bias = ga.bias;
    float* __restrict__ y = ga.y;
    float* __restrict__ part = ga.part;
    const int xr = ga.xr, xlog = ga.xlog;
    // mode: INT8 -> per-tensor flag (also the template flag PT, so that no
    // stage holds a branch); INT4 -> strips per scale column (a multiple of
    // 16: one scale column per 128-column tile).  Workgroup b computes split
    // b % KS (stages [kt0, kt1) of sps each) of tile b / KS.  xr > 0 (no K
    // split): each XCD takes a rectangle of xr tile rows (see below).
    constexpr int SW = (BITS == 4) ? 8 : 4;
    constexpr int NT = SH::NT, BM = SH::BM, BN = SH::BN, RB = SH::RB, CB = SH::CB;
    constexpr int EA = BM * kB3KG / NT;  // A entries (row, k group) per thread
    constexpr int EB = BN * kB3KG / NT;  // B entries (column, k group) per thread
    static_assert(BM * kB3KG % NT == 0 && EA >= 1 && BN * kB3KG % NT == 0 && EB >= 1, "entries spread evenly");
    static_assert(BITS == 8 || BN == 128, "an INT4 tile spans one scale column");
    __shared__ uint4 As[2][3][kB3KG][BM];
    __shared__ uint4 Bs[2][kB3KG][BN];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % SH::WM, wn = wave / SH::WM;
    const int ntn = (N + BN - 1) / BN;
    // Without a K split, tiles of one x row block run on one XCD (workgroups
    // go round-robin over the 8 XCDs, each with its own L2): C4's L2 misses
    // had every XCD fetch nearly all of x.  Measured 1-2% faster on the large
    // shapes; with a split (small grids) the plain order measured better.
    const int bsw = KS == 1 ? xcd_swizzle(blockIdx.x, gridDim.x, xlog) : (int)blockIdx.x;
    const int tile = bsw / KS, split = bsw - tile * KS;
    int tm = tile / ntn, tn = tile - tm * ntn;
    if (xr > 0) {
        // The grid's tiles fall into one rectangle of xr tile rows by per / xr
        // tile columns per XCD (its share of the swizzled ids), so an XCD's
        // L2 fetches xr row blocks of x and per / xr column blocks of codes
        // instead of every column block (C4 on 8 XCDs: 16 MiB per XCD, not 20).
        const int per = (int)gridDim.x >> xlog, x = tile / per, l = tile - x * per;
        const int bw = per / xr, rects_m = (gridDim.x / ntn) / xr;
        tm = (x % rects_m) * xr + l % xr;
        tn = (x / rects_m) * bw + l / xr;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = (Kpad + kB3BK - 1) / kB3BK;
    const int kt0 = split * sps, kt1 = (kt0 + sps) < KT ? (kt0 + sps) : KT;

    // LDS access rule measured on gfx950: a 16-lane group of a 128-bit LDS
    // access runs at full rate when it touches 16 consecutive 16-byte slots in
    // lane order; other orders cost up to 8x.  So entry e of a stage (A: row,
    // k group; B: column, k group) is row/column (e % 16) + 16 * (e / 64) of k
    // group (e / 16) % 4, thread t takes entries t, t + NT, ..., and the MFMA
    // operand reads are the same 16-slot runs.
    const int akg = (tid >> 4) & 3, ar = (tid & 15) + 16 * (tid >> 6);
    constexpr int kStep = NT / 4;  // rows or columns between a thread's entries
    const int mrows = (M - m0) < BM ? (M - m0) : BM;
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(x + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 4u);
    // Scale of column k of A (zero past K): per-channel scales[k], INT4 the
    // tile's scale column devscales[sc][k].  Per-tensor: x itself goes into A
    // (zero past K) and the epilogue multiplies by scales[0].
    __amdgpu_buffer_rsrc_t rS;
    if constexpr (BITS == 8)
        rS = make_rsrc(S, PT ? 4u : (uint32_t)K * 4u);
    else
        rS = make_rsrc(S + (int64_t)((n0 / SW) / mode) * Kpad, (uint32_t)K * 4u);
    // B side: an entry holds the eight k of its k group for one column.
    // INT8: the column's dword of the two strip chunks (row quads 2 * kg and
    // 2 * kg + 1) that hold them; strips past NS read as zero.  INT4: one
    // dword of the k-octet copy, block (column / 16, stage) dword 16 kg +
    // column % 16, which holds exactly those eight codes; column blocks past
    // the weight's read as zero.
    const int KB = (Kpad + kB3BK - 1) / kB3BK;
    __amdgpu_buffer_rsrc_t rW;
    if constexpr (BITS == 8) {
        const int nstr = (NS - n0 / SW) < (BN / SW) ? (NS - n0 / SW) : (BN / SW);
        rW = make_rsrc(W + (int64_t)(n0 / SW) * RQ, (uint32_t)nstr * (uint32_t)RQ * 16u);
    } else {
        const int ncb = ((NS + 1) / 2 - n0 / 16) < (BN / 16) ? ((NS + 1) / 2 - n0 / 16) : (BN / 16);
        rW = make_rsrc(W + ((int64_t)ga.ko + (int64_t)(n0 / 16) * KB) * 16, (uint32_t)ncb * (uint32_t)KB * 256u);
    }

    struct Regs {
        float4 a[EA][2];  // [entry][quad]
        float4 s[2];      // scales of the thread's eight k
        uint2 b[EB];      // [entry]: INT8 {lo, hi} dwords, INT4 the k-octet dword in .x
    };
    auto load = [&](Regs& rg, int kt) {
        const int kb = kt * kB3BK + akg * 8;
        const int soff = kt * kB3BK * 4;
#pragma unroll
        for (int h = 0; h < EA; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int vo = ((ar + kStep * h) * K + akg * 8 + 4 * q) * 4;
                if (KALIGN4) {
                    rg.a[h][q] = buf_load4f<true>(rX, kb + 4 * q < K ? vo : kOobOff, soff);
                } else {
                    float t[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        t[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rX, kb + 4 * q + r < K ? vo + 4 * r : kOobOff, soff, 0));
                    rg.a[h][q] = make_float4(t[0], t[1], t[2], t[3]);
                }
            }
        if constexpr (!PT) {
#pragma unroll
            for (int q = 0; q < 2; ++q) rg.s[q] = buf_load4f<KALIGN4>(rS, (akg * 8 + 4 * q) * 4, soff);
        }
        if constexpr (BITS == 8) {
            // RQ is a multiple of 4, so both row quads of the pair are in or out together.
            const bool in = kt * kB3RQ + 2 * akg < RQ;
            const int bsoff = kt * kB3RQ * 16;
#pragma unroll
            for (int c = 0; c < EB; ++c) {
                const int n = ar + kStep * c;
                const int vd = ((n / SW) * RQ + 2 * akg) * 16 + (n & 3) * 4;
                rg.b[c].x = __builtin_amdgcn_raw_buffer_load_b32(rW, in ? vd : kOobOff, bsoff, 0);
                rg.b[c].y = __builtin_amdgcn_raw_buffer_load_b32(rW, in ? vd + 16 : kOobOff, bsoff, 0);
            }
        } else {
            const bool in = kt < KB;
#pragma unroll
            for (int c = 0; c < EB; ++c) {
                const int n = ar + kStep * c;
                const int vd = (n >> 4) * KB * 256 + (16 * akg + (n & 15)) * 4;
                rg.b[c].x = __builtin_amdgcn_raw_buffer_load_b32(rW, in ? vd : kOobOff, kt * 256, 0);
            }
        }
    };
    auto store = [&](const Regs& rg, int buf) {
#pragma unroll
        for (int h = 0; h < EA; ++h) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                v[i] = PT ? f4get(rg.a[h][i >> 2], i & 3) : f4get(rg.a[h][i >> 2], i & 3) * f4get(rg.s[i >> 2], i & 3);
            const int row = ar + kStep * h;
            split3(v, As[buf][0][akg][row], As[buf][1][akg][row], As[buf][2][akg][row]);
        }
#pragma unroll
        for (int c = 0; c < EB; ++c) {
            if constexpr (BITS == 8) {
                // bytes of the column's dword in each chunk: k = 0..3, then 4..7
                const uint32_t lo = rg.b[c].x, hi = rg.b[c].y;
                float f[8];
                f[0] = cvt_sbyte<0>(lo), f[1] = cvt_sbyte<1>(lo), f[2] = cvt_sbyte<2>(lo), f[3] = cvt_sbyte<3>(lo);
                f[4] = cvt_sbyte<0>(hi), f[5] = cvt_sbyte<1>(hi), f[6] = cvt_sbyte<2>(hi), f[7] = cvt_sbyte<3>(hi);
                Bs[buf][akg][ar + kStep * c] = make_uint4(pack_hi16(f[0], f[1]), pack_hi16(f[2], f[3]),
                                                           pack_hi16(f[4], f[5]), pack_hi16(f[6], f[7]));
            } else {
                // the eight codes as 16q (the epilogue divides by 16)
                Bs[buf][akg][ar + kStep * c] = __builtin_bit_cast(uint4, nibbles_bf16x16(rg.b[c].x));
            }
        }
    };

    floatx4 acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int lr = lane & 15, lkg = lane >> 4;
    // Raised wave priority while a wavefront issues its MFMAs lets the two
    // wavefronts of a SIMD drift out of phase: one in its MFMAs, the other
    // loading and splitting.  Measured per form (two runs, builds
    // interleaved): INT4 with the priority over all MFMAs of a stage, 4-5%
    // faster; INT8 per-tensor over the first half (up to the store),
    // 1.4-1.8%; INT8 per-channel, whose store does more VALU work, 1-5% slower
    // with either, so without.  2: whole stage, 1: first half, 0: none.
    constexpr int kPrio = BITS == 4 ? 2 : (PT ? 1 : 0);
    auto stage = [&](int kt, const Regs& next, Regs& fill) {
        const int buf = kt & 1;
        load(fill, kt + 2);  // past the last stage these read zeros
        uint4 bq[CB], af[3][RB];
#pragma unroll
        for (int j = 0; j < CB; ++j) bq[j] = Bs[buf][lkg][wn * 16 * CB + j * 16 + lr];
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < RB; ++i) af[p][i] = As[buf][p][lkg][wm * 16 * RB + i * 16 + lr];
        if constexpr (kPrio > 0) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            if (kPrio == 1 && i == RB / 2) __builtin_amdgcn_s_setprio(0);
            if (i == RB / 2 && kt + 1 < kt1) store(next, buf ^ 1);
#pragma unroll
            for (int j = 0; j < CB; ++j)
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[p][i]),
                                                                        __builtin_bit_cast(bf16x8, bq[j]), acc[i][j],
                                                                        0, 0, 0);
        }
        if constexpr (kPrio == 2) __builtin_amdgcn_s_setprio(0);
        lds_barrier();
    };

    Regs r0, r1;
    load(r0, kt0);
    if (kt0 + 1 < kt1) load(r1, kt0 + 1);
    store(r0, kt0 & 1);
    lds_barrier();
    // lgkmcnt(0) before the loop: a kernel-argument scalar load still pending
    // at the loop header made the compiler wait for all sixteen operand reads
    // (lgkmcnt(0)) before the first MFMA of every other stage, instead of for
    // the few that MFMA reads.  C4 162.1 -> 159.7 us (builds interleaved).
    __builtin_amdgcn_s_waitcnt(0xC07F);
    for (int kt = kt0; kt < kt1; kt += 2) {
        stage(kt, r1, r0);
        if (kt + 1 < kt1) stage(kt + 1, r0, r1);
    }

    // D layout of 16x16x32: lane l, element r -> row 4*(l/16) + r, column l%16.
    const int klo = kt0 * kB3BK, khi = (kt1 * kB3BK) < K ? (kt1 * kB3BK) : K;
    const float s_all = PT ? S[0] : 1.0f;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int n = n0 + wn * 16 * CB + j * 16 + lr;
            if (n >= N) continue;
            const float bv = (bias && KS == 1) ? bias[n] : 0.0f;
            float* out = KS == 1 ? y : part + (int64_t)split * M * N;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 16 * RB + i * 16 + lkg * 4 + r;
                if (m < M) {
                    // INT4 codes entered as 16q: an exact division by 16.
                    float v = BITS == 4 ? acc[i][j][r] * 0.0625f : (PT ? acc[i][j][r] * s_all : acc[i][j][r]);
                    if (!isfinite(v)) v = output_exact<BITS>(x + (int64_t)m * K, W, S, mode, Kpad, RQ, n, klo, khi);
                    out[(int64_t)m * N + n] = (bias && KS == 1) ? v + bv : v;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Skinny INT4 forward on the bf16 matrix cores: batches of a few to 32 rows
// (src/quantization.cpp:199-206 for those shapes).
//
// Each 16 rows of the batch are the rows of one v_mfma_f32_16x16x32_bf16
// (rows past M are zeros; MB such row blocks share every B operand), with the
// three-term split of k_gemm3: A = x * s as three bf16 planes, B = codes
// (exact in bf16), fp32 accumulation.  A workgroup owns C column blocks of 16
// (2C strips of one scale column, so one x * s split serves all of them) over
// all of K, or over one of S equal ranges of 32-row k blocks (split K, for
// weights too narrow to fill the device: the partial sums go to a workspace
// and k_skinny_reduce adds them in split order).  Its NW wavefronts take the
// k blocks of its range in turn and are summed through LDS at the end.  The
// order of every sum depends on the K range and NW only, not on C, MB or the
// number of weights.
//
// B operands straight from the weight's k-octet copy, without LDS: block
// (column block, k block) is 256 bytes whose dword t holds rows 8 (t >> 4) ..
// + 7 of column t & 15, the B operand of lane t as it stands.  Each lane loads
// one dword per k block; the codes are read once, in 256-byte runs per
// wavefront.  (From the strip layout, where a dword holds one row of eight
// columns, the same operand took an 8x8 nibble transpose across eight lanes:
// three DPP exchanges, rotates and bit selects per dword, 10-13% of the gate
// projection's time at 5 to 16 rows.)
// ---------------------------------------------------------------------------

// Lane l's value from lane l ^ 8 within its 16-lane row (DPP row_ror:8): the
// half-row forms exchange the two halves of an A operand with it.
__device__ __forceinline__ uint32_t dpp_xor8(uint32_t v) { return __builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true); }

struct SkinnyArgs {
    const float* x;  // [M, K]
    int M, K, N;
    const uint4* W[3];  // NG weights of equal shape (gate, up), or (NG == 1) nw weights side by side
    const float* SC[3];
    const float* bias[3];
    int spc, Kpad, RQ;
    FastDiv wpc;  // workgroups (column groups) per scale column
    float* y;     // [M, ldy]
    float* part;  // split K: [NG][2^slog][M][N] partial sums
    int nblk;     // grid size
    int slog;     // log2 of the number of K ranges
    int sbs;      // super-blocks (128 rows) per K range
    // Whole-K form only: weight w of nw side by side writes columns
    // w * N .. w * N + N - 1 of y; NORM: the RMSNorm weight and epsilon.
    int ldy;
    int wgpw;     // workgroups per weight
    FastDiv wgd;  // division by wgpw
    const float* gamma;
    float eps;
    int xlog;     // log2 of the device's XCD count
    int ko;       // byte offset / 256 of each weight's k-octet copy (I4Geom::koct_off)
};

// What the skinny kernels' prologues need before their first loads travels
// ahead of the SkinnyArgs copy as scalar kernel arguments, which gfx950
// preloads into SGPRs (as for k_gemv: a by-value struct is never preloaded).
// Kpad is 4 * RQ; pk packs the XCD shift (bits 0-7), the scale-column
// divider's shift (8-15) and log2 of the K ranges (16-23); ko is the k-octet
// copy's offset (fourteen dwords in all, what gfx950 preloads).
struct SkinnyHot {
    const float* x;
    const uint4* W0;
    const float* S0;
    int M, K, RQ, nblk, pk;
    uint32_t wpcm;
    int sbs, ko;
};
inline SkinnyHot skinny_hot(const SkinnyArgs& a) {
    SkinnyHot h;
    h.x = a.x, h.W0 = a.W[0], h.S0 = a.SC[0];
    h.M = a.M, h.K = a.K, h.RQ = a.RQ, h.nblk = a.nblk;
    h.pk = a.xlog | (a.wpc.l << 8) | (a.slog << 16);
    h.wpcm = a.wpc.m;
    h.sbs = a.sbs;
    h.ko = a.ko;
    return h;
}
#define SGQ_SKINNY_HOT_PARAMS                                                                                    \
    const float *__restrict__ hx, const uint4 *__restrict__ hW0, const float *__restrict__ hS0, int hM, int K, \
        int RQ, int nblk, int pk, uint32_t wpcm, int sbs, int ko
#define SGQ_SKINNY_HOT_ARGS(h) h.x, h.W0, h.S0, h.M, h.K, h.RQ, h.nblk, h.pk, h.wpcm, h.sbs, h.ko
__device__ __forceinline__ FastDiv fastdiv_of(uint32_t m, int l) {
    FastDiv f;
    f.m = m, f.l = l;
    return f;
}

// The whole-K form for one row block (5..16 rows over wide weights, no K
// split): NW = 16 wavefronts take 32-row k blocks in turn, U of them per
// batch of loads, and every load of a batch is issued before the first is
// used.  The codes come from the weight's k-octet copy: lane t of a wavefront
// loads dword t of block (column block, kb), rows 8 (t >> 4) .. + 7 of column
// t & 15, which is its B operand as it stands (256 contiguous bytes per
// wavefront load, no exchange between lanes); x and the scales are loaded per
// k block.  NG == 2:
// the gated MLP, h = silu(gate + bias) * (up + bias2).  NG == 1 runs a.wgpw
// workgroups per weight over nw weights of one shape side by side (a LLaMA
// block's q, k and v).  XA: x rows are 16-byte aligned and K % 4 == 0 (float4
// loads); otherwise one float per load.
//
// NORM: the input rows are RMS-normalised first (rms_norm, src/ops.cpp:
// 1532-1556: x * inv_rms * gamma, inv_rms = 1 / sqrt(sum(x^2) / K + eps)), as
// in the GEMV: A = x * (gamma * s), and the epilogue multiplies by inv_rms,
// one factor per row, from the sum of x^2 over the rows the workgroup reads.
//
// HALF (M <= 8): A rows 8..15 are not outputs, so their lanes do half of the
// real rows' work.  Lane n < 8 loads and splits k 8g .. 8g + 3 of row n, lane
// n + 8 k 8g + 4 .. 8g + 7 of the same row, and a row_ror:8 exchange gives
// lane n the upper half of its operand.  The bf16 planes are the same bits as
// without HALF; A rows 8..15 then hold copies whose outputs are never read.
template <int NW, int U, int C, int NG, bool XA, bool NORM, bool HALF>
__global__ __launch_bounds__(NW * 64) void k_skinny3(SGQ_SKINNY_HOT_PARAMS, const SkinnyArgs a) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int Kpad = 4 * RQ;
    const int nkb = (Kpad + 31) >> 5;  // k blocks of 32 rows (KB of the k-octet copy)
    // One weight without the norm (every linear call): the preloaded
    // pointers alone, so that no select waits for the SkinnyArgs copy.
    constexpr bool ONE = NG == 1 && !NORM;
    const int vv = xcd_swizzle(blockIdx.x, nblk, pk & 255);
    const int wt = (NG == 1 && !ONE) ? a.wgd.div(vv) : 0;  // weight of the side-by-side set
    const int v = vv - wt * a.wgpw;
    const int blk0 = v * C;  // first column block
    const int sc = fastdiv_of(wpcm, (pk >> 8) & 255).div(v);
    const uint4* Wq[NG];
    const float* SCq[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        const int wi = NG == 1 ? wt : q;
        Wq[q] = (ONE || wi == 0) ? hW0 : a.W[wi];
        SCq[q] = (ONE || wi == 0) ? hS0 : a.SC[wi];
    }
    __amdgpu_buffer_rsrc_t rW[NG], rS[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        // Column blocks blk0 .. blk0 + C - 1 of the k-octet copy, C * nkb
        // blocks of 256 bytes from block blk0 * nkb.
        rW[q] = make_rsrc(Wq[q] + ((int64_t)ko + (int64_t)blk0 * nkb) * 16, (uint32_t)C * (uint32_t)nkb * 256u);
        rS[q] = make_rsrc(SCq[q] + (int64_t)sc * Kpad, (uint32_t)Kpad * 4u);
    }
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(hx, (uint32_t)hM * (uint32_t)K * 4u);
    __amdgpu_buffer_rsrc_t rG;
    if constexpr (NORM) rG = make_rsrc(a.gamma, (uint32_t)K * 4u);
    float sq = 0.0f;  // NORM: sum of x^2 of this lane's row over its k
    int wv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) wv[c] = c * nkb * 256 + 4 * lane;
    constexpr int XV = HALF ? 4 : 8;  // x values per lane and k block
    const int xr = HALF ? (n & 7) : n, xk = HALF ? 4 * (n >> 3) : 0;
    const bool row_live = xr < hM;
    const int xrow = xr * K * 4;
    floatx4 acc[NG][C];
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[q][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    // K blocks kb0, kb0 + NW, ..., U of them per batch.  A block past the end
    // reads x and the scales as zeros (its code dwords are zeros past the
    // range, else another column block's, multiplied by zero), so partial
    // batches need no branch.
    for (int kb0 = wave; kb0 < nkb; kb0 += NW * U) {
        uint32_t w[U][NG][C];
        float xv[U][XV], sv[U][NG][XV], gv[NORM ? U : 1][XV];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = kb0 + u * NW;
#pragma unroll
            for (int q = 0; q < NG; ++q)
#pragma unroll
                for (int c = 0; c < C; ++c)
                    w[u][q][c] = buf_load4_stream(rW[q], wv[c], kb * 256);
            const int k0 = kb * 32 + 8 * g + xk;
#pragma unroll
            for (int h = 0; h < XV / 4; ++h) {
                const int kk = k0 + 4 * h;
                if constexpr (XA) {
                    const float4 xq = buf_load4f<true>(rX, row_live && kk < K ? xrow + kk * 4 : kOobOff, 0);
                    xv[u][4 * h] = xq.x, xv[u][4 * h + 1] = xq.y, xv[u][4 * h + 2] = xq.z, xv[u][4 * h + 3] = xq.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        xv[u][4 * h + i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rX, row_live && kk + i < K ? xrow + (kk + i) * 4 : kOobOff, 0, 0));
                }
#pragma unroll
                for (int q = 0; q < NG; ++q) {
                    const float4 s4 = buf_load4f<true>(rS[q], kk * 4, 0);
                    sv[u][q][4 * h] = s4.x, sv[u][q][4 * h + 1] = s4.y, sv[u][q][4 * h + 2] = s4.z,
                                 sv[u][q][4 * h + 3] = s4.w;
                }
                if constexpr (NORM) {
                    const float4 g4 = buf_load4f<XA>(rG, kk * 4, 0);
                    gv[u][4 * h] = g4.x, gv[u][4 * h + 1] = g4.y, gv[u][4 * h + 2] = g4.z, gv[u][4 * h + 3] = g4.w;
                }
            }
        }
        // Every load of the batch is issued before the first is used.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (NORM) {
#pragma unroll
                for (int i = 0; i < XV; ++i) sq = fmaf(xv[u][i], xv[u][i], sq);
            }
#pragma unroll
            for (int q = 0; q < NG; ++q) {
                float xs[XV];
#pragma unroll
                for (int i = 0; i < XV; ++i) xs[i] = NORM ? xv[u][i] * (gv[u][i] * sv[u][q][i]) : xv[u][i] * sv[u][q][i];
                uint4 ah, am, al;
                if constexpr (HALF) {
                    uint2 h2, m2, l2;
                    split3_4(xs, h2, m2, l2);
                    ah = make_uint4(h2.x, h2.y, dpp_xor8(h2.x), dpp_xor8(h2.y));
                    am = make_uint4(m2.x, m2.y, dpp_xor8(m2.x), dpp_xor8(m2.y));
                    al = make_uint4(l2.x, l2.y, dpp_xor8(l2.x), dpp_xor8(l2.y));
                } else {
                    split3(xs, ah, am, al);
                }
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    const bf16x8 b = nibbles_bf16x16(w[u][q][c]);
                    acc[q][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah), b, acc[q][c], 0, 0, 0);
                    acc[q][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, am), b, acc[q][c], 0, 0, 0);
                    acc[q][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al), b, acc[q][c], 0, 0, 0);
                }
            }
        }
    }
    // NORM: the rows' sums of x^2 added in a fixed order: the four lane
    // groups of a wavefront by lane exchanges, then the wavefronts through
    // LDS; inv_rms per row.
    __shared__ float sqr[NORM ? NW : 1][16];
    __shared__ float inv_rms[16];
    if constexpr (NORM) {
        sq += xor_lane<32>(sq, lane);
        sq += xor_lane<16>(sq, lane);
        if constexpr (HALF) sq += xor_lane<8>(sq, lane);  // the two halves of a row's k
        if (lane < 16) sqr[wave][lane] = sq;
        __syncthreads();
        if (threadIdx.x < 16) {
            float ss = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) ss += sqr[w2][threadIdx.x];
            inv_rms[threadIdx.x] = 1.0f / sqrtf(ss / (float)K + a.eps);
        }
    }
    // Accumulator element r of lane l is output row 4 * (l >> 4) + r of
    // column lane l & 15 of its block.  The wavefronts' partial tiles are
    // summed in wavefront order (deterministic), one weight at a time through
    // the same LDS; thread t keeps output t (t + NW * 64, ...) of each.
    constexpr int OPT = (256 * C + NW * 64 - 1) / (NW * 64);
    __shared__ float red[NW][C][4][64];
    float o[NG][OPT];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        if (q > 0) __syncthreads();  // every thread has read the previous weight's partials
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][c][r][lane] = acc[q][c][r];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < OPT; ++i) {
            const int t = threadIdx.x + i * NW * 64;
            const int c = t >> 8, m = (t >> 4) & 15, sl = t & 15;
            const int col = 16 * (blk0 + c) + sl;
            const int strip = col >> 3, el = col & 7;
            float s = 0.0f;
            if (t < 256 * C && m < a.M && col < a.N) {
#pragma unroll
                for (int w2 = 0; w2 < NW; ++w2) s += red[w2][c][m & 3][16 * (m >> 2) + sl];
                s *= 0.0625f;  // the codes entered as 16q
                // h + m + l turns an infinite x * s into inf - inf: recompute
                // a non-finite total as the reference's k-order sum.
                if (!isfinite(s))
                    s = i4_column_exact<NORM>(Wq[q], SCq[q], strip, el, a.spc, a.Kpad, a.RQ, a.x + (int64_t)m * K,
                                              a.gamma, 0, K);
                if constexpr (NORM) s = s * inv_rms[m];
                const float* bq = a.bias[NG == 1 ? wt : q];
                if (bq) s = s + bq[col];
            }
            o[q][i] = s;
        }
    }
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
        const int t = threadIdx.x + i * NW * 64;
        const int c = t >> 8, m = (t >> 4) & 15, sl = t & 15;
        const int col = 16 * (blk0 + c) + sl;
        if (t < 256 * C && m < a.M && col < a.N) {
            float r0 = o[0][i];
            if constexpr (NG == 2) r0 = silu_f32(o[0][i]) * o[1][i];
            a.y[(int64_t)m * a.ldy + (int64_t)wt * a.N + col] = r0;
        }
    }
}


// The super-block form (any row blocks, optional K split).  NG == 2: the gated MLP, gate and up blocks of the same columns in one
// workgroup, h = silu(gate + bias) * (up + bias2) (split K: in
// k_skinny_reduce).  XA: x rows are 16-byte aligned and K % 4 == 0 (float4
// loads); otherwise one float per load.  MB: row blocks of 16 (M <= 16 MB).
//
// The K range is walked in super-blocks of 128 rows, wavefront w taking
// super-blocks w, w + NW, ...  A super-block is four k blocks of 32 rows of
// the weight's k-octet copy: for k block i = 0..3, lane t loads dword t of
// block (column block, 4 sb + i), rows 8 (t >> 4) .. + 7 of column t & 15,
// which is the B operand of MFMA i as it stands (four 256-byte runs per
// wavefront and column block, 1 KB contiguous), and x rows 32 i + 8 g ..
// 32 i + 8 g + 7 of its batch row as two quads, the matching A operand.  The
// scales of the workgroup's K range sit in LDS (read once, coalesced); the
// next super-block's codes and x are loaded while the current one is
// computed.
template <int NW, int C, int NG, bool XA, int MB, bool HALF>
struct SkinnyRegs {
    uint4 w[NG][C];                // dword i: the B operand of k block i
    float4 xq[MB][HALF ? 4 : 8];  // x quads of each batch row (HALF: half of them)
};

// Quad t of a lane covers k block i = t / 2, rows 32 i + 8 g + 4 (t % 2) ..
// + 3.  HALF (one row block, M <= 8): as in k_skinny3, lane n < 8 takes the
// first quad of each k block of row n (quad t is k block t) and lane n + 8 the
// second; a row_ror:8 exchange completes each A operand (the same bf16
// planes).
template <int NW, int C, int NG, bool XA, int MB, bool SPLIT, bool HALF>
__global__ __launch_bounds__(NW * 64) void k_skinny_sb(SGQ_SKINNY_HOT_PARAMS, const SkinnyArgs a) {
    static_assert(!HALF || MB == 1, "the half-row form has one row block");
    constexpr int XT = HALF ? 4 : 8;  // x quads per lane, row block and super-block
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int Kpad = 4 * RQ, slog = (pk >> 16) & 255;
    const int nkb = (Kpad + 31) >> 5;  // k blocks of 32 rows (KB of the k-octet copy)
    // Workgroup v: K range v % S of column group v / S (the ranges of one
    // column group are neighbours, so they share an XCD's L2 for the scales).
    const int v = xcd_swizzle(blockIdx.x, nblk, pk & 255);
    const int split = SPLIT ? (v & ((1 << slog) - 1)) : 0;
    const int cgrp = SPLIT ? (v >> slog) : v;
    const int blk0 = cgrp * C;  // first column block
    const int sc = fastdiv_of(wpcm, (pk >> 8) & 255).div(cgrp);
    const int nsb = (Kpad + kSkinnySB - 1) / kSkinnySB;
    const int sb_lo = SPLIT ? split * sbs : 0;
    const int sb_hi = SPLIT ? min(nsb, sb_lo + sbs) : nsb;
    const int row0 = sb_lo * kSkinnySB;  // first row of the range

    // The range's scales (rows row0 .. row0 + rows - 1 of the scale column,
    // zeros past Kpad) are loaded ahead of the first super-block's codes and
    // x, so that storing them into LDS waits for them alone.
    constexpr int SCI = kSkinnyRangeRows / 4 / (NW * 64);  // float4 per thread and weight
    static_assert(SCI * NW * 64 * 4 == kSkinnyRangeRows, "the scale rows spread evenly");
    __shared__ float4 ssc[NG][kSkinnyRangeRows / 4];
    const int rows4 = (sb_hi - sb_lo) * (kSkinnySB / 4);
    float4 sreg[NG][SCI];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        const __amdgpu_buffer_rsrc_t rS = make_rsrc((q == 0 ? hS0 : a.SC[q]) + (int64_t)sc * Kpad, (uint32_t)Kpad * 4u);
#pragma unroll
        for (int it = 0; it < SCI; ++it) {
            const int r4 = threadIdx.x + it * NW * 64;
            sreg[q][it] = buf_load4f<true>(rS, r4 < rows4 ? (row0 + 4 * r4) * 4 : kOobOff, 0);
        }
    }

    __amdgpu_buffer_rsrc_t rW[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q)
        rW[q] = make_rsrc((q == 0 ? hW0 : a.W[q]) + ((int64_t)ko + (int64_t)blk0 * nkb) * 16,
                          (uint32_t)C * (uint32_t)nkb * 256u);
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(hx, (uint32_t)hM * (uint32_t)K * 4u);
    int wv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) wv[c] = c * nkb * 256 + 4 * lane;
    const int xr = HALF ? (n & 7) : n, hq = HALF ? (n >> 3) : 0;
    bool row_live[MB];
    int xrow[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        row_live[b] = xr + 16 * b < hM;
        xrow[b] = row_live[b] ? (xr + 16 * b) * K * 4 : 0;
    }
    // Quad t of a lane: k block t / 2 (HALF: t) of the super-block, rows
    // 8 g + 4 (t % 2) (HALF: 8 g + 4 hq) .. + 3 of it.
    auto qrow = [&](int t) { return HALF ? 32 * t + 8 * g + 4 * hq : 32 * (t >> 1) + 8 * g + 4 * (t & 1); };

    // Loads of super-block sb; one past the range reads x as zeros (and codes
    // that are then multiplied by zero).
    auto load = [&](SkinnyRegs<NW, C, NG, XA, MB, HALF>& r, int sb) {
        const bool in = sb < sb_hi;
#pragma unroll
        for (int q = 0; q < NG; ++q)
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const int so = sb * (4 * 256);
                r.w[q][c] = make_uint4(buf_load4_stream(rW[q], wv[c], so), buf_load4_stream(rW[q], wv[c], so + 256),
                                       buf_load4_stream(rW[q], wv[c], so + 512), buf_load4_stream(rW[q], wv[c], so + 768));
            }
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int t = 0; t < XT; ++t) {
                const int kk = sb * kSkinnySB + qrow(t);
                if constexpr (XA) {
                    r.xq[b][t] = buf_load4f<true>(rX, in && row_live[b] && kk < K ? xrow[b] + kk * 4 : kOobOff, 0);
                } else {
                    // One float per load from any 4-byte address; the row's
                    // tail and the rows past M read as zeros by their offset.
                    const int base = in && row_live[b] ? xrow[b] + kk * 4 : kOobOff;
                    float f[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        f[i] = __uint_as_float(
                            __builtin_amdgcn_raw_buffer_load_b32(rX, kk + i < K ? base + 4 * i : kOobOff, 0, 0));
                    r.xq[b][t] = make_float4(f[0], f[1], f[2], f[3]);
                }
            }
    };

    floatx4 acc[NG][MB][C];
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int c = 0; c < C; ++c) acc[q][b][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](SkinnyRegs<NW, C, NG, XA, MB, HALF>& r, int sb) {
        // A super-block past the range has x = 0; its scale reads stay inside
        // the range's LDS rows.
        const int lr = (min(sb, sb_hi - 1) - sb_lo) * (kSkinnySB / 4);
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            float4 s4[XT];
#pragma unroll
            for (int t = 0; t < XT; ++t) s4[t] = ssc[q][lr + qrow(t) / 4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint4 ah[MB], am[MB], al[MB];
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    // k block i: quads 2i, 2i + 1 (HALF: quad i, the other half in lane n ^ 8).
                    float xs[8];
#pragma unroll
                    for (int h = 0; h < (HALF ? 1 : 2); ++h)
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int t = HALF ? i : 2 * i + h;
                            xs[4 * h + u] = f4get(r.xq[b][t], u) * f4get(s4[t], u);
                        }
                    if constexpr (HALF) {
                        uint2 h2, m2, l2;
                        split3_4(xs, h2, m2, l2);
                        ah[b] = make_uint4(h2.x, h2.y, dpp_xor8(h2.x), dpp_xor8(h2.y));
                        am[b] = make_uint4(m2.x, m2.y, dpp_xor8(m2.x), dpp_xor8(m2.y));
                        al[b] = make_uint4(l2.x, l2.y, dpp_xor8(l2.x), dpp_xor8(l2.y));
                    } else {
                        split3(xs, ah[b], am[b], al[b]);
                    }
                }
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    const uint32_t wd = i == 0 ? r.w[q][c].x : (i == 1 ? r.w[q][c].y : (i == 2 ? r.w[q][c].z : r.w[q][c].w));
                    const bf16x8 bq = nibbles_bf16x16(wd);
#pragma unroll
                    for (int b = 0; b < MB; ++b) {
                        acc[q][b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[b]), bq,
                                                                               acc[q][b][c], 0, 0, 0);
                        acc[q][b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, am[b]), bq,
                                                                               acc[q][b][c], 0, 0, 0);
                        acc[q][b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[b]), bq,
                                                                               acc[q][b][c], 0, 0, 0);
                    }
                }
            }
        }
    };

    // Two register sets: the loads of the next super-block are in flight
    // while the current one is computed.
    SkinnyRegs<NW, C, NG, XA, MB, HALF> ra, rb;
    int sb = sb_lo + wave;
    load(ra, sb);
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
        for (int it = 0; it < SCI; ++it) {
            const int r4 = threadIdx.x + it * NW * 64;
            if (r4 < rows4) ssc[q][r4] = sreg[q][it];
        }
    lds_barrier();  // the scales are in LDS (the codes and x loads stay in flight)
    for (; sb < sb_hi; sb += 2 * NW) {
        load(rb, sb + NW);
        compute(ra, sb);
        if (sb + NW >= sb_hi) break;  // wave-uniform: no empty super-block computed
        load(ra, sb + 2 * NW);
        compute(rb, sb + NW);
    }

    // Accumulator element r of lane l is output row 4 * (l >> 4) + r (of its
    // row block) of column lane l & 15 of its column block.  The wavefronts'
    // partial tiles are summed in wavefront order (deterministic), one weight
    // and row block at a time through LDS; thread t keeps output t
    // (t + NW * 64, ...) of each.
    constexpr int OPT = (256 * C + NW * 64 - 1) / (NW * 64);
    __shared__ float red[NW][C][4][64];
    const int klo = row0, khi = min(K, sb_hi * kSkinnySB);
    float o[NG][MB][OPT];
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (q > 0 || b > 0) __syncthreads();  // every thread has read the previous tile's partials
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave][c][r][lane] = acc[q][b][c][r];
            __syncthreads();
#pragma unroll
            for (int i = 0; i < OPT; ++i) {
                const int t = threadIdx.x + i * NW * 64;
                const int c = t >> 8, mr = (t >> 4) & 15, sl = t & 15;
                const int m = mr + 16 * b;
                const int col = 16 * (blk0 + c) + sl;
                const int strip = col >> 3, el = col & 7;
                float s = 0.0f;
                if (t < 256 * C && m < a.M && col < a.N) {
#pragma unroll
                    for (int w2 = 0; w2 < NW; ++w2) s += red[w2][c][mr & 3][16 * (mr >> 2) + sl];
                    s *= 0.0625f;  // the codes entered as 16q
                    // h + m + l turns an infinite x * s into inf - inf: recompute
                    // a non-finite total as the reference's k-order sum.
                    if (!isfinite(s))
                        s = i4_column_exact<false>(a.W[q], a.SC[q], strip, el, a.spc, a.Kpad, a.RQ,
                                                   a.x + (int64_t)m * K, nullptr, klo, khi);
                    if (!SPLIT && a.bias[q]) s = s + a.bias[q][col];
                }
                o[q][b][i] = s;
            }
        }
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < OPT; ++i) {
            const int t = threadIdx.x + i * NW * 64;
            const int c = t >> 8, m = ((t >> 4) & 15) + 16 * b, sl = t & 15;
            const int col = 16 * (blk0 + c) + sl;
            if (t < 256 * C && m < a.M && col < a.N) {
                const int64_t at = (int64_t)m * a.N + col;
                if constexpr (SPLIT) {
                    const int64_t MN = (int64_t)a.M * a.N;
#pragma unroll
                    for (int q = 0; q < NG; ++q) a.part[((int64_t)q << a.slog | split) * MN + at] = o[q][b][i];
                } else {
                    float r0 = o[0][b][i];
                    if constexpr (NG == 2) r0 = silu_f32(o[0][b][i]) * o[1][b][i];
                    a.y[at] = r0;
                }
            }
        }
}

// INT8 batches of a few to 128 rows of little work on the bf16 matrix cores
// (src/quantization.cpp:189-197 for those shapes), the INT8 counterpart of
// k_skinny3.  Each 16 rows of a row tile are the rows of one
// v_mfma_f32_16x16x32_bf16 (MB row blocks share every B operand), with the
// three-term split of k_gemm3: A = x (per tensor; the epilogue multiplies by
// scales[0]) or x * scales[k] (per channel) as three bf16 planes, B = codes
// (exact in bf16), fp32 accumulation.  A workgroup owns C column blocks of
// 16 (4C strips) and MB row blocks over all of K; its NW wavefronts take the
// 32-row k blocks in turn, U per batch of loads, every load of a batch issued
// before the first is used, and are summed through LDS in wavefront order.
// The order of every sum depends on K and NW only.
//
// B operand straight from the strip layout, without a transpose: dword d of
// an INT8 chunk is column 4j + d over the chunk's four rows, so lane l
// (g = l >> 4; column n = l & 15 of its block: strip n >> 2, dword n & 3)
// takes that dword of row quads 2g and 2g + 1 of the k block, rows
// 8g .. 8g + 7 of its column.  A block past the end reads x (and per-channel
// scales) as zeros; its code dwords are whatever follows and are multiplied
// by zero.
struct Skinny8Args {
    const float* x;  // [M, K]
    int M, K, N;
    const uint4* W;
    const float* S;  // per tensor: scales[0]; per channel: scales[K]
    const float* bias;
    int RQ, NS, Kpad;
    int ncg;      // column groups (workgroups per row tile)
    FastDiv cgd;  // division by ncg
    float* y;
    int nblk;
    int xlog;  // log2 of the device's XCD count
};
// k_skinny8's prologue fields as preloaded scalar arguments (as SkinnyHot):
// Kpad is 4 * RQ; pk packs the XCD shift (bits 0-7) and the column-group
// divider's shift (8-15).
struct Skinny8Hot {
    const float* x;
    const uint4* W;
    const float* S;
    int M, K, RQ, NS, nblk, pk;
    uint32_t cgdm;
    int ncg;
};
inline Skinny8Hot skinny8_hot(const Skinny8Args& a) {
    Skinny8Hot h;
    h.x = a.x, h.W = a.W, h.S = a.S;
    h.M = a.M, h.K = a.K, h.RQ = a.RQ, h.NS = a.NS, h.nblk = a.nblk;
    h.pk = a.xlog | (a.cgd.l << 8);
    h.cgdm = a.cgd.m;
    h.ncg = a.ncg;
    return h;
}

// HALF (one row block, M <= 8): lane n < 8 loads and splits k 8g .. 8g + 3
// of row n, lane n + 8 k 8g + 4 .. 8g + 7 of the same row, and a row_ror:8
// exchange completes each A operand (the same bf16 planes), as in k_skinny3.
template <int NW, int U, int C, int MB, bool PT, bool XA, bool HALF>
__global__ __launch_bounds__(NW * 64) void k_skinny8(const float* __restrict__ hx, const uint4* __restrict__ hW,
                                                        const float* __restrict__ hS, int hM, int K, int RQ, int NS,
                                                        int nblk, int pk, uint32_t cgdm, int ncg,
                                                        const Skinny8Args a) {
    static_assert(!HALF || MB == 1, "the half-row form has one row block");
    constexpr int XV = HALF ? 4 : 8;  // x values per lane, row block and k block
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int Kpad = 4 * RQ;
    const int v = xcd_swizzle(blockIdx.x, nblk, pk & 255);  // row tile major: an XCD's workgroups share x rows
    const int rt = fastdiv_of(cgdm, (pk >> 8) & 255).div(v), cg = v - rt * ncg;
    const int m0 = rt * 16 * MB, s0 = cg * 4 * C;
    const int mrows = min(16 * MB, hM - m0), nstr = min(4 * C, NS - s0);
    // Rows past M and strips past NS lie past the ends of these buffers and read as zeros.
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(hW + (int64_t)s0 * RQ, (uint32_t)nstr * (uint32_t)RQ * 16u);
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(hx + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t rS = make_rsrc(hS, PT ? 4u : (uint32_t)K * 4u);
    int wv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) wv[c] = ((4 * c + (n >> 2)) * RQ + 2 * g) * 16 + (n & 3) * 4;
    const int xr = HALF ? (n & 7) : n, xk = HALF ? 4 * (n >> 3) : 0;
    floatx4 acc[MB][C];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[b][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int nkb = (Kpad + 31) >> 5;
    for (int kb0 = wave; kb0 < nkb; kb0 += NW * U) {
        uint32_t w[U][C][2];
        float xv[U][MB][XV], sv[U][XV];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = kb0 + u * NW;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                w[u][c][0] = __builtin_amdgcn_raw_buffer_load_b32(rW, wv[c], kb * 128, 0);
                w[u][c][1] = __builtin_amdgcn_raw_buffer_load_b32(rW, wv[c] + 16, kb * 128, 0);
            }
            const int k0 = kb * 32 + 8 * g + xk;
#pragma unroll
            for (int h = 0; h < XV / 4; ++h) {
                const int kk = k0 + 4 * h;
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    const int xo = (16 * b + xr) * K * 4;
                    if constexpr (XA) {
                        const float4 xq = buf_load4f<true>(rX, kk < K ? xo + kk * 4 : kOobOff, 0);
                        xv[u][b][4 * h] = xq.x, xv[u][b][4 * h + 1] = xq.y, xv[u][b][4 * h + 2] = xq.z,
                                     xv[u][b][4 * h + 3] = xq.w;
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            xv[u][b][4 * h + i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                rX, kk + i < K ? xo + (kk + i) * 4 : kOobOff, 0, 0));
                    }
                }
                if constexpr (!PT) {
                    const float4 sq = buf_load4f<XA>(rS, kk * 4, 0);
                    sv[u][4 * h] = sq.x, sv[u][4 * h + 1] = sq.y, sv[u][4 * h + 2] = sq.z, sv[u][4 * h + 3] = sq.w;
                }
            }
        }
        // Every load of the batch is issued before the first is used.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            bf16x8 bq[C];
#pragma unroll
            for (int c = 0; c < C; ++c) {
                // bytes of the column's dword in each chunk: k = 0..3, then 4..7
                const uint32_t lo = w[u][c][0], hi = w[u][c][1];
                const uint4 bb = make_uint4(pack_hi16(cvt_sbyte<0>(lo), cvt_sbyte<1>(lo)),
                                            pack_hi16(cvt_sbyte<2>(lo), cvt_sbyte<3>(lo)),
                                            pack_hi16(cvt_sbyte<0>(hi), cvt_sbyte<1>(hi)),
                                            pack_hi16(cvt_sbyte<2>(hi), cvt_sbyte<3>(hi)));
                bq[c] = __builtin_bit_cast(bf16x8, bb);
            }
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                float xs[XV];
#pragma unroll
                for (int i = 0; i < XV; ++i) xs[i] = PT ? xv[u][b][i] : xv[u][b][i] * sv[u][i];
                uint4 ah, am, al;
                if constexpr (HALF) {
                    uint2 h2, m2, l2;
                    split3_4(xs, h2, m2, l2);
                    ah = make_uint4(h2.x, h2.y, dpp_xor8(h2.x), dpp_xor8(h2.y));
                    am = make_uint4(m2.x, m2.y, dpp_xor8(m2.x), dpp_xor8(m2.y));
                    al = make_uint4(l2.x, l2.y, dpp_xor8(l2.x), dpp_xor8(l2.y));
                } else {
                    split3(xs, ah, am, al);
                }
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah), bq[c], acc[b][c], 0, 0, 0);
                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, am), bq[c], acc[b][c], 0, 0, 0);
                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al), bq[c], acc[b][c], 0, 0, 0);
                }
            }
        }
    }
    // Accumulator element r of lane l is output row 4 * (l >> 4) + r of
    // column l & 15 of its block.  The wavefronts' partial tiles are summed
    // in wavefront order through LDS; thread t then owns output t
    // (t + NW * 64, ...): block bc = t >> 8, row (t >> 4) & 15, column t & 15.
    constexpr int NBC = MB * C;
    constexpr int OPT = (256 * NBC + NW * 64 - 1) / (NW * 64);
    __shared__ float red[NW][NBC][4][64];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][b * C + c][r][lane] = acc[b][c][r];
    __syncthreads();
    const float s_all = PT ? a.S[0] : 1.0f;
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
        const int t = threadIdx.x + i * NW * 64;
        const int bc = t >> 8, mi = (t >> 4) & 15, nl = t & 15;
        const int m = m0 + 16 * (bc / C) + mi, col = 16 * (cg * C + bc % C) + nl;
        if (t < 256 * NBC && m < a.M && col < a.N) {
            float s = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) s += red[w2][bc][mi & 3][16 * (mi >> 2) + nl];
            if constexpr (PT) s = s * s_all;
            // h + m + l turns an infinite x into inf - inf: recompute a
            // non-finite total as the reference's k-order sum.
            if (!isfinite(s)) s = output_exact<8>(a.x + (int64_t)m * K, a.W, a.S, PT ? 1 : 0, a.Kpad, a.RQ, col, 0, K);
            a.y[(int64_t)m * a.N + col] = a.bias ? s + a.bias[col] : s;
        }
    }
}

// The skinny kernel's K ranges added in range order, plus the bias; NG == 2:
// h = silu(gate + bias) * (up + bias2).  part is [NG][S][M*N].
template <int NG>
__global__ __launch_bounds__(kThreads) void k_skinny_reduce(const float* __restrict__ part, int S, int64_t MN, int N,
                                                            const float* __restrict__ bias,
                                                            const float* __restrict__ bias2, float* __restrict__ y) {
    for (int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; o < MN; o += (int64_t)gridDim.x * blockDim.x) {
        float r[NG];
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            float t[kSkinnyMaxSplits];
#pragma unroll
            for (int sp = 0; sp < kSkinnyMaxSplits; ++sp)  // all loads first
                t[sp] = sp < S ? part[((int64_t)q * S + sp) * MN + o] : 0.0f;
            float v = 0.0f;
#pragma unroll
            for (int sp = 0; sp < kSkinnyMaxSplits; ++sp)
                if (sp < S) v += t[sp];
            const float* bq = q == 0 ? bias : bias2;
            if (bq) v = v + bq[o % N];
            r[q] = v;
        }
        if constexpr (NG == 2)
            y[o] = silu_f32(r[0]) * r[1];
        else
            y[o] = r[0];
    }
}

// h[i] = silu(h[i]) * u[i]: the gated MLP's elementwise tail after two
// separate projections (mul of equal shapes is one multiply, ops.cpp:239-253).
__global__ __launch_bounds__(kThreads) void k_silu_mul(float* __restrict__ h, const float* __restrict__ u, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        h[i] = silu_f32(h[i]) * u[i];
}

// y[m][n] = sum over splits s = 0..KS-1, in that order, of part[s][m][n] (+ bias[n]).
constexpr int kMaxSplits = 16;
__global__ __launch_bounds__(kThreads) void k_splitk_reduce(const float* __restrict__ part, int KS, int64_t MN, int N,
                                                            const float* __restrict__ bias, float* __restrict__ y) {
    for (int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; o < MN; o += (int64_t)gridDim.x * blockDim.x) {
        float t[kMaxSplits];
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; ++sp) t[sp] = sp < KS ? part[sp * MN + o] : 0.0f;  // all loads first
        float r = 0.0f;
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; ++sp)
            if (sp < KS) r += t[sp];
        if (bias) r = r + bias[o % N];
        y[o] = r;
    }
}

// ---------------------------------------------------------------------------
// Generic INT4 forward over the flat layout (shapes the strip layout cannot
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

bool x_aligned4(const float* x, int64_t K) { return K % 4 == 0 && (((uintptr_t)x) & 15) == 0; }

#define SGQ_GEMV_HOT_ARGS(h, ag) h.x, h.W0, h.S0, h.K, h.RQ, h.NS, h.M, h.nblk, h.pk, h.spcm, ag
template <int BITS, int MT, int NW, int U, int NG, int SPW, bool STREAM>
hipError_t gemv_launch_st(const GemvArgs& a, int nw, hipStream_t s) {
    const dim3 grid((unsigned)(((a.NS + SPW - 1) / SPW) << a.Plog), (unsigned)nw);
    GemvArgs ag = a;
    ag.nblk = (int)grid.x;
    if (a.Kpad != 4 * a.RQ || a.Plog > 255 || a.xlog > 255) return hipErrorInvalidValue;  // GemvHot's packing
    const GemvHot h = gemv_hot(ag, BITS);
    const bool k4 = a.K % 4 == 0;
    if constexpr (BITS == 4 && SPW == 1) {  // the norm-fused form serves the INT4 LLaMA block
        if (a.gamma) {
            if (k4)
                k_gemv<BITS, MT, NW, U, true, NG, SPW, true, STREAM><<<grid, NG * NW * 64, 0, s>>>(SGQ_GEMV_HOT_ARGS(h, ag));
            else
                k_gemv<BITS, MT, NW, U, false, NG, SPW, true, STREAM><<<grid, NG * NW * 64, 0, s>>>(SGQ_GEMV_HOT_ARGS(h, ag));
            return hipGetLastError();
        }
    }
    if (a.gamma) return hipErrorInvalidValue;
    if (k4)
        k_gemv<BITS, MT, NW, U, true, NG, SPW, false, STREAM><<<grid, NG * NW * 64, 0, s>>>(SGQ_GEMV_HOT_ARGS(h, ag));
    else
        k_gemv<BITS, MT, NW, U, false, NG, SPW, false, STREAM><<<grid, NG * NW * 64, 0, s>>>(SGQ_GEMV_HOT_ARGS(h, ag));
    return hipGetLastError();
}
#undef SGQ_GEMV_HOT_ARGS

// Codes take the streaming policy when one row group reads them (Plog 0);
// the row groups of a larger batch each read the strip again, and its second
// read should hit the L2 (measured on 2048->2048 at 16 rows: 5.65 us plain,
// 5.99 streaming; at 8 rows in two groups of four: 4.39 plain, 4.51
// streaming).  One and two rows always run as one group.
template <int BITS, int MT, int NW, int U, int NG, int SPW>
hipError_t gemv_launch_nu(const GemvArgs& a, int nw, hipStream_t s) {
    if (MT < 4 || a.Plog == 0) return gemv_launch_st<BITS, MT, NW, U, NG, SPW, true>(a, nw, s);
    if constexpr (MT >= 4) return gemv_launch_st<BITS, MT, NW, U, NG, SPW, false>(a, nw, s);
    return hipErrorInvalidValue;
}

// Wavefronts per workgroup and weight (each workgroup owns one strip).
// Measured on MI355X for K in 2048..11008 and M in 1..8, 4, 8 and 16
// wavefronts per strip are within a few percent of each other; 4 keeps the
// cross-wave LDS reduction short.
constexpr int kGemvWaves = 4;

// Row quads a lane keeps in flight at most (each holds codes, a scale quad and
// an x quad per row): all of K = 4096 (M = 1, four wavefronts) or 8192 (eight)
// in one batch at M = 1, less as the rows multiply.
constexpr int gemv_umax(int rows) { return rows <= 1 ? 8 : (rows <= 2 ? 4 : (rows <= 4 ? 2 : 1)); }

template <int BITS, int MT, int NG, int SPW, int NW>
hipError_t gemv_launch_spw(const GemvArgs& a, int nw, hipStream_t s) {
    // Row quads in flight per lane: enough for all of K in one batch where the
    // register budget allows (gemv_umax), else batches of UMAX.
    constexpr int UMAX = gemv_umax(MT * SPW);
    const int per_lane = (a.RQ + NW * 64 - 1) / (NW * 64);
#define SGQ_GEMV_NU(U_)                                                                              \
    if constexpr (U_ <= UMAX) {                                                                      \
        if (per_lane > (U_ == 8 ? 6 : (U_ == 6 ? 4 : U_ / 2)) || U_ == 1) return gemv_launch_nu<BITS, MT, NW, U_, NG, SPW>(a, nw, s); \
    }
    SGQ_GEMV_NU(8)
    SGQ_GEMV_NU(6)
    SGQ_GEMV_NU(4)
    SGQ_GEMV_NU(2)
    SGQ_GEMV_NU(1)
#undef SGQ_GEMV_NU
    return hipErrorInvalidValue;
}

template <int BITS, int MT, int NG>
hipError_t gemv_launch(const GemvArgs& a, int nw, hipStream_t s) {
    if constexpr (BITS == 4 && NG == 1 && MT <= 2) {
        // Two strips per workgroup (they must share a scale column) load each
        // x and scale quad once for both: a third fewer load instructions per
        // code byte, which is what the one- and two-row GEMV waits on.  Only
        // where that still leaves a workgroup per CU, and with enough
        // wavefronts to keep all of K in one batch of loads.  Measured on
        // MI355X at M=1: 4096->4096 4.30 -> 4.21 us, 4096->11008 7.67 -> 6.93,
        // 11008->4096 7.39 -> 7.22 (16 wavefronts); M=2 4096->11008 9.11 -> 8.52.
        if (nw == 1 && a.mode % 2 == 0 && a.NS >= 2 * a.cus) {
            constexpr int um = gemv_umax(2 * MT);
            if (a.RQ <= um * kGemvWaves * 64) return gemv_launch_spw<BITS, MT, NG, 2, kGemvWaves>(a, nw, s);
            if (a.RQ <= um * 2 * kGemvWaves * 64) return gemv_launch_spw<BITS, MT, NG, 2, 2 * kGemvWaves>(a, nw, s);
            if (a.RQ <= um * 4 * kGemvWaves * 64) return gemv_launch_spw<BITS, MT, NG, 2, 4 * kGemvWaves>(a, nw, s);
        }
    }
    // Few strips for the GPU (under two workgroups per CU) and a K long enough
    // for eight wavefronts: split K over eight wavefronts instead of four, so
    // each SIMD holds more than one wavefront to hide load latency.  Measured
    // on MI355X: 5632 -> 2048 at M=8 9.1 -> 7.7 us, M=1 4.8 -> 4.6 us;
    // 2048 -> 2048 at M=4 3.9 -> 3.7 us.
    if (((int64_t)nw * a.NS << a.Plog) < 2 * a.cus && a.RQ >= 8 * 64)
        return gemv_launch_spw<BITS, MT, NG, 1, 2 * kGemvWaves>(a, nw, s);
    // A K too long for one batch of four wavefronts but within one batch of
    // eight: eight wavefronts, so that every load is in flight at once instead
    // of batches that each wait a full memory latency (measured on MI355X,
    // 11008 -> 4096 at M=1: 8.2 -> 7.8 us).
    if constexpr (MT == 1) {
        constexpr int um = gemv_umax(1);
        if (a.RQ > um * kGemvWaves * 64 && a.RQ <= um * 2 * kGemvWaves * 64)
            return gemv_launch_spw<BITS, MT, NG, 1, 2 * kGemvWaves>(a, nw, s);
    }
    return gemv_launch_spw<BITS, MT, NG, 1, kGemvWaves>(a, nw, s);
}

template <int BITS, int NG>
hipError_t gemv_dispatch(GemvArgs a, int64_t M, int nw, hipStream_t s) {
    a.M = (int)M;
    a.cus = device_cus(s);
    a.xlog = xcd_log2(device_xcds(s));
    constexpr int kRowsMax = 8;  // rows per workgroup beyond four
    // All rows in one launch: M <= 4 as one row group, larger M in row groups
    // of kRowsMax (each a workgroup of its own over the same strip), their
    // count rounded up to a power of two for the index arithmetic.
    a.Plog = 0;
    if (M <= 1) return gemv_launch<BITS, 1, NG>(a, nw, s);
    if (M <= 2) return gemv_launch<BITS, 2, NG>(a, nw, s);
    if (M <= 4) {
        // Three or four rows over a weight of fewer strips than compute units:
        // two row groups of two, twice the workgroups.  Measured on MI355X
        // (us): INT4 8192->1024 at 4 rows 5.81-5.98 -> 4.58-4.66, 4096->512 at
        // 3 rows 4.20-4.28 -> 3.35-3.38, 2048->512 at 4 rows 3.31-3.32 ->
        // 2.91-2.97; INT8 4096->512 at 4 rows 3.45-3.56 -> 3.05-3.19.  Two rows
        // as two groups of one measured equal (INT4 8192->1024, INT8
        // 4096->512), and 4096->11008 (1376 strips) keeps one group.
        if (M >= 3 && (int64_t)nw * a.NS < a.cus) {
            a.Plog = 1;
            return gemv_launch<BITS, 2, NG>(a, nw, s);
        }
        return gemv_launch<BITS, 4, NG>(a, nw, s);
    }
    // Five to eight rows over a K of at most 2048 (a row quad or two per
    // lane): two row groups of four, whose lanes reduce half as many
    // accumulators (INT4 32 instead of 64, with the offset-binary decode;
    // INT8 16 instead of 32); at that K the lane and wavefront reduction
    // outweighs the lanes' share of the k loop.  Measured on MI355X (us): INT4
    // g128 2048->2048 at 8 rows 4.74-4.80 -> 4.39; INT8 2048->2048 at 8 rows
    // 4.81-4.83 -> 4.11-4.16, 1024->1024 at 8 rows 2.99-3.01 -> 2.69-2.70,
    // 2048->1024 at 6 rows 3.59-3.62 -> 3.14-3.16; INT4 5632->2048 and
    // 4096->4096 at 8 rows, and 2048->2048 at 16, were slower in groups of four.
    if (M <= 8 && a.K <= 2048) {
        a.Plog = 1;
        return gemv_launch<BITS, 4, NG>(a, nw, s);
    }
    // 5..16 rows whose row groups of eight would leave fewer workgroups than
    // compute units (narrow weights): groups of four, twice the workgroups.
    // Measured on MI355X (us): INT4 8192->1024 at 8 rows 8.34-8.44 -> 5.74-5.79,
    // 2048->512 at 16 rows 4.10-4.12 -> 3.23-3.34; INT8 4096->512 at 8 rows
    // 4.48-4.60 -> 3.29-3.31.  Where groups of eight already fill the device,
    // groups of four were equal or slower (INT4 5632->2048 and 4096->4096 at 8
    // rows, 2048->2048 at 12 and 16).
    if (M <= 16 && (((int64_t)nw * a.NS) << (M > 8 ? 1 : 0)) < a.cus) {
        a.Plog = M > 8 ? 2 : 1;
        return gemv_launch<BITS, 4, NG>(a, nw, s);
    }
    const int64_t groups = (M + kRowsMax - 1) / kRowsMax;
    while ((int64_t)1 << a.Plog < groups) ++a.Plog;
    if (((int64_t)kRowsMax << a.Plog) > kGemvRowsMax) return hipErrorInvalidValue;
    return gemv_launch<BITS, kRowsMax, NG>(a, nw, s);
}

GemvArgs gemv_args(const float* x, int64_t K, int64_t N, int mode, int64_t Kpad, int64_t RQ, int64_t NS, float* y,
                   int64_t ldy, const float* res) {
    GemvArgs a{};
    a.Plog = 0;
    a.x = x;
    a.K = (int)K;
    a.N = (int)N;
    a.mode = mode;
    a.spc = FastDiv((uint32_t)(mode > 0 ? mode : 1));
    a.Kpad = (int)Kpad;
    a.RQ = (int)RQ;
    a.NS = (int)NS;
    a.y = y;
    a.ldy = (int)ldy;
    a.res = res;
    return a;
}

// Wavefronts per workgroup of k_skinny_sb (each takes every 8th super-block
// of its range) and of k_skinny3 (every 16th 32-row k block); the summation
// order depends on them, so each is the same for every plan of its form.
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyWholeKWaves = 16;

// One k_skinny3 launch (and, with split K, its reduce) for the plan's C and
// MB; NG weights of equal shape with their devscales and biases.
template <int C, int NG, int MB, bool XA>
hipError_t skinny_launch(const float* x, int64_t M, int64_t K, int64_t N, const void* const* packed,
                         const float* const* devscales, const float* const* bias, const I4Geom& g, int form, int S,
                         float* y, float* part, const SkinnyExtra& ex, hipStream_t s) {
    if (form == 0 && S != 1) return hipErrorInvalidValue;
    // Side-by-side weights, a row stride and the folded RMSNorm: whole-K form only.
    const bool plain = ex.nw == 1 && ex.ldy == N && !ex.gamma;
    if ((!plain && form != 0) || ex.nw < 1 || ex.nw > 3 || (NG == 2 && ex.nw != 1)) return hipErrorInvalidValue;
    // Side-by-side weights come with the norm (the LLaMA block's q, k and v):
    // the plain kernels take their one weight from the preloaded arguments.
    if (ex.nw != 1 && !ex.gamma) return hipErrorInvalidValue;
    if (g.Kpad != 4 * g.RQ) return hipErrorInvalidValue;  // SkinnyHot carries RQ only
    SkinnyArgs a{};
    a.x = x;
    a.M = (int)M;
    a.K = (int)K;
    a.N = (int)N;
    const int nq = NG == 1 ? ex.nw : NG;
    for (int q = 0; q < nq; ++q) {
        a.W[q] = (const uint4*)packed[q];
        a.SC[q] = devscales[q];
        a.bias[q] = bias[q];
    }
    a.ldy = (int)ex.ldy;
    a.wgpw = (int)(g.NS / (2 * C));
    a.wgd = FastDiv((uint32_t)a.wgpw);
    a.gamma = ex.gamma;
    a.eps = ex.eps;
    a.spc = (int)g.spc;
    a.Kpad = (int)g.Kpad;
    a.RQ = (int)g.RQ;
    a.wpc = FastDiv((uint32_t)(g.spc / (2 * C)));
    a.y = y;
    a.part = part;
    int slog = 0;
    while ((1 << slog) < S) ++slog;
    a.slog = slog;
    a.sbs = (int)ceil_div(ceil_div(g.Kpad, kSkinnySB), S);
    a.nblk = (int)(g.NS / (2 * C)) << slog;  // skinny_plan: 2C divides spc, which divides NS
    a.xlog = xcd_log2(device_xcds(s));
    a.ko = (int)(g.koct_off() / 256);
    if (form == 0) {
        if constexpr (MB == 1) {
            constexpr int U = NG == 1 ? 4 : 2;  // register budget of 16 wavefronts per CU
            a.nblk *= ex.nw;
            const SkinnyHot h = skinny_hot(a);
#define SGQ_SKINNY3(NORM_)                                                                                 \
    if (M <= 8)                                                                                            \
        k_skinny3<kSkinnyWholeKWaves, U, C, NG, XA, NORM_, true><<<a.nblk, kSkinnyWholeKWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a); \
    else                                                                                                   \
        k_skinny3<kSkinnyWholeKWaves, U, C, NG, XA, NORM_, false><<<a.nblk, kSkinnyWholeKWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a);
            if (ex.gamma) {
                // The norm-fused form keeps two column blocks (register budget).
                if constexpr (C == 2) {
                    SGQ_SKINNY3(true)
                } else {
                    return hipErrorInvalidValue;
                }
            } else {
                SGQ_SKINNY3(false)
            }
#undef SGQ_SKINNY3
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    const bool half = MB == 1 && M <= 8;
    const SkinnyHot h = skinny_hot(a);
    if (S > 1 && half)
        k_skinny_sb<kSkinnyWaves, C, NG, XA, MB, true, MB == 1><<<a.nblk, kSkinnyWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a);
    else if (S > 1)
        k_skinny_sb<kSkinnyWaves, C, NG, XA, MB, true, false><<<a.nblk, kSkinnyWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a);
    else if (half)
        k_skinny_sb<kSkinnyWaves, C, NG, XA, MB, false, MB == 1><<<a.nblk, kSkinnyWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a);
    else
        k_skinny_sb<kSkinnyWaves, C, NG, XA, MB, false, false><<<a.nblk, kSkinnyWaves * 64, 0, s>>>(SGQ_SKINNY_HOT_ARGS(h), a);
    if (S > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t MN = M * N;
        int64_t blocks = ceil_div(MN, kThreads);
        if (blocks > 4096) blocks = 4096;
        k_skinny_reduce<NG><<<(unsigned)blocks, kThreads, 0, s>>>(part, S, MN, (int)N, bias[0],
                                                                  NG == 2 ? bias[1] : nullptr, y);
    }
    return hipGetLastError();
}
#undef SGQ_SKINNY_HOT_ARGS
#undef SGQ_SKINNY_HOT_PARAMS

template <int NG>
hipError_t skinny_dispatch(const SkinnyPlan& p, const float* x, int64_t M, int64_t K, int64_t N,
                           const void* const* packed, const float* const* devscales, const float* const* bias,
                           const I4Geom& g, float* y, float* part, const SkinnyExtra& ex, hipStream_t s) {
    // The super-block form of the gated MLP, and two row blocks of
    // unaligned x, keep two column blocks per workgroup, within the register
    // budget (C does not change the order of any sum).
    if (p.C != 2 && p.C != 4) return hipErrorInvalidValue;
#define SGQ_SKINNY(C_, MB_, XA_) \
    return skinny_launch<C_, NG, MB_, XA_>(x, M, K, N, packed, devscales, bias, g, p.form, p.S, y, part, ex, s)
    const bool xa = x_aligned4(x, K);
    // The norm-fused form runs two column blocks per workgroup (C does not
    // change the order of any sum).
    if (p.C == 4 && p.MB == 1 && (NG == 1 || p.form == 0) && !ex.gamma) {
        if (xa) SGQ_SKINNY(4, 1, true);
        SGQ_SKINNY(4, 1, false);
    }
    if constexpr (NG == 1) {
        if (p.C == 4 && xa && !ex.gamma) SGQ_SKINNY(4, 2, true);
    }
    if (p.MB == 1) {
        if (xa) SGQ_SKINNY(2, 1, true);
        SGQ_SKINNY(2, 1, false);
    }
    if (xa) SGQ_SKINNY(2, 2, true);
    SGQ_SKINNY(2, 2, false);
#undef SGQ_SKINNY
}

template <int C, int MB, bool PT, bool XA>
hipError_t skinny8_launch(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          const float* bias, float* y, hipStream_t s) {
    const I8Geom g(K, N);
    Skinny8Args a{};
    a.x = x;
    a.M = (int)M;
    a.K = (int)K;
    a.N = (int)N;
    a.W = (const uint4*)packed;
    a.S = scales;
    a.bias = bias;
    a.RQ = (int)g.RQ;
    a.NS = (int)g.NS;
    a.Kpad = (int)g.Kpad;
    a.ncg = (int)ceil_div(g.NS, 4 * C);
    a.cgd = FastDiv((uint32_t)a.ncg);
    a.y = y;
    a.nblk = (int)(ceil_div(M, 16 * MB) * a.ncg);
    a.xlog = xcd_log2(device_xcds(s));
    constexpr int U = MB == 1 ? 4 : 2;  // register budget of 16 wavefronts per CU
    if (g.Kpad != 4 * g.RQ) return hipErrorInvalidValue;  // Skinny8Hot carries RQ only
    const Skinny8Hot h = skinny8_hot(a);
    if (MB == 1 && M <= 8)
        k_skinny8<kSkinnyWholeKWaves, U, C, MB, PT, XA, MB == 1><<<a.nblk, kSkinnyWholeKWaves * 64, 0, s>>>(h.x, h.W, h.S, h.M, h.K, h.RQ, h.NS, h.nblk, h.pk, h.cgdm, h.ncg, a);
    else
        k_skinny8<kSkinnyWholeKWaves, U, C, MB, PT, XA, false><<<a.nblk, kSkinnyWholeKWaves * 64, 0, s>>>(h.x, h.W, h.S, h.M, h.K, h.RQ, h.NS, h.nblk, h.pk, h.cgdm, h.ncg, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_skinny_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                            bool per_tensor, const float* bias, const Skinny8Plan& p, float* y, hipStream_t s) {
    const bool xa = x_aligned4(x, K);
#define SGQ_SKINNY8(C_, MB_)                                                                      \
    if (p.C == C_ && p.MB == MB_) {                                                                \
        if (per_tensor)                                                                           \
            return xa ? skinny8_launch<C_, MB_, true, true>(x, M, K, N, packed, scales, bias, y, s)  \
                      : skinny8_launch<C_, MB_, true, false>(x, M, K, N, packed, scales, bias, y, s); \
        return xa ? skinny8_launch<C_, MB_, false, true>(x, M, K, N, packed, scales, bias, y, s)     \
                  : skinny8_launch<C_, MB_, false, false>(x, M, K, N, packed, scales, bias, y, s);   \
    }
    SGQ_SKINNY8(1, 1)
    SGQ_SKINNY8(2, 1)
    SGQ_SKINNY8(1, 2)
    SGQ_SKINNY8(2, 2)
#undef SGQ_SKINNY8
    return hipErrorInvalidValue;
}

hipError_t launch_skinny_i4(const float* x, int64_t M, int64_t K, int64_t N, int ng, const void* const* packed,
                            const float* const* devscales, const float* const* bias, const I4Geom& g,
                            const SkinnyPlan& p, float* y, void* ws, hipStream_t s, const SkinnyExtra* extra) {
    if (p.C == 0 || (p.S > 1 && !ws)) return hipErrorInvalidValue;
    SkinnyExtra ex;
    if (extra) ex = *extra;
    if (ex.ldy == 0) ex.ldy = N;
    if (ng == 1) return skinny_dispatch<1>(p, x, M, K, N, packed, devscales, bias, g, y, (float*)ws, ex, s);
    if (ng == 2) return skinny_dispatch<2>(p, x, M, K, N, packed, devscales, bias, g, y, (float*)ws, ex, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, hipStream_t s) {
    return launch_gemv_i4_multi(x, M, K, N, 1, &packed, &devscales, &bias, g, y, N, nullptr, nullptr, 0.0f, s);
}

hipError_t launch_gemv_i4_multi(const float* x, int64_t M, int64_t K, int64_t N, int nw, const void* const* packed,
                                const float* const* devscales, const float* const* bias, const I4Geom& g, float* y,
                                int64_t ldy, const float* res, const float* gamma, float eps, hipStream_t s) {
    if (nw < 1 || nw > 3) return hipErrorInvalidValue;
    GemvArgs a = gemv_args(x, K, N, (int)g.spc, g.Kpad, g.RQ, g.NS, y, ldy, res);
    a.gamma = gamma;
    a.eps = eps;
    for (int w = 0; w < nw; ++w) {
        a.W[w] = (const uint4*)packed[w];
        a.SC[w] = devscales[w];
        a.bias[w] = bias[w];
    }
    return gemv_dispatch<4, 1>(a, M, nw, s);
}

hipError_t launch_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, hipStream_t s) {
    I8Geom g(K, N);
    GemvArgs a = gemv_args(x, K, N, per_tensor ? 1 : 0, g.Kpad, g.RQ, g.NS, y, N, nullptr);
    a.W[0] = (const uint4*)packed;
    a.SC[0] = scales;
    a.bias[0] = bias;
    return gemv_dispatch<8, 1>(a, M, 1, s);
}

hipError_t launch_swiglu_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_g,
                                 const float* devscales_g, const float* bias_g, const void* packed_u,
                                 const float* devscales_u, const float* bias_u, const I4Geom& g, float* h,
                                 hipStream_t s, const float* gamma, float eps) {
    GemvArgs a = gemv_args(x, K, N, (int)g.spc, g.Kpad, g.RQ, g.NS, h, N, nullptr);
    a.gamma = gamma;
    a.eps = eps;
    a.W[0] = (const uint4*)packed_g;
    a.W[1] = (const uint4*)packed_u;
    a.SC[0] = devscales_g;
    a.SC[1] = devscales_u;
    a.bias[0] = bias_g;
    a.bias[1] = bias_u;
    return gemv_dispatch<4, 2>(a, M, 1, s);
}

hipError_t launch_swiglu_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_g,
                                 const float* scales_g, const float* bias_g, const void* packed_u,
                                 const float* scales_u, const float* bias_u, bool per_tensor, float* h,
                                 hipStream_t s) {
    I8Geom g(K, N);
    GemvArgs a = gemv_args(x, K, N, per_tensor ? 1 : 0, g.Kpad, g.RQ, g.NS, h, N, nullptr);
    a.W[0] = (const uint4*)packed_g;
    a.W[1] = (const uint4*)packed_u;
    a.SC[0] = scales_g;
    a.SC[1] = scales_u;
    a.bias[0] = bias_g;
    a.bias[1] = bias_u;
    return gemv_dispatch<8, 2>(a, M, 1, s);
}

hipError_t launch_silu_mul(float* h, const float* u, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = ceil_div(n, kThreads);
    if (blocks > 4096) blocks = 4096;
    k_silu_mul<<<(unsigned)blocks, kThreads, 0, s>>>(h, u, n);
    return hipGetLastError();
}

// CU count per device, read from the runtime once per device (0: not read
// yet).  A forward call asks for it once or twice; the attribute query cost
// about 0.26 us of host time per eager C2 call (6.62 -> 6.36 us).
constexpr int kCuCacheDevices = 64;
std::atomic<int> g_device_cus[kCuCacheDevices];

int device_cus(hipStream_t s) {
    int dev = 0;
    if (hipStreamGetDevice(s, &dev) != hipSuccess) {
        (void)hipGetLastError();  // leave no error behind for the launch check
        if (hipGetDevice(&dev) != hipSuccess) {
            (void)hipGetLastError();
            return (int)kMaxCus;
        }
    }
    const bool cache = dev >= 0 && dev < kCuCacheDevices;
    if (cache) {
        const int c = g_device_cus[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) {
        (void)hipGetLastError();
        return (int)kMaxCus;
    }
    cus = cus < kMaxCus ? cus : (int)kMaxCus;
    if (cache) g_device_cus[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// XCD count per device, read once like the CU count (0: not read yet).  A
// full MI355X has 8; its compute partitions report 4, 2 or 1.
std::atomic<int> g_device_xcds[kCuCacheDevices];

int device_xcds(hipStream_t s) {
    int dev = 0;
    if (hipStreamGetDevice(s, &dev) != hipSuccess) {
        (void)hipGetLastError();
        if (hipGetDevice(&dev) != hipSuccess) {
            (void)hipGetLastError();
            return 1;
        }
    }
    const bool cache = dev >= 0 && dev < kCuCacheDevices;
    if (cache) {
        const int c = g_device_xcds[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x < 1) {
        (void)hipGetLastError();
        x = 1;  // unknown: the identity workgroup order, correct on any device
    }
    x = x < kMaxXcds ? x : kMaxXcds;
    if (cache) g_device_xcds[dev].store(x, std::memory_order_relaxed);
    return x;
}

int xcd_log2(int xcds) {
    int l = 0;
    while ((2 << l) <= xcds) ++l;
    return (1 << l) == xcds ? l : 0;  // not a power of two: the identity order
}

GemmPlan gemm_plan(int64_t M, int64_t K, int64_t N, const GemmTile& t, int64_t cus) {
    const int64_t tiles = ceil_div(M, t.bm) * ceil_div(N, t.bn);
    const int64_t KT = ceil_div(round_up(K, kPadK), kBK);
    GemmPlan p{1, (int)KT};
    if (cus < 1) cus = 1;
    if (cus > kMaxCus) cus = kMaxCus;
    // Splits fill the resident slots, rounded down: a grid just past them
    // runs its last few workgroups as a second pass (4096->11008 at 128 rows,
    // 86 tiles of 128 x 128: 6 splits, 516 workgroups on 512 slots, 94 us; 5
    // splits 61 us).
    const int64_t slots = t.per_cu * cus;
    if (tiles < slots && KT >= 4) {
        int64_t ks = slots / tiles;
        if (ks > KT / 2) ks = KT / 2;  // at least two stages per split
        if (ks > kMaxSplits) ks = kMaxSplits;
        if (ks > 1) {
            p.sps = (int)ceil_div(KT, ks);
            p.KS = (int)ceil_div(KT, p.sps);  // no split without stages
        }
    }
    return p;
}

// Tile of the three-term GEMM for a code width and batch (the fp32 kernel
// uses the 128 x 128 tile), with the workgroups a split-K grid gives each CU:
// two of the 128 x 128 tiles, one of the 128 x 256 (its LDS and registers fill
// the CU), four of the 32-row tile (28 KB of LDS) and two of the 64-row tile.
// Three of the latter fit (40 KB of LDS) but cost more in partial tiles
// (KS * M * N * 4 bytes, written and read back) than they gain: 2048->6144 at
// 64 rows 16 splits 31.6 us, 10 splits 24.3 us; 4096->11008 at 48 rows 9
// splits 50.4 us, 5 splits 42.1 us.
GemmTile gemm_tile(int bits, int64_t M) {
    if (M <= 32) return GemmTile{32, kBN, 4};
    if (M <= 64) return GemmTile{64, kBN, 2};
    return bits == 8 ? GemmTile{kBM, 2 * kBN, 1} : GemmTile{kBM, kBN, 2};
}

int64_t gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    // Either code width (and the fp32 kernel's 128 x 128 tile) on the largest
    // device: room for the largest plan on any device.
    int64_t ks = gemm_plan(M, K, N, GemmTile{kBM, kBN, 2}, kMaxCus).KS;
    for (int bits : {4, 8}) {
        const int64_t k = gemm_plan(M, K, N, gemm_tile(bits, M), kMaxCus).KS;
        if (k > ks) ks = k;
    }
    return ks > 1 ? ks * M * N * 4 : 0;
}

// Which GEMM kernel a shape takes and its tile: the three-term bf16 kernel
// folds the scale into A, so a tile's columns must share their scale (always
// for INT8's 256-column tiles; for INT4 when a scale column spans a multiple
// of 16 strips, i.e. a group that is a multiple of 128).
static bool gemm_three_term(int bits, int mode) { return bits == 8 || mode % 16 == 0; }

int64_t gemm_launch_ws_bytes(int bits, int64_t M, int64_t K, int64_t N, int mode, int64_t cus) {
    const bool three = gemm_three_term(bits, mode);
    const GemmPlan p = gemm_plan(M, K, N, three ? gemm_tile(bits, M) : GemmTile{kBM, kBN, 2}, cus);
    return p.KS > 1 ? (int64_t)p.KS * M * N * 4 : 0;
}

void linear_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int64_t cus, int* path, int* ks) {
    *ks = 1;
    if (bits == 4 && !I4Geom(K, N, group_size).tiled) {
        *path = 3;
        return;
    }
    if (bits == 4) {
        const SkinnyPlan sp = skinny_plan(M, K, I4Geom(K, N, group_size), cus < kMaxCus ? cus : kMaxCus);
        if (sp.C > 0) {
            *path = 4;
            *ks = sp.S;
            return;
        }
    } else if (skinny8_plan(M, K, N, cus < kMaxCus ? cus : kMaxCus).C > 0) {
        *path = 4;
        return;
    }
    if (linear_uses_gemv(M, K, N)) {
        *path = 0;
        return;
    }
    const int mode = bits == 4 ? (int)I4Geom(K, N, group_size).spc : 0;
    const bool three = gemm_three_term(bits, mode);
    *path = three ? 1 : 2;
    *ks = gemm_plan(M, K, N, three ? gemm_tile(bits, M) : GemmTile{kBM, kBN, 2}, cus).KS;
}

// Tile rows per XCD rectangle for a grid of tm x tn tiles without a K split
// on a device of `xcds` XCDs: the divisor a of both tm and per = tm * tn /
// xcds (per / a dividing tn) that minimises what one XCD's L2 fetches, a row
// blocks of x (xb bytes each) and per / a column blocks of codes (wb bytes
// each); 0 when the grid does not tile into xcds such rectangles (the plain
// XCD order then).
int xcd_rect_rows_impl(int64_t tm, int64_t tn, int64_t xb, int64_t wb, int64_t xcds) {
    const int64_t T = tm * tn;
    if (xcds < 1 || T % xcds != 0) return 0;
    const int64_t per = T / xcds;
    int best = 0;
    int64_t cost = 0;
    for (int64_t a = 1; a <= per && a <= tm; ++a) {
        if (per % a || tm % a || tn % (per / a) || (tm / a) * (tn / (per / a)) != xcds) continue;
        const int64_t c = a * xb + (per / a) * wb;
        if (best == 0 || c < cost) best = (int)a, cost = c;
    }
    return best;
}

int gemm_rect_rows(int bits, int64_t M, int64_t K, int64_t N, int mode, int64_t cus, int64_t xcds) {
    const bool three = gemm_three_term(bits, mode);
    const GemmTile t = three ? gemm_tile(bits, M) : GemmTile{kBM, kBN, 2};
    if (!three || gemm_plan(M, K, N, t, cus).KS != 1) return 0;
    return xcd_rect_rows_impl(ceil_div(M, t.bm), ceil_div(N, t.bn), t.bm * K * 4, t.bn * K * bits / 8, xcds);
}

namespace {

template <int BITS>
hipError_t gemm_launch(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* sc, int mode,
                       int64_t Kpad, int64_t RQ, int64_t NS, const float* bias, float* y, void* ws, hipStream_t s) {
    // INT4 groups that are not a multiple of 128 take the fp32-MFMA kernel.
    const bool three = gemm_three_term(BITS, mode);
    const GemmTile t = three ? gemm_tile(BITS, M) : GemmTile{kBM, kBN, 2};
    const GemmPlan p = gemm_plan(M, K, N, t, device_cus(s));
    float* part = p.KS > 1 ? (float*)ws : nullptr;
    const dim3 grid((unsigned)(ceil_div(M, t.bm) * ceil_div(N, t.bn) * p.KS));
    const int xcds = device_xcds(s);
    const int xr = p.KS == 1 ? xcd_rect_rows_impl(ceil_div(M, t.bm), ceil_div(N, t.bn), t.bm * K * 4,
                                                  t.bn * K * BITS / 8, xcds)
                             : 0;
    const int xlog = xcd_log2(xcds);
    const bool k4 = x_aligned4(x, K);
    const bool pt = BITS == 8 && mode;
    // INT4: the k-octet copy follows the strips at their bytes rounded up to
    // 256 (I4Geom::koct_off).
    const int ko = BITS == 4 ? (int)ceil_div(NS * RQ * 16, 256) : 0;
    using Big = typename std::conditional<BITS == 8, G3Wide, G3Tile>::type;
#define SGQ_GEMM3(SH, A4, PT_)                                                                                 \
    k_gemm3<BITS, A4, (PT_) && BITS == 8, SH><<<grid, SH::NT, 0, s>>>(Gemm3Args{                                \
        x, (int)M, (int)K, (int)N, (const uint4*)packed, sc, mode, (int)Kpad, (int)RQ, (int)NS, p.KS, p.sps, bias, \
        y, part, xr, xlog, ko})
#define SGQ_GEMM3_SHAPE(SH)               \
    if (k4 && pt)                         \
        SGQ_GEMM3(SH, true, true);        \
    else if (k4)                          \
        SGQ_GEMM3(SH, true, false);       \
    else if (pt)                          \
        SGQ_GEMM3(SH, false, true);       \
    else                                  \
        SGQ_GEMM3(SH, false, false);
    if (three && t.bm == 32) {
        SGQ_GEMM3_SHAPE(G3Rows32)
    } else if (three && t.bm == 64) {
        SGQ_GEMM3_SHAPE(G3Rows64)
    } else if (three) {
        SGQ_GEMM3_SHAPE(Big)
    } else if (k4)
        k_gemm<BITS, true><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, sc, mode,
                                                     (int)Kpad, (int)RQ, (int)NS, p.KS, p.sps, bias, y, part);
    else
        k_gemm<BITS, false><<<grid, kThreads, 0, s>>>(x, (int)M, (int)K, (int)N, (const uint4*)packed, sc, mode,
                                                      (int)Kpad, (int)RQ, (int)NS, p.KS, p.sps, bias, y, part);
#undef SGQ_GEMM3_SHAPE
#undef SGQ_GEMM3
    if (p.KS > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t MN = M * N;
        int64_t blocks = ceil_div(MN, kThreads);
        if (blocks > 4096) blocks = 4096;
        k_splitk_reduce<<<(unsigned)blocks, kThreads, 0, s>>>(part, p.KS, MN, (int)N, bias, y);
    }
    return hipGetLastError();
}
}  // namespace

hipError_t launch_gemm_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, void* ws, hipStream_t s) {
    I8Geom g(K, N);
    return gemm_launch<8>(x, M, K, N, packed, scales, per_tensor ? 1 : 0, g.Kpad, g.RQ, g.NS, bias, y, ws, s);
}

hipError_t launch_gemm_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, void* ws,
                          hipStream_t s) {
    return gemm_launch<4>(x, M, K, N, packed, devscales, (int)g.spc, g.Kpad, g.RQ, g.NS, bias, y, ws, s);
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
