// sgq_internal.h -- device layouts and kernel launchers shared by the HIP
// translation units of libsgq.so.  Not part of the public C ABI (include/sgq.h).
//
// Device layouts
// --------------
// The reference keeps one fp32 per code (src/quantization.cpp:32-37,127-153);
// this library streams packed codes instead.  Both tiled layouts cut the
// [K,N] weight into super-tiles of 16 rows (k) by TN columns (n), 1024 bytes
// each, stored column-block-major: super-tile (cb, kt) starts at byte
// (cb * KT + kt) * 1024, where KT = Kpad / 16.  A super-tile holds 64 chunks
// of 16 bytes; chunk c covers rows 4*(c>>4) .. +3 ("band") and one strip of
// columns (c & 15).  A wavefront loading super-tile t with lane = chunk reads
// 1 KiB of contiguous memory in one 128-bit load per lane.
//
//   INT8 (TN = 64):  strip = 4 columns.  Dword d of a chunk is column
//                    4*strip + d; byte r of that dword is row 4*band + r.
//                    Codes are two's-complement int8.
//   INT4 (TN = 128): strip = 8 columns.  Dword r of a chunk is row
//                    4*band + r; nibble e (bits 4e..4e+3) is column
//                    8*strip + e.  Codes are two's-complement int4.
//
// Rows past K and columns past N are padding with code 0.  INT4 tiled keeps
// its scales transposed, devscales[sc][Kpad], one column per `spc` strips:
// spc = group/8 when N % group == 0 (groups never straddle rows, so a whole
// group of columns shares one scale per row), else spc = 1 (one scale per
// 8-column strip and row; valid because group % 8 == 0 and N % 8 == 0 keep
// every strip inside one group).  INT4 flat (any shape) is the flattened
// tensor with two codes per byte, element i in byte i/2, low nibble first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgq {

constexpr int64_t kTileK = 16;
constexpr int64_t kI8TileN = 64;
constexpr int64_t kI4TileN = 128;
constexpr int64_t kTileBytes = 1024;

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

struct I8Geom {
    int64_t K, N, Kpad, Npad, KT, NCB;
    explicit I8Geom(int64_t k, int64_t n)
        : K(k), N(n), Kpad(round_up(k, kTileK)), Npad(round_up(n, kI8TileN)), KT(Kpad / kTileK),
          NCB(Npad / kI8TileN) {}
    int64_t bytes() const { return NCB * KT * kTileBytes; }
};

struct I4Geom {
    int64_t K, N, G, Kpad, Npad, KT, NCB, spc, nsc;
    bool tiled;
    I4Geom(int64_t k, int64_t n, int64_t g)
        : K(k), N(n), G(g <= 0 ? 32 : g), Kpad(round_up(k, kTileK)), Npad(round_up(n, kI4TileN)),
          KT(Kpad / kTileK), NCB(Npad / kI4TileN) {
        tiled = (N % 8 == 0) && (G % 8 == 0);
        spc = (tiled && N % G == 0) ? G / 8 : 1;
        nsc = tiled ? ceil_div(NCB * 16, spc) : 0;
    }
    int64_t bytes() const { return tiled ? NCB * KT * kTileBytes : ceil_div(K * N, 2); }
    int64_t devscale_count() const { return tiled ? nsc * Kpad : 0; }
};

// GEMV split-K plan: ksplit k-ranges of `tps` super-tiles each per column block.
struct GemvPlan {
    int ksplit;
    int tps;
};
GemvPlan gemv_plan(int64_t KT, int64_t NCB);
constexpr int kGemvMaxM = 16;

// ---- launchers (return hipError_t of the launch) ----------------------
hipError_t launch_fill_zero(void* p, int64_t bytes, hipStream_t s);
hipError_t launch_fill_bias(float* y, int64_t M, int64_t N, const float* bias, hipStream_t s);

// Scale computation.  absmax over groups of G consecutive elements; writes
// scales[g] = max/qmax and inv[g] = qmax/max (src/quantization.cpp:29-30,63-64,146-147).
hipError_t launch_group_scales(const float* x, int64_t total, int64_t G, int64_t ngroups, float qmax, float* scales,
                               float* inv, hipStream_t s);
// Per-tensor: partial maxima over blocks, then one group over the partials.
int64_t absmax_partial_count(int64_t total);
hipError_t launch_absmax_partial(const float* x, int64_t total, float* partial, int64_t nparts, hipStream_t s);

// Pack kernels.  from_codes == false: src is x and codes are computed with inv;
// from_codes == true: src holds fp32 codes, validated into *bad.  packed and
// qdata may each be null (that output is skipped).
hipError_t launch_pack_i8_tiled(const float* src, bool from_codes, int64_t K, int64_t N, const float* inv,
                                bool per_tensor, void* packed, float* qdata, int* bad, hipStream_t s);
hipError_t launch_pack_i4_tiled(const float* src, bool from_codes, int64_t K, int64_t N, int64_t G,
                                const float* inv, void* packed, float* qdata, int* bad, hipStream_t s);
hipError_t launch_pack_i4_flat(const float* src, bool from_codes, int64_t total, int64_t G, const float* inv,
                               void* packed, float* qdata, int* bad, hipStream_t s);
hipError_t launch_devscales_i4(const float* scales, const I4Geom& g, float* devscales, hipStream_t s);

// Unpack / dequantize to reference layout [K,N].  scales == nullptr: codes only.
hipError_t launch_unpack_i8_tiled(const void* packed, int64_t K, int64_t N, const float* scales, bool per_tensor,
                                  float* out, hipStream_t s);
hipError_t launch_unpack_i4_tiled(const void* packed, int64_t K, int64_t N, int64_t G, const float* scales,
                                  float* out, hipStream_t s);
hipError_t launch_unpack_i4_flat(const void* packed, int64_t total, int64_t G, const float* scales, float* out,
                                 hipStream_t s);

// Forward kernels.
hipError_t launch_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, float* partial, unsigned* counters,
                          hipStream_t s);
hipError_t launch_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, float* partial,
                          unsigned* counters, hipStream_t s);
hipError_t launch_gemm_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, hipStream_t s);
hipError_t launch_gemm_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, hipStream_t s);
hipError_t launch_linear_i4_flat(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                                 const float* scales, int64_t G, const float* bias, float* y, hipStream_t s);

}  // namespace sgq
