// sgq_internal.h -- device layouts and kernel launchers shared by the HIP
// translation units of libsgq.so.  Not part of the public C ABI (include/sgq.h).
//
// Device layouts
// --------------
// The reference keeps one fp32 per code (src/quantization.cpp:32-37,127-153);
// this library streams packed codes instead.  Both packed layouts are
// strip-major: the [K,N] weight is cut into strips of SW consecutive columns,
// each strip is stored contiguously over all rows, four rows ("a row quad")
// per 16-byte chunk.  Chunk (strip j, row quad rq) sits at byte
// (j * RQ + rq) * 16 with RQ = Kpad / 4.  A workgroup that owns a few strips
// therefore streams a few long contiguous runs, and a wavefront whose lanes
// take consecutive row quads of a strip reads 16 * lanes contiguous bytes.
//
//   INT8 (SW = 4):  dword d of a chunk is column 4*j + d; byte r of that
//                   dword is row 4*rq + r.  Two's-complement int8 codes.
//   INT4 (SW = 8):  dword r of a chunk is row 4*rq + r; nibble e (bits
//                   4e..4e+3) is column 8*j + e.  Two's-complement int4.
//
// Rows past K (Kpad = K rounded up to 16) and columns past N are padding
// with code 0.  INT4 strip-major keeps its scales transposed,
// devscales[sc][Kpad], one column per `spc` strips: spc = group/8 when
// N % group == 0 (groups never straddle rows, so a whole group of columns
// shares one scale per row), else spc = 1 (one scale per strip and row; valid
// because group % 8 == 0 and N % 8 == 0 keep every strip inside one group).
// INT4 flat (any other shape) is the flattened tensor with two codes per
// byte, element i in byte i/2, low nibble first.
//
// INT4 strip-major buffers carry a second copy of the codes after the strips,
// at byte koct_off() (the strips' bytes rounded up to 256): k-octet blocks.
// The weight is cut into column blocks of 16 (two strips; NB = ceil(NS / 2))
// and, within each, k blocks of 32 rows (KB = ceil(Kpad / 32)).  Block (cb, kb)
// is 256 bytes at koct_off() + (cb * KB + kb) * 256, so a column block is one
// contiguous run over K.  Dword t = 16 * g + c of a block (g = 0..3, c =
// 0..15) holds column 16 * cb + c at rows 32 * kb + 8 * g + i in nibble i;
// rows past Kpad and columns past N are code 0.  A dword is exactly the B
// operand of lane t of a v_mfma_f32_16x16x32_bf16 (eight consecutive k of one
// column) and a block that MFMA's whole B tile, so the whole-K skinny MFMA
// kernel loads one dword per lane with no exchange between lanes.  The GEMV
// stays on the strips: at one batch row it needs one x * s per code dword
// there, eight per dword here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgq {

constexpr int64_t kPadK = 16;  // rows are padded to a multiple of this

// Compute units the launch heuristics plan for: the count of the device a
// stream runs on (a partition of an MI355X reports its own share), at most
// kMaxCus, the full MI355X.  Split-K workspaces are sized for the largest
// need over every count from 1 to kMaxCus.
constexpr int64_t kMaxCus = 256;

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Division of n in [0, 2^31) by a divisor d >= 1 fixed at launch, as a
// multiply-high, an add and a shift (Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994: m = floor(2^32 (2^l - d) / d)
// + 1 with l = ceil(log2 d); then n / d = (mulhi(n, m) + n) >> l, where the sum
// stays below 2^32 because n < 2^31).  Kernels use it for indices that would
// otherwise need a runtime integer division (about 30 dependent instructions).
struct FastDiv {
    uint32_t m;
    int l;
    __host__ __device__ FastDiv() : m(1), l(0) {}
    __host__ explicit FastDiv(uint32_t d) {
        l = 0;
        while ((1ull << l) < d) ++l;
        m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    }
    __host__ __device__ int div(int n) const {
        const uint32_t hi = (uint32_t)(((uint64_t)(uint32_t)n * m) >> 32);
        return (int)((hi + (uint32_t)n) >> l);
    }
};
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

struct I8Geom {
    int64_t K, N, Kpad, RQ, NS;  // NS strips of 4 columns
    explicit I8Geom(int64_t k, int64_t n)
        : K(k), N(n), Kpad(round_up(k, kPadK)), RQ(Kpad / 4), NS(ceil_div(n, 4)) {}
    int64_t chunks() const { return NS * RQ; }
    int64_t bytes() const { return chunks() * 16; }
};

struct I4Geom {
    int64_t K, N, G, Kpad, RQ, NS, spc, nsc;  // NS strips of 8 columns
    bool tiled;
    I4Geom(int64_t k, int64_t n, int64_t g)
        : K(k), N(n), G(g <= 0 ? 32 : g), Kpad(round_up(k, kPadK)), RQ(Kpad / 4), NS(n / 8) {
        tiled = (N % 8 == 0) && (G % 8 == 0);
        spc = (tiled && N % G == 0) ? G / 8 : 1;
        nsc = tiled ? ceil_div(NS, spc) : 0;
    }
    int64_t chunks() const { return tiled ? NS * RQ : 0; }
    // The k-octet copy (strip-major only): KB k blocks of 32 rows, NB column
    // blocks of 16, starting at byte koct_off().
    int64_t KB() const { return ceil_div(Kpad, 32); }
    int64_t NB() const { return ceil_div(NS, 2); }
    int64_t koct_off() const { return round_up(chunks() * 16, 256); }
    int64_t koct_bytes() const { return tiled ? NB() * KB() * 256 : 0; }
    int64_t bytes() const { return tiled ? koct_off() + koct_bytes() : ceil_div(K * N, 2); }
    int64_t devscale_count() const { return tiled ? nsc * Kpad : 0; }
};

constexpr int kGemvMaxM = 16;  // M <= this runs the GEMV, larger M the MFMA GEMM (but see below)
// The plain forward also runs the GEMV for batches of up to this many rows
// (row groups of 8, one workgroup each) when the work is small: the GEMV's
// time grows with M * K * N at the VALU rate from a fixed ~3 us, the GEMM's
// from ~10-15 us of pipeline fill, split-K partials and reduce.  Measured on
// MI355X with each path forced (INT4 g128): at 16 rows the GEMV wins on every
// shape tried (4096->11008 31 vs 35 us, 2048->2048 5.6 vs 11.8 us); from 17
// rows the GEMM's 32- and 64-row tiles win once M * K * N passes about 2^28
// (4096x4096 at 17..32 rows 19-23 vs 23 us, 4096->11008 at 17 rows 35 vs
// 54 us) and lose below it (2048x2048 at 64 rows 17 vs 14 us).
constexpr int64_t kGemvRowsMax = 128;
constexpr int64_t kGemvSmallWork = (int64_t)1 << 28;  // M * K * N
inline bool linear_uses_gemv(int64_t M, int64_t K, int64_t N) {
    return M <= kGemvMaxM || (M <= kGemvRowsMax && M * K * N <= kGemvSmallWork);
}

// Batches of a few to 32 rows over INT4 weights run on the bf16 matrix cores
// (k_skinny3) instead of the GEMV or the GEMM.  The GEMV's cost grows with
// the rows (one FMA per code and row), the MFMA form's hardly at all.  Its
// workgroups own C column blocks of 16 (2C strips must share a scale column,
// so one split of x * s serves them all):
//  - wide weights (at least 5/8 of a workgroup per CU with C = 4 or 2) give
//    each workgroup all of K.  Measured on MI355X (INT4 g128, graphs of 100
//    calls, GEMV -> MFMA): 4096->11008 at 5 / 8 / 16 rows 19.0 / 19.9 / 31.0
//    -> 15.4 / 15.9 / 17.0 us; 2048->6144 at 8 / 16 rows 8.4 / 12.9 -> 7.4 /
//    8.4; 4096->14336 at 16 rows 37.9 -> 17.4.  With B operands from the
//    k-octet copy three and four rows go there too (GEMV -> MFMA, builds
//    interleaved: 4096->11008 at 3 / 4 rows 11.7-12.0 / 12.7-13.3 -> 11.1-11.4
//    / 11.6-11.8 us, 2048->6144 5.2 / 5.3-5.4 -> 5.0-5.1 / 5.1, 8192->28672 at
//    4 rows 46.5-47.0 -> 39.8-40.0); two rows stay on the GEMV (4096->11008
//    8.8 vs 10.9-11.3 us), as does K below 2048.
//  - narrower weights split K into S ranges (a power of two, enough
//    workgroups to fill the device, at least kSkinnyMinRangeBlocks 32-row k
//    blocks each).  Every workgroup of the GEMV or of the unsplit kernel
//    reads all M rows of x, which for M >= 4 is more than its codes; a range
//    reads its own slice.  The partial sums go to the caller's workspace and
//    a second kernel adds them in range order.
constexpr int64_t kSkinnyMinRows = 3;        // wide weights
constexpr int64_t kSkinnyNarrowMinRows = 5;  // split K
constexpr int64_t kSkinnyMaxRows = 32;       // two row blocks of 16
constexpr int64_t kSkinnyMinK = 2048;        // wide weights
constexpr int64_t kSkinnyNarrowMinK = 1024;  // split K
constexpr int64_t kSkinnyMaxK = (int64_t)1 << 24;  // strip offsets (2C strips of Kpad rows) in 32 bits
constexpr int kSkinnyMaxSplits = 16;
constexpr int64_t kSkinnySB = 128;            // rows per super-block (the kernel's unit of K)
constexpr int64_t kSkinnyRangeRows = 8192;    // rows of a K range (its scales are kept in LDS)
constexpr int64_t kSkinnyMinRangeBlocks = 8;  // super-blocks of a split K range, at least
struct SkinnyPlan {
    int C = 0;     // column blocks of 16 per workgroup; 0: not the skinny kernel
    int S = 1;     // K ranges (1: no split, no workspace)
    int MB = 1;    // row blocks of 16
    int form = 1;  // 0: k_skinny3 (whole K, one row block), 1: k_skinny_sb (super-blocks)
};
// Narrow weights split K only from this much work, M rounded up to the
// GEMV's row group of 8 (its time steps up with each group).  Measured (us,
// GEMV or GEMM -> split): 11008 -> 4096 at 8 / 10 / 16 rows 19.6 / 31.7 /
// 32.0 -> 18.3 / 18.5 / 20.2; 4096 -> 4096 at 12 / 16 / 24 rows 14.0 / 14.6 /
// 21.8 -> 10.4 / 10.9 / 14.1; 5632 -> 2048 at 24 rows 20.3 -> 15.6.  Kept:
// 4096 -> 4096 at 8 rows (9.2 vs 10.3), 5632 -> 2048 at 16 (11.7 vs 12.4),
// 2048 -> 2048 (5.8 vs 9.0 at 16 rows), four rows (11008 -> 4096 13.7 vs
// 17.7).
constexpr int64_t kSkinnyNarrowWork = (int64_t)1 << 28;
// K ranges for ncg column groups of a K of nsb super-blocks on cus CUs:
// narrow weights split to fill the device (ranges of at least
// kSkinnyMinRangeBlocks super-blocks); every range holds at most
// kSkinnyRangeRows rows.  0: K is too long for kSkinnyMaxSplits ranges.
inline int skinny_splits(int64_t ncg, int64_t nsb, int64_t cus, bool narrow) {
    int S = 1;
    if (narrow) {
        while (ncg * S < cus && S < kSkinnyMaxSplits) S *= 2;
        while (S > 1 && nsb < kSkinnyMinRangeBlocks * S) S /= 2;
    }
    while (ceil_div(nsb, S) * kSkinnySB > kSkinnyRangeRows) {
        if (S >= kSkinnyMaxSplits) return 0;
        S *= 2;
    }
    return S;
}
inline SkinnyPlan skinny_plan(int64_t M, int64_t K, const I4Geom& g, int64_t cus) {
    SkinnyPlan p;
    // x is addressed through 32-bit buffer offsets: M * K * 4 bytes <= 2^30.
    if (M < 1 || M > kSkinnyMaxRows || K < 1 || K > kSkinnyMaxK || M * K > ((int64_t)1 << 28) || !g.tiled ||
        g.spc % 2 != 0)
        return p;
    const int MB = M > 16 ? 2 : 1;
    const int64_t nsb = ceil_div(g.Kpad, kSkinnySB);
    for (int c = 4; c >= 2; c /= 2)
        if (g.spc % (2 * c) == 0 && g.NS / (2 * c) * 8 >= 5 * cus) {
            if (M < kSkinnyMinRows || K < kSkinnyMinK) return p;
            // One row block: the whole-K form (any K).  Two: super-blocks,
            // K split only as far as the scales of a range fit LDS.
            p.form = MB == 1 ? 0 : 1;
            p.S = MB == 1 ? 1 : skinny_splits(g.NS / (2 * c), nsb, cus, false);
            p.C = p.S > 0 ? c : 0;
            p.MB = MB;
            if (p.C == 0) p.S = 1;
            return p;
        }
    const int c = g.spc % 8 == 0 ? 4 : (g.spc % 4 == 0 ? 2 : 0);
    if (c == 0 || M < kSkinnyNarrowMinRows || K < kSkinnyNarrowMinK) return p;
    if (round_up(M, 8) * K * g.N < kSkinnyNarrowWork) return p;
    p.S = skinny_splits(g.NS / (2 * c), nsb, cus, true);
    p.C = p.S > 1 ? c : 0;  // too short to split (or too long for the ranges): not this kernel
    p.MB = MB;
    if (p.C == 0) p.S = 1;
    return p;
}
// INT8 batches on the bf16 matrix cores (k_skinny8): workgroups of MB row
// blocks of 16 (two above 16 rows) by C column blocks of 16 over all of K, no
// workspace.  C = 2 where that still gives a workgroup per CU.  The GEMV
// keeps four rows and little work (its time is a fixed ~3 us plus
// round_up(M, 8) * K * N at the VALU rate); above 16 rows the GEMM keeps
// M * K * N > 2^29 (its wider tiles read each x row for more columns).
// Measured on MI355X (INT8 per tensor, us, GEMV or GEMM -> skinny): 1024^2 at
// 128 rows 11.2 -> 6.8; 2048^2 at 9 / 64 / 128 rows 6.5 / 16.8 / 27.5 -> 5.7
// / 11.2 / 12.5; 4096^2 at 8 / 16 / 32 rows 11.0 / 17.2 / 20.3 -> 9.3 / 11.8
// / 19.6.  Left to the GEMV: 1024^2 at 16 rows (3.9 vs 5.5), 2048^2 at 8
// (4.7 vs 5.6).  Left to the GEMM: 4096^2 at 80 / 128 rows (30.6 / 33.9 vs
// 40.2 / 41.4), 4096 -> 11008 at 32 rows (28.6 vs 41.5); 4096^2 at 64 rows
// (24.6 vs 22.2) falls past the bound too.
constexpr int64_t kSkinny8MinRows = 5;
constexpr int64_t kSkinny8MaxRows = 128;
constexpr int64_t kSkinny8MinWork = (int64_t)1 << 26;  // round_up(M, 8) * K * N
constexpr int64_t kSkinny8MaxWork = (int64_t)1 << 29;  // M * K * N, above 16 rows
struct Skinny8Plan {
    int C = 0;   // column blocks of 16 per workgroup; 0: not this kernel
    int MB = 1;  // row blocks of 16
};
inline Skinny8Plan skinny8_plan(int64_t M, int64_t K, int64_t N, int64_t cus) {
    Skinny8Plan p;
    // x rows of a tile ((16 MB) * K * 4 bytes) through 32-bit offsets.
    if (M < kSkinny8MinRows || M > kSkinny8MaxRows || K < 1 || K >= kSkinnyMaxK || N < 1) return p;
    if (round_up(M, 8) * K * N < kSkinny8MinWork) return p;
    if (M > kGemvMaxM && M * K * N > kSkinny8MaxWork) return p;
    p.MB = M > 16 ? 2 : 1;
    p.C = ceil_div(M, 16 * p.MB) * ceil_div(ceil_div(N, 4), 8) >= cus ? 2 : 1;
    return p;
}
// Workspace of a skinny launch with NG weights: the K ranges' partial sums.
inline int64_t skinny_ws_bytes(const SkinnyPlan& p, int64_t M, int64_t N, int NG) {
    return p.C > 0 && p.S > 1 ? (int64_t)NG * p.S * M * N * 4 : 0;
}
// The largest such workspace over every group size and every device of 1 to
// kMaxCus CUs.  Neither extreme alone bounds it: the K splits of the narrow
// form grow with the CU count, while a device with few CUs can call a weight
// wide that a larger one calls narrow or leaves to the GEMV, and the wide
// form's two-row-block batches split K (as far as the scales of a range fit
// LDS) whatever the CU count.  The wide test (at most a CU count) holds on
// every device below some count and the narrow splits are monotone in it, so
// one CU (every weight that can be wide is) and kMaxCus (the most narrow
// splits) cover all of them; the CPU tests sweep every count to confirm it.
// The group sizes stand for every other: the plan depends on the group only
// through the column blocks per workgroup (2 when spc % 4 == 0, 4 when spc %
// 8 == 0), which 32 and 64 realise wherever any larger group does.
inline int64_t skinny_ws_bound(int64_t M, int64_t K, int64_t N, int NG) {
    int64_t ws = 0;
    for (int64_t G : {16, 32, 64, 128})
        for (int64_t cus : {(int64_t)1, kMaxCus}) {
            const int64_t w = skinny_ws_bytes(skinny_plan(M, K, I4Geom(K, N, G), cus), M, N, NG);
            if (w > ws) ws = w;
        }
    return ws;
}

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

// out[i] = q[i] * scales[idx(i)]: idx = 0 (mode 0), i / div (mode 1).
hipError_t launch_dequant_codes(const float* q, const float* scales, int64_t total, int mode, int64_t div, float* out,
                                hipStream_t s);

// Forward kernels.
hipError_t launch_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, hipStream_t s);
hipError_t launch_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, hipStream_t s);
// INT8 forward on k_skinny8 for a plan of skinny8_plan (C > 0).
hipError_t launch_skinny_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                            bool per_tensor, const float* bias, const Skinny8Plan& p, float* y, hipStream_t s);
// Skinny MFMA forward (plan p from skinny_plan, p.C > 0) of ng (1 or 2) tiled
// INT4 weights of one shape on one input: ng == 1 writes y = x * W + bias,
// ng == 2 the gated MLP h = silu(x * Wg + bg) * (x * Wu + bu).  With split K,
// ws holds skinny_ws_bytes(p, M, N, ng) bytes (16-byte aligned).
// The whole-K form (p.form == 0, p.S == 1) can also run nw (1..3, ng == 1)
// weights of one shape side by side, weight w writing columns w * N .. w * N
// + N - 1 of rows of ldy floats, and fold an RMSNorm of x (gamma, eps) into
// the projections, as launch_gemv_i4_multi does.
struct SkinnyExtra {
    int nw = 1;
    int64_t ldy = 0;  // 0: N
    const float* gamma = nullptr;
    float eps = 0.0f;
};
hipError_t launch_skinny_i4(const float* x, int64_t M, int64_t K, int64_t N, int ng, const void* const* packed,
                            const float* const* devscales, const float* const* bias, const I4Geom& g,
                            const SkinnyPlan& p, float* y, void* ws, hipStream_t s,
                            const SkinnyExtra* extra = nullptr);
// nw (1..3) tiled INT4 weights of one shape [K, N] side by side on one input:
// weight w writes y[m * ldy + w * N + n] (+ res at the same index when res is
// set).  gamma (optional): the input is rms_norm(x, gamma, eps), applied
// inside the kernel.  Strip layout only; M <= kGemvMaxM.
hipError_t launch_gemv_i4_multi(const float* x, int64_t M, int64_t K, int64_t N, int nw, const void* const* packed,
                                const float* const* devscales, const float* const* bias, const I4Geom& g, float* y,
                                int64_t ldy, const float* res, const float* gamma, float eps, hipStream_t s);
// MFMA GEMM (M > kGemvMaxM).  Grids with fewer 128x128 tiles than CUs split K
// over workgroups; their partial tiles go to ws (gemm_workspace_bytes(M, K, N)
// bytes, 0 when K is not split) and a second kernel adds them in fixed order.
struct GemmPlan {
    int KS, sps;  // splits of K, 32-row stages per split
};
struct GemmTile {
    int64_t bm, bn, per_cu;  // tile rows and columns, workgroups resident per CU
};
int device_cus(hipStream_t s);
// XCDs of the device `s` runs on (hipDeviceAttributeNumberOfXccs, 1 if the
// runtime does not say, at most kMaxXcds), read once per device; the kernels
// that place workgroups by XCD take xcd_log2 of it (0, the identity order,
// for a count that is not a power of two).
constexpr int kMaxXcds = 16;
int device_xcds(hipStream_t s);
int xcd_log2(int xcds);
// Tile rows of the GEMM's per-XCD rectangles for this shape on a device of
// `cus` CUs and `xcds` XCDs (0: the plain order; the grid splits K or does
// not tile into one rectangle per XCD).  mode: INT4 strips per scale column.
int gemm_rect_rows(int bits, int64_t M, int64_t K, int64_t N, int mode, int64_t cus, int64_t xcds);
GemmPlan gemm_plan(int64_t M, int64_t K, int64_t N, const GemmTile& t, int64_t cus);
// Tile of the three-term GEMM for a code width and batch: 32 or 64 rows by
// 128 columns for batches of up to 32 or 64 rows, else 128 x 256 (INT8) or
// 128 x 128 (INT4).
GemmTile gemm_tile(int bits, int64_t M);
int64_t gemm_workspace_bytes(int64_t M, int64_t K, int64_t N);
// The workspace bytes the GEMM launch of this shape (INT4: mode = spc, INT8:
// unused) takes on `cus` compute units: what launch_gemm_i8/i4 writes.
int64_t gemm_launch_ws_bytes(int bits, int64_t M, int64_t K, int64_t N, int mode, int64_t cus);
// The plan a forward of this shape runs on `cus` compute units: path 0 the
// GEMV, 1 the three-term bf16 GEMM, 2 the fp32 GEMM, 3 the flat INT4 kernel,
// 4 the skinny MFMA kernel; ks the K splits (1: none).
void linear_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int64_t cus, int* path, int* ks);
hipError_t launch_gemm_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                          bool per_tensor, const float* bias, float* y, void* ws, hipStream_t s);
hipError_t launch_gemm_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                          const float* devscales, const I4Geom& g, const float* bias, float* y, void* ws,
                          hipStream_t s);
hipError_t launch_linear_i4_flat(const float* x, int64_t M, int64_t K, int64_t N, const void* packed,
                                 const float* scales, int64_t G, const float* bias, float* y, hipStream_t s);

// Gated MLP: h = silu(x*Wg + bg) * (x*Wu + bu).  The GEMV form (M <= kGemvMaxM)
// runs both weights in one launch (as does the skinny kernel, launch_skinny_i4
// with ng == 2); larger batches run two projections and launch_silu_mul
// (h = silu(h) * u, elementwise over n floats).
hipError_t launch_swiglu_gemv_i8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_g,
                                 const float* scales_g, const float* bias_g, const void* packed_u,
                                 const float* scales_u, const float* bias_u, bool per_tensor, float* h,
                                 hipStream_t s);
hipError_t launch_swiglu_gemv_i4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_g,
                                 const float* devscales_g, const float* bias_g, const void* packed_u,
                                 const float* devscales_u, const float* bias_u, const I4Geom& g, float* h,
                                 hipStream_t s, const float* gamma = nullptr, float eps = 0.0f);
hipError_t launch_silu_mul(float* h, const float* u, int64_t n, hipStream_t s);

// ---- LLaMA block decode step (sgq_decode.hip) ---------------------------
hipError_t launch_rms_norm(const float* x, int64_t rows, int64_t D, const float* g, float eps, float* out,
                           hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* y, int64_t n, hipStream_t s);
hipError_t launch_embedding(const float* idx, int64_t n, const float* w, int64_t V, int64_t E, float* out,
                            hipStream_t s);
// Attention of one new token per sequence over its cache: keys split into
// NC chunks of CS, combined by a second kernel when NC > 1.
constexpr int kAttnMaxChunk = 64;     // keys per chunk
constexpr int kAttnMaxChunks = 1024;  // chunks per sequence (max_len <= 65536)
struct AttnPlan {
    int CS, NC;
};
AttnPlan attn_plan(int64_t B, int64_t max_len);
int64_t attn_max_len();
int64_t attn_workspace_floats(int64_t B, int64_t D, int64_t max_len);
// q, knew, vnew: rows of B sequences with row stride ldq; kc, vc: [B][max_tokens][D];
// pos[b]: cached positions of sequence b before this step (the new row goes
// to pos[b]); part: attn_workspace_floats floats; ctx: [B, D].
hipError_t launch_attention_decode(const float* q, const float* knew, const float* vnew, int64_t ldq, int64_t B,
                                   int64_t D, float* kc, float* vc, int64_t max_tokens, const int32_t* pos,
                                   int64_t max_len, float scale, float* part, float* ctx, hipStream_t s);

}  // namespace sgq
