// sgq_abi.hip -- the extern "C" entry points of libsgq.so (declared in include/sgq.h).
//
// Every function validates its arguments on the host, then enqueues kernels
// on the caller's stream.  No allocation; the only per-thread state is the
// last error message.  The one piece of process state is the per-device
// address of the static scratch array used by sgq_linear_int4_noalloc
// (written once per device).
#include "sgq.h"
#include "sgq_internal.h"

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>

#define SGQ_ABI_VERSION 2

using namespace sgq;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return SGQ_OK;
}

#define SGQ_HIP(expr, what)                                                                   \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) return fail(SGQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e_)); \
    } while (0)

constexpr int64_t kMaxDim = (int64_t)1 << 30;
constexpr int64_t kAlign = 256;
constexpr int64_t kPartialMax = 1024;

int64_t align_up(int64_t v) { return round_up(v, kAlign); }

// Quantize / pack workspace: [inv: ngroups floats][partials: 1024 floats][bad flag].
struct QuantWs {
    int64_t inv_off, part_off, bad_off, total;
};
QuantWs quant_ws(int64_t ngroups) {
    QuantWs w;
    w.inv_off = 0;
    w.part_off = align_up((ngroups > 0 ? ngroups : 1) * 4);
    w.bad_off = w.part_off + align_up(kPartialMax * 4);
    w.total = w.bad_off + kAlign;
    return w;
}

int64_t int4_groups(int64_t total, int64_t G) { return ceil_div(total, G <= 0 ? 32 : G); }

// A workspace holds split-K partials: of the GEMM when its tile grid is
// smaller than the GPU (see gemm_plan), of the skinny INT4 kernel over weights
// too narrow to fill it (see skinny_plan); the GEMV owns whole columns.  The
// size is the largest either could need on any device and for any group
// size (neither is an argument here).
int64_t linear_ws_bytes(int bits, int64_t M, int64_t K, int64_t N) {
    // The INT8 skinny kernel's batches (on any device) need none.
    if (bits == 8 && skinny8_plan(M, K, N, kMaxCus).C > 0) return 0;
    const int64_t gemm = linear_uses_gemv(M, K, N) ? 0 : gemm_workspace_bytes(M, K, N);
    const int64_t skinny = bits == 4 ? skinny_ws_bound(M, K, N, 1) : 0;
    return gemm > skinny ? gemm : skinny;
}

int check_linear_ws(const char* fn, int bits, int64_t M, int64_t K, int64_t N, const void* workspace,
                    int64_t workspace_bytes) {
    const int64_t need = linear_ws_bytes(bits, M, K, N);
    if (need == 0) return ok();
    if (!workspace || workspace_bytes < need)
        return fail(SGQ_ERR_WORKSPACE, "%s: workspace needs %lld bytes", fn, (long long)need);
    if ((((uintptr_t)workspace) & 15) != 0) return fail(SGQ_ERR_WORKSPACE, "%s: workspace must be 16-byte aligned", fn);
    return ok();
}

// Gated MLP workspace: nothing for the one-launch GEMV; otherwise
// [up projection: M*N floats, 256-byte aligned][split-K partials of either GEMM].
// The flat INT4 layout always takes the two-projection form.  Tiled INT4
// batches the skinny kernel takes (one launch for both weights) need its
// split-K partials of both weights; the size covers every device (a device
// with fewer CUs may run the GEMV or GEMM form instead).
int64_t swiglu_ws_bytes(int bits, bool flat, int64_t M, int64_t K, int64_t N, int64_t group_size) {
    int64_t skinny = 0;
    if (bits == 4 && !flat && K > 0)
        for (int64_t cus : {(int64_t)1, kMaxCus}) {  // every device (see skinny_ws_bound)
            const int64_t w = skinny_ws_bytes(skinny_plan(M, K, I4Geom(K, N, group_size), cus), M, N, 2);
            if (w > skinny) skinny = w;
        }
    int64_t other = 0;
    // The one-launch GEMV form takes the batches the plain forward runs on the
    // GEMV; INT8 batches of the skinny kernel run it once per weight, up into
    // the workspace (no split K).
    const bool skinny8 = bits == 8 && K > 0 && skinny8_plan(M, K, N, kMaxCus).C > 0;
    if (flat || skinny8 || !linear_uses_gemv(M, K, N) || K == 0) {
        const int64_t split =
            (!flat && !skinny8 && !linear_uses_gemv(M, K, N)) ? gemm_workspace_bytes(M, K, N) : 0;
        other = align_up(M * N * 4) + split;
    }
    return skinny > other ? skinny : other;
}

bool aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

// The launch about to run takes `need` bytes of workspace (its plan on this
// device): refuse it when the caller passed less.  The size queries bound
// every device's need, so this only fails for a workspace sized by hand.
int check_launch_ws(const char* fn, int64_t need, const void* workspace, int64_t workspace_bytes) {
    if (need <= 0) return SGQ_OK;
    if (!workspace || workspace_bytes < need)
        return fail(SGQ_ERR_WORKSPACE, "%s: this device's launch needs %lld bytes of workspace", fn, (long long)need);
    if (!aligned16(workspace)) return fail(SGQ_ERR_WORKSPACE, "%s: workspace must be 16-byte aligned", fn);
    return SGQ_OK;
}

// LLaMA block decode workspace, each region 256-byte aligned:
//   n [B*D] | qkv [3*B*D] | ctx [B*D] | h [B*D] | hid [B*H] | tmp [B*max(D,H)]
//   | attention partials | GEMM split-K partials (the GEMM path only)
struct DecodeWs {
    int64_t n, qkv, ctx, h, hid, tmp, part, split, total;
};
// The block's GEMV forms (RMSNorm folded in, q/k/v side by side, residual
// epilogues) serve the batches on which every projection runs the GEMV.
bool decode_uses_gemv(int64_t B, int64_t D, int64_t H) {
    return linear_uses_gemv(B, D, 3 * D) && linear_uses_gemv(B, D, H) && linear_uses_gemv(B, H, D);
}

// The block's norm-fused projections on the GEMV path run the skinny MFMA
// kernel's whole-K form instead where the forward's plan gives it for the
// projection's total width (q, k and v side by side: 3 * N), with two column
// blocks per workgroup (the norm-fused form), which must tile each weight.
SkinnyPlan decode_skinny_plan(int64_t B, int64_t K, int64_t N, int nw, int64_t G, int cus) {
    const I4Geom g(K, N, G);
    SkinnyPlan p = skinny_plan(B, K, I4Geom(K, nw * N, G), cus);
    if (p.C == 0 || p.form != 0 || p.S != 1 || g.spc % 4 != 0 || g.NS % 4 != 0) return SkinnyPlan{};
    return p;
}

DecodeWs decode_ws(int64_t B, int64_t D, int64_t H, int64_t max_len) {
    DecodeWs w;
    int64_t o = 0;
    auto take = [&](int64_t floats) {
        const int64_t at = o;
        o += align_up((floats > 0 ? floats : 1) * 4);
        return at;
    };
    w.n = take(B * D);
    w.qkv = take(3 * B * D);
    w.ctx = take(B * D);
    w.h = take(B * D);
    w.hid = take(B * H);
    w.tmp = take(B * (D > H ? D : H));
    w.part = take(attn_workspace_floats(B, D, max_len));
    int64_t split = 0;
    if (!decode_uses_gemv(B, D, H)) {
        const int64_t a = gemm_workspace_bytes(B, D, D), b = gemm_workspace_bytes(B, D, H),
                      c = gemm_workspace_bytes(B, H, D);
        split = a > b ? a : b;
        split = split > c ? split : c;
    }
    w.split = o;
    o += align_up(split > 0 ? split : 1);
    w.total = o;
    return w;
}

bool bad_dims(int64_t a, int64_t b) { return a < 0 || b < 0 || a > kMaxDim || b > kMaxDim || a * b > ((int64_t)1 << 40); }

// The forward kernels address a strip of codes, a scale column and a row of x
// (GEMV: Kpad * 4 bytes each) or a 128-row tile of x (GEMM: 128 * K * 4 bytes)
// through 32-bit buffer offsets.  Shapes past those limits are refused with
// SGQ_ERR_UNSUPPORTED instead of wrapping into wrong outputs.
constexpr int64_t kGemvMaxKpad = ((int64_t)1 << 29) - kPadK;  // Kpad * 4 < 2^31
constexpr int64_t kGemmMaxK = (int64_t)1 << 22;               // 128 * K * 4 <= 2^31
bool forward_fits(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size) {
    if (round_up(K, kPadK) > kGemvMaxKpad) return false;
    if (linear_uses_gemv(M, K, N)) return true;
    if (K > kGemmMaxK) return false;
    if (bits == 4) {  // the fp32-MFMA kernel (groups not a multiple of 128) maps all devscales at once
        const I4Geom g(K, N, group_size);
        if (g.tiled && g.spc % 16 != 0 && g.devscale_count() * 4 >= ((int64_t)1 << 32)) return false;
    }
    return true;
}

int check_codes_flag(const int* dflag, hipStream_t s) {
    int host_flag = 0;
    SGQ_HIP(hipMemcpyAsync(&host_flag, dflag, sizeof(int), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(flag)");
    SGQ_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (host_flag) return fail(SGQ_ERR_CODES, "qdata holds a value that is not an integer code in range");
    return ok();
}


// ---- static scratch of sgq_linear_int4_noalloc ------------------------------
// The split-K partials of the no-allocation forward live in this array: one
// copy per GPU, created when the library's code object is loaded on that GPU
// and held until the process ends.  Host code never uses the array's name as
// an address (on the host it is a stand-in symbol); the device address comes
// from hipGetSymbolAddress, once per device, with that device current.
constexpr int64_t kScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
std::once_flag g_scratch_once[kScratchDevices];
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_status[kScratchDevices];

// The scratch address on the device `stream` runs on, which must be the
// calling thread's current device (the symbol is resolved with it current).
int scratch_for_stream(const char* fn, hipStream_t stream, void** out) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) {
        (void)hipGetLastError();
        return fail(SGQ_ERR_HIP, "%s: no current device", fn);
    }
    if (stream) {
        int sdev = cur;
        if (hipStreamGetDevice(stream, &sdev) != hipSuccess) {
            (void)hipGetLastError();
            return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: cannot query the stream's device", fn);
        }
        if (sdev != cur)
            return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: the stream's device (%d) is not the current device (%d)", fn,
                        sdev, cur);
    }
    if (cur < 0 || cur >= kScratchDevices) return fail(SGQ_ERR_UNSUPPORTED, "%s: device %d out of range", fn, cur);
    std::call_once(g_scratch_once[cur], [cur] {
        void* p = nullptr;
        g_scratch_status[cur] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (g_scratch_status[cur] != hipSuccess) (void)hipGetLastError();
        g_scratch_ptr[cur] = p;
    });
    if (g_scratch_status[cur] != hipSuccess || !g_scratch_ptr[cur])
        return fail(SGQ_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(g_scratch_status[cur]));
    *out = g_scratch_ptr[cur];
    return SGQ_OK;
}

int linear_int4(const char* fn, const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                const float* devscales, int64_t group_size, const float* bias, float* y, void* workspace,
                int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad shape", fn);
    if (M == 0 || N == 0) return ok();
    if (!y) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    if (K == 0) {
        SGQ_HIP(launch_fill_bias(y, M, N, bias, s), "fill_bias");
        return ok();
    }
    const I4Geom g(K, N, group_size);
    if (!x || !packed) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (!g.tiled) {
        if (!scales) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: flat layout needs scales", fn);
        SGQ_HIP(launch_linear_i4_flat(x, M, K, N, packed, scales, g.G, bias, y, s), "linear_i4_flat");
        return ok();
    }
    if (!devscales) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: tiled layout needs devscales", fn);
    if (!aligned16(packed) || !aligned16(devscales))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: packed and devscales must be 16-byte aligned", fn);
    if (!forward_fits(4, M, K, N, g.G))
        return fail(SGQ_ERR_UNSUPPORTED, "%s: K = %lld is too long for this batch", fn, (long long)K);
    const int st = check_linear_ws(fn, 4, M, K, N, workspace, workspace_bytes);
    if (st != SGQ_OK) return st;
    const int cus = device_cus(s);
    const SkinnyPlan sp = skinny_plan(M, K, g, cus);
    if (sp.C > 0) {
        const int lw = check_launch_ws(fn, skinny_ws_bytes(sp, M, N, 1), workspace, workspace_bytes);
        if (lw != SGQ_OK) return lw;
        SGQ_HIP(launch_skinny_i4(x, M, K, N, 1, &packed, &devscales, &bias, g, sp, y, workspace, s), "skinny_i4");
    } else if (linear_uses_gemv(M, K, N)) {
        SGQ_HIP(launch_gemv_i4(x, M, K, N, packed, devscales, g, bias, y, s), "gemv_i4");
    } else {
        const int lw = check_launch_ws(fn, gemm_launch_ws_bytes(4, M, K, N, (int)g.spc, cus), workspace,
                                       workspace_bytes);
        if (lw != SGQ_OK) return lw;
        SGQ_HIP(launch_gemm_i4(x, M, K, N, packed, devscales, g, bias, y, workspace, s), "gemm_i4");
    }
    return ok();
}

}  // namespace

extern "C" {

const char* sgq_last_error(void) { return g_err; }

int sgq_abi_version(void) { return SGQ_ABI_VERSION; }

int64_t sgq_int8_packed_bytes(int64_t K, int64_t N) {
    if (bad_dims(K, N)) return -1;
    return I8Geom(K, N).bytes();
}

int sgq_int4_layout(int64_t K, int64_t N, int64_t group_size) {
    return I4Geom(K, N, group_size).tiled ? SGQ_LAYOUT_INT4_TILED : SGQ_LAYOUT_INT4_FLAT;
}

int64_t sgq_int4_packed_bytes(int64_t K, int64_t N, int64_t group_size) {
    if (bad_dims(K, N)) return -1;
    return I4Geom(K, N, group_size).bytes();
}

int64_t sgq_int4_devscale_count(int64_t K, int64_t N, int64_t group_size) {
    if (bad_dims(K, N)) return -1;
    return I4Geom(K, N, group_size).devscale_count();
}

int64_t sgq_int8_scale_count(int64_t rows, int64_t cols, int scheme) {
    if (bad_dims(rows, cols)) return -1;
    return scheme == SGQ_PER_TENSOR_SYMMETRIC ? 1 : rows;
}

int64_t sgq_int4_scale_count(int64_t rows, int64_t cols, int64_t group_size) {
    if (bad_dims(rows, cols)) return -1;
    return int4_groups(rows * cols, group_size);
}

int64_t sgq_quantize_workspace_bytes(int bits, int64_t rows, int64_t cols, int64_t group_size) {
    if (bad_dims(rows, cols)) return -1;
    const int64_t ngroups = bits == 8 ? rows : int4_groups(rows * cols, group_size);
    return quant_ws(ngroups).total;
}

int64_t sgq_linear_workspace_bytes(int bits, int64_t M, int64_t K, int64_t N) {
    if (bad_dims(M, K) || bad_dims(K, N) || (bits != 8 && bits != 4)) return -1;
    return linear_ws_bytes(bits, M, K, N);
}

int sgq_linear_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int compute_units, int* path,
                    int* k_splits) {
    if (bad_dims(M, K) || bad_dims(K, N) || (bits != 8 && bits != 4) || compute_units < 0 || !path || !k_splits)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_plan: bad argument");
    const int64_t cus = compute_units > 0 ? compute_units : device_cus(nullptr);
    linear_plan(bits, M, K, N, group_size, cus, path, k_splits);
    return ok();
}

int sgq_gemm_xcd_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int compute_units, int xcds,
                      int* rect_rows, int* xcd_log2_out) {
    if (bad_dims(M, K) || bad_dims(K, N) || (bits != 8 && bits != 4) || compute_units < 0 || xcds < 0 ||
        !rect_rows || !xcd_log2_out)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_gemm_xcd_plan: bad argument");
    const int64_t cus = compute_units > 0 ? compute_units : device_cus(nullptr);
    int64_t x = xcds > 0 ? xcds : device_xcds(nullptr);
    if (x > kMaxXcds) x = kMaxXcds;
    const int mode = bits == 4 ? (int)I4Geom(K, N, group_size).spc : 0;
    *rect_rows = gemm_rect_rows(bits, M, K, N, mode, cus < kMaxCus ? cus : kMaxCus, x);
    *xcd_log2_out = xcd_log2((int)x);
    return ok();
}

int64_t sgq_swiglu_workspace_bytes(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size) {
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N) || (bits != 8 && bits != 4)) return -1;
    if (M == 0 || N == 0) return 0;
    return swiglu_ws_bytes(bits, bits == 4 && !I4Geom(K, N, group_size).tiled, M, K, N, group_size);
}

int sgq_workspace_init(void* workspace, int64_t workspace_bytes, void* stream) {
    if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_workspace_init: bad workspace");
    SGQ_HIP(launch_fill_zero(workspace, workspace_bytes, (hipStream_t)stream), "fill_zero");
    return ok();
}

int sgq_quantize_int8(const float* x, int64_t rows, int64_t cols, int scheme, float* qdata_f32, float* scales,
                      void* packed, void* workspace, int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(rows, cols)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int8: bad shape");
    if (scheme != SGQ_PER_TENSOR_SYMMETRIC && scheme != SGQ_PER_CHANNEL_SYMMETRIC)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int8: scheme must be per-tensor or per-channel");
    if (scheme == SGQ_PER_CHANNEL_SYMMETRIC && rows == 0)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int8: per-channel needs rows > 0");
    const int64_t total = rows * cols;
    if (!scales || (total > 0 && !x)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int8: null pointer");
    if (packed && !aligned16(packed))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int8: packed must be 16-byte aligned");
    const QuantWs w = quant_ws(rows);
    if (!workspace || workspace_bytes < w.total)
        return fail(SGQ_ERR_WORKSPACE, "sgq_quantize_int8: workspace needs %lld bytes", (long long)w.total);
    char* ws = (char*)workspace;
    float* inv = (float*)(ws + w.inv_off);
    const bool per_tensor = scheme == SGQ_PER_TENSOR_SYMMETRIC;
    if (per_tensor) {
        float* part = (float*)(ws + w.part_off);
        const int64_t nparts = absmax_partial_count(total);
        SGQ_HIP(launch_absmax_partial(x, total, part, nparts, s), "absmax_partial");
        SGQ_HIP(launch_group_scales(part, nparts, nparts, 1, 127.0f, scales, inv, s), "group_scales");
    } else {
        SGQ_HIP(launch_group_scales(x, total, cols, rows, 127.0f, scales, inv, s), "group_scales");
    }
    if ((packed || qdata_f32) && total > 0)
        SGQ_HIP(launch_pack_i8_tiled(x, false, rows, cols, inv, per_tensor, packed, qdata_f32, nullptr, s),
                "pack_i8_tiled");
    return ok();
}

int sgq_quantize_int4(const float* x, int64_t rows, int64_t cols, int64_t group_size, float* qdata_f32,
                      float* scales, void* packed, float* devscales, void* workspace, int64_t workspace_bytes,
                      void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(rows, cols)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int4: bad shape");
    const int64_t total = rows * cols;
    const I4Geom g(rows, cols, group_size);
    const int64_t ngroups = int4_groups(total, g.G);
    if ((ngroups > 0 && !scales) || (total > 0 && !x))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int4: null pointer");
    if (packed && g.tiled && !devscales)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int4: tiled layout needs devscales");
    if (packed && g.tiled && !aligned16(packed))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_quantize_int4: packed must be 16-byte aligned");
    const QuantWs w = quant_ws(ngroups);
    if (!workspace || workspace_bytes < w.total)
        return fail(SGQ_ERR_WORKSPACE, "sgq_quantize_int4: workspace needs %lld bytes", (long long)w.total);
    float* inv = (float*)((char*)workspace + w.inv_off);
    if (ngroups > 0) SGQ_HIP(launch_group_scales(x, total, g.G, ngroups, 7.0f, scales, inv, s), "group_scales");
    if (total > 0) {
        if (packed && g.tiled) {
            SGQ_HIP(launch_pack_i4_tiled(x, false, rows, cols, g.G, inv, packed, qdata_f32, nullptr, s),
                    "pack_i4_tiled");
            SGQ_HIP(launch_devscales_i4(scales, g, devscales, s), "devscales_i4");
        } else if (packed || qdata_f32) {
            SGQ_HIP(launch_pack_i4_flat(x, false, total, g.G, inv, packed, qdata_f32, nullptr, s), "pack_i4_flat");
        }
    } else if (packed && g.tiled && g.devscale_count() > 0) {
        SGQ_HIP(launch_devscales_i4(scales, g, devscales, s), "devscales_i4");
    }
    return ok();
}

int sgq_pack_int8(const float* qdata_f32, int64_t K, int64_t N, void* packed, void* workspace,
                  int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int8: bad shape");
    if (!packed || (K * N > 0 && !qdata_f32)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int8: null pointer");
    if (!aligned16(packed)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int8: packed must be 16-byte aligned");
    const QuantWs w = quant_ws(K);
    if (!workspace || workspace_bytes < w.total)
        return fail(SGQ_ERR_WORKSPACE, "sgq_pack_int8: workspace needs %lld bytes", (long long)w.total);
    int* flag = (int*)((char*)workspace + w.bad_off);
    SGQ_HIP(launch_fill_zero(flag, sizeof(int), s), "fill_zero");
    SGQ_HIP(launch_pack_i8_tiled(qdata_f32, true, K, N, nullptr, false, packed, nullptr, flag, s), "pack_i8_tiled");
    return check_codes_flag(flag, s);
}

int sgq_pack_int4(const float* qdata_f32, const float* scales, int64_t K, int64_t N, int64_t group_size,
                  void* packed, float* devscales, void* workspace, int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int4: bad shape");
    const I4Geom g(K, N, group_size);
    if (!packed || (K * N > 0 && (!qdata_f32 || !scales)) || (g.tiled && !devscales))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int4: null pointer");
    if (g.tiled && !aligned16(packed))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_pack_int4: packed must be 16-byte aligned");
    const QuantWs w = quant_ws(int4_groups(K * N, g.G));
    if (!workspace || workspace_bytes < w.total)
        return fail(SGQ_ERR_WORKSPACE, "sgq_pack_int4: workspace needs %lld bytes", (long long)w.total);
    int* flag = (int*)((char*)workspace + w.bad_off);
    SGQ_HIP(launch_fill_zero(flag, sizeof(int), s), "fill_zero");
    if (g.tiled) {
        SGQ_HIP(launch_pack_i4_tiled(qdata_f32, true, K, N, g.G, nullptr, packed, nullptr, flag, s), "pack_i4_tiled");
        SGQ_HIP(launch_devscales_i4(scales, g, devscales, s), "devscales_i4");
    } else {
        SGQ_HIP(launch_pack_i4_flat(qdata_f32, true, K * N, g.G, nullptr, packed, nullptr, flag, s), "pack_i4_flat");
    }
    return check_codes_flag(flag, s);
}

int sgq_unpack_int8(const void* packed, int64_t K, int64_t N, float* qdata_f32, void* stream) {
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_unpack_int8: bad shape");
    if (K * N > 0 && (!packed || !qdata_f32)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_unpack_int8: null pointer");
    if (!aligned16(packed)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_unpack_int8: packed must be 16-byte aligned");
    SGQ_HIP(launch_unpack_i8_tiled(packed, K, N, nullptr, false, qdata_f32, (hipStream_t)stream), "unpack_i8");
    return ok();
}

int sgq_unpack_int4(const void* packed, int64_t K, int64_t N, int64_t group_size, float* qdata_f32, void* stream) {
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_unpack_int4: bad shape");
    if (K * N > 0 && (!packed || !qdata_f32)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_unpack_int4: null pointer");
    const I4Geom g(K, N, group_size);
    hipStream_t s = (hipStream_t)stream;
    if (g.tiled)
        SGQ_HIP(launch_unpack_i4_tiled(packed, K, N, g.G, nullptr, qdata_f32, s), "unpack_i4_tiled");
    else
        SGQ_HIP(launch_unpack_i4_flat(packed, K * N, g.G, nullptr, qdata_f32, s), "unpack_i4_flat");
    return ok();
}

int sgq_dequantize_int8(const void* packed, const float* scales, int scheme, int64_t K, int64_t N, float* out,
                        void* stream) {
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int8: bad shape");
    if (scheme != SGQ_PER_TENSOR_SYMMETRIC && scheme != SGQ_PER_CHANNEL_SYMMETRIC)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int8: bad scheme");
    if (K * N > 0 && (!packed || !scales || !out))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int8: null pointer");
    if (K * N > 0 && !aligned16(packed))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int8: packed must be 16-byte aligned");
    SGQ_HIP(launch_unpack_i8_tiled(packed, K, N, scales, scheme == SGQ_PER_TENSOR_SYMMETRIC, out,
                                   (hipStream_t)stream),
            "unpack_i8");
    return ok();
}

int sgq_dequantize_int4(const void* packed, const float* scales, int64_t K, int64_t N, int64_t group_size,
                        float* out, void* stream) {
    if (bad_dims(K, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int4: bad shape");
    if (K * N > 0 && (!packed || !scales || !out))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int4: null pointer");
    const I4Geom g(K, N, group_size);
    if (K * N > 0 && g.tiled && !aligned16(packed))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_int4: packed must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    if (g.tiled)
        SGQ_HIP(launch_unpack_i4_tiled(packed, K, N, g.G, scales, out, s), "unpack_i4_tiled");
    else
        SGQ_HIP(launch_unpack_i4_flat(packed, K * N, g.G, scales, out, s), "unpack_i4_flat");
    return ok();
}

int sgq_dequantize_codes(const float* qdata_f32, const float* scales, int bits, int scheme, int64_t rows,
                         int64_t cols, int64_t group_size, float* out, void* stream) {
    if (bad_dims(rows, cols)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_codes: bad shape");
    if (bits != 8 && bits != 4) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_codes: bits must be 8 or 4");
    if (bits == 8 && scheme != SGQ_PER_TENSOR_SYMMETRIC && scheme != SGQ_PER_CHANNEL_SYMMETRIC)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_codes: bad scheme");
    const int64_t total = rows * cols;
    if (total == 0) return ok();
    if (!qdata_f32 || !scales || !out) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_dequantize_codes: null pointer");
    int mode = 1;
    int64_t div = 1;
    if (bits == 8) {
        mode = scheme == SGQ_PER_TENSOR_SYMMETRIC ? 0 : 1;
        div = cols;
    } else {
        div = group_size <= 0 ? 32 : group_size;
    }
    SGQ_HIP(launch_dequant_codes(qdata_f32, scales, total, mode, div, out, (hipStream_t)stream), "dequant_codes");
    return ok();
}

int sgq_linear_int8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                    int scheme, const float* bias, float* y, void* workspace, int64_t workspace_bytes,
                    void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_int8: bad shape");
    if (scheme != SGQ_PER_TENSOR_SYMMETRIC && scheme != SGQ_PER_CHANNEL_SYMMETRIC)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_int8: bad scheme");
    if (M == 0 || N == 0) return ok();
    if (!y) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_int8: null output");
    if (K == 0) {
        SGQ_HIP(launch_fill_bias(y, M, N, bias, s), "fill_bias");
        return ok();
    }
    if (!x || !packed || !scales) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_int8: null pointer");
    const bool per_tensor = scheme == SGQ_PER_TENSOR_SYMMETRIC;
    if (!aligned16(packed) || (!per_tensor && !aligned16(scales)))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_linear_int8: packed and per-channel scales must be 16-byte aligned");
    if (!forward_fits(8, M, K, N, 0))
        return fail(SGQ_ERR_UNSUPPORTED, "sgq_linear_int8: K = %lld is too long for this batch", (long long)K);
    const Skinny8Plan sp = skinny8_plan(M, K, N, device_cus(s));
    if (sp.C > 0) {
        SGQ_HIP(launch_skinny_i8(x, M, K, N, packed, scales, per_tensor, bias, sp, y, s), "skinny_i8");
    } else if (linear_uses_gemv(M, K, N)) {
        SGQ_HIP(launch_gemv_i8(x, M, K, N, packed, scales, per_tensor, bias, y, s), "gemv_i8");
    } else {
        const int st = check_linear_ws("sgq_linear_int8", 8, M, K, N, workspace, workspace_bytes);
        if (st != SGQ_OK) return st;
        const int lw = check_launch_ws("sgq_linear_int8", gemm_launch_ws_bytes(8, M, K, N, 0, device_cus(s)),
                                       workspace, workspace_bytes);
        if (lw != SGQ_OK) return lw;
        SGQ_HIP(launch_gemm_i8(x, M, K, N, packed, scales, per_tensor, bias, y, workspace, s), "gemm_i8");
    }
    return ok();
}

int sgq_linear_int4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                    const float* devscales, int64_t group_size, const float* bias, float* y, void* workspace,
                    int64_t workspace_bytes, void* stream) {
    return linear_int4("sgq_linear_int4", x, M, K, N, packed, scales, devscales, group_size, bias, y, workspace,
                       workspace_bytes, stream);
}

int sgq_linear_int4_noalloc(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                            const float* devscales, int64_t group_size, const float* bias, float* y, void* stream) {
    const char* fn = "sgq_linear_int4_noalloc";
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad shape", fn);
    const int64_t need = linear_ws_bytes(4, M, K, N);
    if (need > kScratchBytes)
        return fail(SGQ_ERR_UNSUPPORTED, "%s: this shape needs %lld bytes of scratch, more than the %lld of the static "
                    "array (use sgq_linear_int4 with a workspace)", fn, (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    if (need > 0) {
        const int st = scratch_for_stream(fn, (hipStream_t)stream, &ws);
        if (st != SGQ_OK) return st;
    }
    return linear_int4(fn, x, M, K, N, packed, scales, devscales, group_size, bias, y, ws, need > 0 ? kScratchBytes : 0,
                       stream);
}

int sgq_swiglu_int8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_gate,
                    const float* scales_gate, const float* bias_gate, const void* packed_up, const float* scales_up,
                    const float* bias_up, int scheme, float* h, void* workspace, int64_t workspace_bytes,
                    void* stream) {
    hipStream_t s = (hipStream_t)stream;
    const char* fn = "sgq_swiglu_int8";
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad shape", fn);
    if (scheme != SGQ_PER_TENSOR_SYMMETRIC && scheme != SGQ_PER_CHANNEL_SYMMETRIC)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad scheme", fn);
    if (M == 0 || N == 0) return ok();
    if (!h) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    const int64_t need = swiglu_ws_bytes(8, false, M, K, N, 0);
    if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
        return fail(SGQ_ERR_WORKSPACE, "%s: workspace needs %lld bytes, 16-byte aligned", fn, (long long)need);
    float* u = (float*)workspace;
    if (K == 0) {  // both projections are their biases
        SGQ_HIP(launch_fill_bias(h, M, N, bias_gate, s), "fill_bias");
        SGQ_HIP(launch_fill_bias(u, M, N, bias_up, s), "fill_bias");
        SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
        return ok();
    }
    if (!x || !packed_gate || !scales_gate || !packed_up || !scales_up)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    const bool per_tensor = scheme == SGQ_PER_TENSOR_SYMMETRIC;
    if (!aligned16(packed_gate) || !aligned16(packed_up) ||
        (!per_tensor && (!aligned16(scales_gate) || !aligned16(scales_up))))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: packed and per-channel scales must be 16-byte aligned", fn);
    if (!forward_fits(8, M, K, N, 0))
        return fail(SGQ_ERR_UNSUPPORTED, "%s: K = %lld is too long for this batch", fn, (long long)K);
    // The skinny kernel's batches take it for both projections, so that the
    // gated MLP's sums are those of two forward calls.
    const Skinny8Plan sp = skinny8_plan(M, K, N, device_cus(s));
    if (sp.C > 0) {
        SGQ_HIP(launch_skinny_i8(x, M, K, N, packed_gate, scales_gate, per_tensor, bias_gate, sp, h, s), "skinny_i8");
        SGQ_HIP(launch_skinny_i8(x, M, K, N, packed_up, scales_up, per_tensor, bias_up, sp, u, s), "skinny_i8");
        SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
        return ok();
    }
    if (linear_uses_gemv(M, K, N)) {
        SGQ_HIP(launch_swiglu_gemv_i8(x, M, K, N, packed_gate, scales_gate, bias_gate, packed_up, scales_up, bias_up,
                                      per_tensor, h, s),
                "swiglu_gemv_i8");
        return ok();
    }
    const int lw = check_launch_ws(fn, align_up(M * N * 4) + gemm_launch_ws_bytes(8, M, K, N, 0, device_cus(s)),
                                   workspace, workspace_bytes);
    if (lw != SGQ_OK) return lw;
    void* split = (char*)workspace + align_up(M * N * 4);
    SGQ_HIP(launch_gemm_i8(x, M, K, N, packed_gate, scales_gate, per_tensor, bias_gate, h, split, s), "gemm_i8");
    SGQ_HIP(launch_gemm_i8(x, M, K, N, packed_up, scales_up, per_tensor, bias_up, u, split, s), "gemm_i8");
    SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
    return ok();
}

int sgq_swiglu_int4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_gate,
                    const float* scales_gate, const float* devscales_gate, const float* bias_gate,
                    const void* packed_up, const float* scales_up, const float* devscales_up, const float* bias_up,
                    int64_t group_size, float* h, void* workspace, int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    const char* fn = "sgq_swiglu_int4";
    if (bad_dims(M, K) || bad_dims(K, N) || bad_dims(M, N)) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad shape", fn);
    if (M == 0 || N == 0) return ok();
    if (!h) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    const I4Geom g(K, N, group_size);
    const int64_t need = swiglu_ws_bytes(4, !g.tiled, M, K, N, group_size);
    if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
        return fail(SGQ_ERR_WORKSPACE, "%s: workspace needs %lld bytes, 16-byte aligned", fn, (long long)need);
    float* u = (float*)workspace;
    if (K == 0) {
        SGQ_HIP(launch_fill_bias(h, M, N, bias_gate, s), "fill_bias");
        SGQ_HIP(launch_fill_bias(u, M, N, bias_up, s), "fill_bias");
        SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
        return ok();
    }
    if (!x || !packed_gate || !packed_up) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (!g.tiled) {
        if (!scales_gate || !scales_up) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: flat layout needs scales", fn);
        SGQ_HIP(launch_linear_i4_flat(x, M, K, N, packed_gate, scales_gate, g.G, bias_gate, h, s), "linear_i4_flat");
        SGQ_HIP(launch_linear_i4_flat(x, M, K, N, packed_up, scales_up, g.G, bias_up, u, s), "linear_i4_flat");
        SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
        return ok();
    }
    if (!devscales_gate || !devscales_up)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: tiled layout needs devscales", fn);
    if (!aligned16(packed_gate) || !aligned16(packed_up) || !aligned16(devscales_gate) || !aligned16(devscales_up))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: packed and devscales must be 16-byte aligned", fn);
    if (!forward_fits(4, M, K, N, g.G))
        return fail(SGQ_ERR_UNSUPPORTED, "%s: K = %lld is too long for this batch", fn, (long long)K);
    // The same path as two forward calls of these shapes, so the gate and up
    // sums are the plain forward's.
    const int cus = device_cus(s);
    const SkinnyPlan sp = skinny_plan(M, K, g, cus);
    if (sp.C > 0) {
        const int lw = check_launch_ws(fn, skinny_ws_bytes(sp, M, N, 2), workspace, workspace_bytes);
        if (lw != SGQ_OK) return lw;
        const void* pk[2] = {packed_gate, packed_up};
        const float* ds[2] = {devscales_gate, devscales_up};
        const float* bs[2] = {bias_gate, bias_up};
        SGQ_HIP(launch_skinny_i4(x, M, K, N, 2, pk, ds, bs, g, sp, h, workspace, s), "skinny_i4");
        return ok();
    }
    if (linear_uses_gemv(M, K, N)) {
        SGQ_HIP(launch_swiglu_gemv_i4(x, M, K, N, packed_gate, devscales_gate, bias_gate, packed_up, devscales_up,
                                      bias_up, g, h, s),
                "swiglu_gemv_i4");
        return ok();
    }
    const int lw = check_launch_ws(fn, align_up(M * N * 4) + gemm_launch_ws_bytes(4, M, K, N, (int)g.spc, cus),
                                   workspace, workspace_bytes);
    if (lw != SGQ_OK) return lw;
    void* split = (char*)workspace + align_up(M * N * 4);
    SGQ_HIP(launch_gemm_i4(x, M, K, N, packed_gate, devscales_gate, g, bias_gate, h, split, s), "gemm_i4");
    SGQ_HIP(launch_gemm_i4(x, M, K, N, packed_up, devscales_up, g, bias_up, u, split, s), "gemm_i4");
    SGQ_HIP(launch_silu_mul(h, u, M * N, s), "silu_mul");
    return ok();
}

int64_t sgq_llama_decode_workspace_bytes(int64_t B, int64_t D, int64_t H, int64_t max_len) {
    if (B < 0 || D <= 0 || H <= 0 || max_len < 1 || bad_dims(B, D) || bad_dims(B, H) || bad_dims(max_len, D))
        return -1;
    return decode_ws(B, D, H, max_len).total;
}

int sgq_rms_norm(const float* x, int64_t rows, int64_t D, const float* g, float eps, float* out, void* stream) {
    if (bad_dims(rows, D)) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_rms_norm: bad shape");
    if (rows == 0 || D == 0) return ok();
    if (!x || !g || !out) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_rms_norm: null pointer");
    SGQ_HIP(launch_rms_norm(x, rows, D, g, eps, out, (hipStream_t)stream), "rms_norm");
    return ok();
}

int sgq_embedding(const float* indices, int64_t n, const float* weight, int64_t num_embeddings,
                  int64_t embedding_dim, float* out, void* stream) {
    if (n < 0 || bad_dims(num_embeddings, embedding_dim) || bad_dims(n, embedding_dim) || n > 0x7fffffff)
        return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_embedding: bad shape");
    if (n == 0 || embedding_dim == 0) return ok();
    if (!indices || !weight || !out) return fail(SGQ_ERR_INVALID_ARGUMENT, "sgq_embedding: null pointer");
    SGQ_HIP(launch_embedding(indices, n, weight, num_embeddings, embedding_dim, out, (hipStream_t)stream),
            "embedding");
    return ok();
}

int sgq_llama_block_decode_int4(const sgq_llama_block_int4* blk, const float* x, float* out, int64_t B,
                                float* k_cache, float* v_cache, int64_t max_tokens, const int32_t* pos,
                                int64_t max_len, void* workspace, int64_t workspace_bytes, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    const char* fn = "sgq_llama_block_decode_int4";
    if (!blk) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null block", fn);
    const int64_t D = blk->D, H = blk->H, G = blk->group_size;
    if (B < 0 || D <= 0 || H <= 0 || bad_dims(B, D) || bad_dims(B, H) || bad_dims(D, H))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: bad shape", fn);
    if (max_tokens < 1 || max_len < 1 || max_len > max_tokens || bad_dims(max_tokens, D))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: need 1 <= max_len <= max_tokens", fn);
    if (D > 8192) return fail(SGQ_ERR_UNSUPPORTED, "%s: D > 8192", fn);
    if (max_len > attn_max_len())
        return fail(SGQ_ERR_UNSUPPORTED, "%s: max_len > %lld", fn, (long long)attn_max_len());
    const I4Geom gdd(D, D, G), gdh(D, H, G), ghd(H, D, G);
    if (!gdd.tiled || !gdh.tiled || !ghd.tiled)
        return fail(SGQ_ERR_UNSUPPORTED, "%s: D, H and group_size must be multiples of 8 (tiled INT4 layout)", fn);
    if (H > kGemmMaxK)  // the down projection's K, within both forward kernels' 32-bit offsets
        return fail(SGQ_ERR_UNSUPPORTED, "%s: H > %lld", fn, (long long)kGemmMaxK);
    const sgq_int4_linear* lin[7] = {&blk->q, &blk->k, &blk->v, &blk->o, &blk->gate, &blk->up, &blk->down};
    for (int i = 0; i < 7; ++i) {
        if (!lin[i]->packed || !lin[i]->devscales) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null weight", fn);
        if (!aligned16(lin[i]->packed) || !aligned16(lin[i]->devscales))
            return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: packed and devscales must be 16-byte aligned", fn);
    }
    if (!blk->norm1 || !blk->norm2) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null norm weight", fn);
    if (B == 0) return ok();
    if (!x || !out || !k_cache || !v_cache || !pos) return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (!aligned16(k_cache) || !aligned16(v_cache))
        return fail(SGQ_ERR_INVALID_ARGUMENT, "%s: caches must be 16-byte aligned", fn);
    const DecodeWs w = decode_ws(B, D, H, max_len);
    if (!workspace || workspace_bytes < w.total || !aligned16(workspace))
        return fail(SGQ_ERR_WORKSPACE, "%s: workspace needs %lld bytes, 16-byte aligned", fn, (long long)w.total);
    char* base = (char*)workspace;
    float* n = (float*)(base + w.n);
    float* qkv = (float*)(base + w.qkv);
    float* ctx = (float*)(base + w.ctx);
    float* h = (float*)(base + w.h);
    float* hid = (float*)(base + w.hid);
    float* tmp = (float*)(base + w.tmp);
    float* part = (float*)(base + w.part);
    void* split = base + w.split;

    // attn->forward(norm1->forward(x)), then the residual: h = x + o(ctx).
    // The GEMV path applies each RMSNorm inside the projection that reads it.
    const bool gemv = decode_uses_gemv(B, D, H);
    const int cus = gemv ? device_cus(s) : 0;
    if (gemv) {
        const void* pk[3] = {blk->q.packed, blk->k.packed, blk->v.packed};
        const float* ds[3] = {blk->q.devscales, blk->k.devscales, blk->v.devscales};
        const float* bs[3] = {blk->q.bias, blk->k.bias, blk->v.bias};
        const SkinnyPlan sq = decode_skinny_plan(B, D, D, 3, G, cus);
        if (sq.C > 0) {
            SkinnyExtra ex;
            ex.nw = 3;
            ex.ldy = 3 * D;
            ex.gamma = blk->norm1;
            ex.eps = blk->eps;
            SGQ_HIP(launch_skinny_i4(x, B, D, D, 1, pk, ds, bs, gdd, sq, qkv, nullptr, s, &ex), "skinny_qkv");
        } else {
            SGQ_HIP(launch_gemv_i4_multi(x, B, D, D, 3, pk, ds, bs, gdd, qkv, 3 * D, nullptr, blk->norm1, blk->eps,
                                         s),
                    "gemv_qkv");
        }
        SGQ_HIP(launch_attention_decode(qkv, qkv + D, qkv + 2 * D, 3 * D, B, D, k_cache, v_cache, max_tokens, pos,
                                        max_len, blk->attn_scale, part, ctx, s),
                "attention");
        SGQ_HIP(launch_gemv_i4_multi(ctx, B, D, D, 1, &blk->o.packed, &blk->o.devscales, &blk->o.bias, gdd, h, D, x,
                                     nullptr, 0.0f, s),
                "gemv_o");
    } else {
        SGQ_HIP(launch_rms_norm(x, B, D, blk->norm1, blk->eps, n, s), "rms_norm");
        float* qb = qkv;
        float* kb = qkv + B * D;
        float* vb = qkv + 2 * B * D;
        SGQ_HIP(launch_gemm_i4(n, B, D, D, blk->q.packed, blk->q.devscales, gdd, blk->q.bias, qb, split, s), "gemm_q");
        SGQ_HIP(launch_gemm_i4(n, B, D, D, blk->k.packed, blk->k.devscales, gdd, blk->k.bias, kb, split, s), "gemm_k");
        SGQ_HIP(launch_gemm_i4(n, B, D, D, blk->v.packed, blk->v.devscales, gdd, blk->v.bias, vb, split, s), "gemm_v");
        SGQ_HIP(launch_attention_decode(qb, kb, vb, D, B, D, k_cache, v_cache, max_tokens, pos, max_len,
                                        blk->attn_scale, part, ctx, s),
                "attention");
        SGQ_HIP(launch_gemm_i4(ctx, B, D, D, blk->o.packed, blk->o.devscales, gdd, blk->o.bias, tmp, split, s),
                "gemm_o");
        SGQ_HIP(launch_add(x, tmp, h, B * D, s), "add");
    }
    // h + mlp->forward(norm2->forward(h))
    if (gemv) {
        const SkinnyPlan sg = decode_skinny_plan(B, D, H, 1, G, cus);
        if (sg.C > 0) {
            const void* pk[2] = {blk->gate.packed, blk->up.packed};
            const float* ds[2] = {blk->gate.devscales, blk->up.devscales};
            const float* bs[2] = {blk->gate.bias, blk->up.bias};
            SkinnyExtra ex;
            ex.gamma = blk->norm2;
            ex.eps = blk->eps;
            SGQ_HIP(launch_skinny_i4(h, B, D, H, 2, pk, ds, bs, gdh, sg, hid, nullptr, s, &ex), "skinny_gate_up");
        } else {
            SGQ_HIP(launch_swiglu_gemv_i4(h, B, D, H, blk->gate.packed, blk->gate.devscales, blk->gate.bias,
                                          blk->up.packed, blk->up.devscales, blk->up.bias, gdh, hid, s, blk->norm2,
                                          blk->eps),
                    "swiglu_gemv");
        }
        SGQ_HIP(launch_gemv_i4_multi(hid, B, H, D, 1, &blk->down.packed, &blk->down.devscales, &blk->down.bias, ghd,
                                     out, D, h, nullptr, 0.0f, s),
                "gemv_down");
    } else {
        SGQ_HIP(launch_rms_norm(h, B, D, blk->norm2, blk->eps, n, s), "rms_norm");
        SGQ_HIP(launch_gemm_i4(n, B, D, H, blk->gate.packed, blk->gate.devscales, gdh, blk->gate.bias, hid, split, s),
                "gemm_gate");
        SGQ_HIP(launch_gemm_i4(n, B, D, H, blk->up.packed, blk->up.devscales, gdh, blk->up.bias, tmp, split, s),
                "gemm_up");
        SGQ_HIP(launch_silu_mul(hid, tmp, B * H, s), "silu_mul");
        SGQ_HIP(launch_gemm_i4(hid, B, H, D, blk->down.packed, blk->down.devscales, ghd, blk->down.bias, tmp, split,
                               s),
                "gemm_down");
        SGQ_HIP(launch_add(h, tmp, out, B * D, s), "add");
    }
    return ok();
}

}  // extern "C"
