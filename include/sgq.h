/*
 * sgq.h -- C ABI of the MI355X (gfx950) quantized-linear library, libsgq.so.
 *
 * This is the drop-in boundary for SovereignGrad's quantized inference path.
 * Each entry point replaces one piece of the reference (paths relative to the
 * reference checkout); the reference has no GPU code for this path, so these
 * replace its host functions, called with device pointers.
 *
 * Conventions (shared by every function below):
 *   - Plain pointers and sizes.  Every pointer argument is DEVICE memory
 *     (hipMalloc'd or equivalent) unless stated otherwise.  The library never
 *     allocates or frees; callers own every buffer, including workspaces.
 *   - `stream` is a hipStream_t passed as void*; NULL means the default
 *     stream.  Calls are asynchronous on that stream unless stated otherwise.
 *   - Return value: SGQ_OK (0) or an SGQ_ERR_* code.  sgq_last_error() gives
 *     a message for the calling thread's most recent failure.  Argument errors
 *     are detected before anything is launched.
 *   - Reentrant: no mutable global state; safe to call concurrently from
 *     several host threads as long as each concurrent call has its own
 *     workspace.
 *   - Alignment: packed buffers, devscales and per-channel INT8 scales must be
 *     16-byte aligned (hipMalloc gives 256); x may have any 4-byte alignment.
 *
 * Weight shape convention: W is [K, N] row-major ([in_features,
 * out_features], include/sovereigngrad/nn.hpp:938) and the forward is
 * y[M,N] = x[M,K] . dequant(W) (+ bias[1,N]) (src/quantization.cpp:189-206).
 *
 * Device layouts ("packed" buffers) are this library's own; they are built by
 * sgq_quantize_* or sgq_pack_* and read back with sgq_unpack_* /
 * sgq_dequantize_*.  The reference-layout tensors (fp32 codes `qdata` [K,N],
 * fp32 `scales`) are bit-identical to what the reference produces.
 */
#ifndef SGQ_H
#define SGQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define SGQ_OK 0
#define SGQ_ERR_INVALID_ARGUMENT 1 /* null pointer, negative size, bad scheme   */
#define SGQ_ERR_UNSUPPORTED 2      /* shape/layout combination not supported   */
#define SGQ_ERR_WORKSPACE 3        /* workspace missing or too small           */
#define SGQ_ERR_HIP 4              /* a HIP runtime call failed                */
#define SGQ_ERR_CODES 5            /* codes not integral / out of range (pack) */

/* ---- quantization schemes (include/sovereigngrad/quantization.hpp:11-15) */
#define SGQ_PER_TENSOR_SYMMETRIC 0
#define SGQ_PER_CHANNEL_SYMMETRIC 1
#define SGQ_GROUPED_ASYMMETRIC 2

/* ---- INT4 device layouts ----------------------------------------------- */
#define SGQ_LAYOUT_INT4_TILED 0 /* N % 8 == 0 and group % 8 == 0: fast kernels */
#define SGQ_LAYOUT_INT4_FLAT 1  /* any shape: flat nibble stream, generic kernels */

/* Message for the calling thread's last failed call ("" if none). */
const char* sgq_last_error(void);

/* Library ABI version (SGQ_ABI_VERSION).  2: packed INT4 buffers of the
 * strip-major layout hold a second, k-octet copy of the codes (one byte per
 * code in all); buffers packed by version 1 must be packed again. */
int sgq_abi_version(void);

/* ---- size queries (host-only; no GPU work) ----------------------------- */

/* Bytes of the packed INT8 buffer for a [K,N] weight. */
int64_t sgq_int8_packed_bytes(int64_t K, int64_t N);

/* INT4 layout chosen for a [K,N] weight with this group size
 * (group_size <= 0 means 32, as src/quantization.cpp:118). */
int sgq_int4_layout(int64_t K, int64_t N, int64_t group_size);

/* Bytes of the packed INT4 buffer for a [K,N] weight.  The strip-major
 * layout (sgq_int4_layout() == 0) holds the codes twice, in the strips the
 * GEMV reads and in blocks whose dwords are matrix-core operands (read by
 * the 3..32-row and GEMM forms), about one byte per code; the flat layout
 * half a byte per code. */
int64_t sgq_int4_packed_bytes(int64_t K, int64_t N, int64_t group_size);

/* Number of floats in the INT4 device-scale buffer (0 for the flat layout,
 * which reads the reference-layout scales directly). */
int64_t sgq_int4_devscale_count(int64_t K, int64_t N, int64_t group_size);

/* Number of reference-layout scales: 1 (per-tensor), rows (per-channel),
 * ceil(rows*cols/group) (INT4), following src/quantization.cpp:22,44-48,119. */
int64_t sgq_int8_scale_count(int64_t rows, int64_t cols, int scheme);
int64_t sgq_int4_scale_count(int64_t rows, int64_t cols, int64_t group_size);

/* Workspace bytes needed by sgq_quantize_int8 / sgq_quantize_int4 / sgq_pack_*. */
int64_t sgq_quantize_workspace_bytes(int bits, int64_t rows, int64_t cols, int64_t group_size);

/* Workspace bytes needed by sgq_linear_int8 / sgq_linear_int4 for batch M.
 * Nonzero when a kernel splits K over workgroups, whose partial outputs (KS *
 * M * N floats) are summed by a second kernel in fixed order: the GEMM (M >
 * 16, except batches of up to 128 rows with M * K * N <= 2^28, which run the
 * GEMV) when its grid of output tiles (32 or 64 rows by 128 columns for
 * batches of up to 32 or 64 rows; else 128 rows by 256 columns for INT8, 128
 * for INT4) is smaller than the GPU, and for INT4 the skinny MFMA kernel over
 * weights too narrow to fill the GPU (M >= 5 with (M rounded up to 8) * K * N
 * >= 2^28) or, with 17..32 rows, over a K longer than 8192 rows (the INT8
 * skinny kernel never splits K).  The size is the largest any
 * group size and device could need.  0 otherwise (the GEMV and the other
 * kernels own whole outputs per workgroup), and the workspace arguments may
 * then be NULL/0.  The contents need no initialisation and are overwritten by
 * each call; calls that overlap in time must not share one workspace.
 * 16-byte alignment required. */
int64_t sgq_linear_workspace_bytes(int bits, int64_t M, int64_t K, int64_t N);

/* The kernel a forward of this shape runs and its K splits, on a device
 * with `compute_units` CUs (0: the calling thread's current device; a full
 * MI355X has 256, a partition fewer).  *path: 0 the GEMV, 1 the three-term
 * bf16 MFMA GEMM, 2 the fp32 MFMA GEMM (INT4 groups that are not a multiple
 * of 128), 3 the generic kernel of the flat INT4 layout, 4 the skinny bf16
 * MFMA kernels (INT4: 5..32 rows over a weight wide enough to fill the
 * device with workgroups of 32 or 64 columns, and 5..32 rows over narrower
 * weights with (M rounded up to 8) * K * N >= 2^28, K split; INT8: 5..128
 * rows with (M rounded up to 8) * K * N >= 2^26, above 16 rows only while
 * M * K * N <= 2^29, whole K).  *k_splits: 1, or the number of
 * workgroups sharing each output tile's K range (the GEMM on grids smaller
 * than the device, the skinny kernel's K ranges).  sgq_linear_workspace_bytes sizes for the
 * largest device, so it covers every plan.  Host-only; this library's own
 * extension (the reference has no launch planning). */
int sgq_linear_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int compute_units, int* path,
                    int* k_splits);

/* How the MFMA GEMM of this shape places its workgroups on a device of
 * `compute_units` CUs (0: the current device's) and `xcds` XCDs (0: the
 * current device's, hipDeviceAttributeNumberOfXccs; a full MI355X has 8, its
 * compute partitions 4, 2 or 1).  *rect_rows: tile rows of the output
 * rectangle each XCD takes when the grid splits into one rectangle per XCD
 * without a K split (0: the plain order); *xcd_log2: log2 of the XCD count
 * the kernels permute workgroup ids by (0, the identity, for a count that is
 * not a power of two).  Host-only; this library's own extension (the
 * reference has no launch planning).  Placement changes speed only, never a
 * result. */
int sgq_gemm_xcd_plan(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size, int compute_units, int xcds,
                      int* rect_rows, int* xcd_log2);

/* Zero-fills a workspace with a kernel (no hipMemset), on `stream`. */
int sgq_workspace_init(void* workspace, int64_t workspace_bytes, void* stream);

/* ---- quantize (construction path) ------------------------------------- */

/* Replaces quantization::quantize_int8 (src/quantization.cpp:11-78) for a
 * device tensor viewed as [rows, cols].  scheme SGQ_PER_TENSOR_SYMMETRIC or
 * SGQ_PER_CHANNEL_SYMMETRIC; per-channel means one scale per row, like the
 * reference.  (The reference also takes the per-tensor branch for rank<2
 * tensors; callers pass scheme 0 for those.)
 *   qdata_f32  optional [rows*cols] fp32 codes in reference layout, bit-exact
 *              (including -0.0 codes).
 *   scales     required, sgq_int8_scale_count() floats, bit-exact.
 *   packed     optional, sgq_int8_packed_bytes(rows, cols) bytes (K=rows, N=cols).
 */
int sgq_quantize_int8(const float* x, int64_t rows, int64_t cols, int scheme, float* qdata_f32,
                      float* scales, void* packed, void* workspace, int64_t workspace_bytes, void* stream);

/* Replaces quantization::quantize_int4 (src/quantization.cpp:113-159): groups
 * of group_size consecutive elements of the flattened tensor (group_size <= 0
 * means 32).  The packed layout treats the tensor as [rows, cols].
 *   qdata_f32  optional [rows*cols] fp32 codes, bit-exact.
 *   scales     required, sgq_int4_scale_count() floats, bit-exact.
 *   packed     optional, sgq_int4_packed_bytes() bytes.
 *   devscales  required when packed is given and the layout is TILED
 *              (sgq_int4_devscale_count() floats), else ignored.
 */
int sgq_quantize_int4(const float* x, int64_t rows, int64_t cols, int64_t group_size, float* qdata_f32,
                      float* scales, void* packed, float* devscales, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* ---- repack / unpack (persistence bridge) ------------------------------ */

/* Packs reference-layout fp32 codes (as stored in a QuantizedTensor's qdata,
 * or loaded by load_state_dict, src/module.cpp:114-134) into the device layout.
 * Returns SGQ_ERR_CODES (after synchronising `stream`) when a code is not an
 * integer in [-128,127] (INT8) or [-8,7] (INT4). */
int sgq_pack_int8(const float* qdata_f32, int64_t K, int64_t N, void* packed, void* workspace,
                  int64_t workspace_bytes, void* stream);
int sgq_pack_int4(const float* qdata_f32, const float* scales, int64_t K, int64_t N, int64_t group_size,
                  void* packed, float* devscales, void* workspace, int64_t workspace_bytes, void* stream);

/* Writes the fp32 codes [K,N] in reference layout from a packed buffer (codes
 * that were -0.0 come back as +0.0; every other code is exact). */
int sgq_unpack_int8(const void* packed, int64_t K, int64_t N, float* qdata_f32, void* stream);
int sgq_unpack_int4(const void* packed, int64_t K, int64_t N, int64_t group_size, float* qdata_f32,
                    void* stream);

/* ---- dequantize ------------------------------------------------------- */

/* Replaces quantization::dequantize_int8 (src/quantization.cpp:80-111):
 * out[k,n] = code * scale with one IEEE multiply, scale = scales[0] for
 * per-tensor, scales[k] for per-channel. */
int sgq_dequantize_int8(const void* packed, const float* scales, int scheme, int64_t K, int64_t N, float* out,
                        void* stream);

/* Replaces quantization::dequantize_int4 (src/quantization.cpp:161-187):
 * out[i] = code[i] * scales[i / group_size] over the flattened [K,N]. */
int sgq_dequantize_int4(const void* packed, const float* scales, int64_t K, int64_t N, int64_t group_size,
                        float* out, void* stream);

/* Replaces dequantize_int8 / dequantize_int4 bit for bit from the
 * reference-layout fp32 codes (qdata [rows*cols]): out[i] = qdata[i] * s(i),
 * one IEEE multiply, with s(i) = scales[0] (bits 8, per-tensor),
 * scales[i / cols] (bits 8, per-channel) or scales[i / group_size] (bits 4;
 * group_size <= 0 means 32), following src/quantization.cpp:90-107,173-184. */
int sgq_dequantize_codes(const float* qdata_f32, const float* scales, int bits, int scheme, int64_t rows,
                         int64_t cols, int64_t group_size, float* out, void* stream);

/* ---- forward ---------------------------------------------------------- */

/* Replaces quantization::quantized_matmul_int8 (src/quantization.cpp:189-197)
 * and with it nn::QuantizedLinear::forward (include/sovereigngrad/nn.hpp:956-958):
 *   y[M,N] = x[M,K] . (codes * scales) (+ bias[N])   fp32 accumulate.
 * scales are the reference-layout scales (1 or K floats).  bias may be NULL.
 * Dispatch (sgq_linear_plan): 5..128 rows with (M rounded up to 8) * K * N
 * >= 2^26 (above 16 rows only while M * K * N <= 2^29) run the skinny bf16
 * MFMA kernel (whole K per workgroup, no workspace); other batches of up to
 * 16 rows, and up to 128 rows with M * K * N <= 2^28, the wavefront GEMV (row
 * groups of 8); larger batches the LDS-staged MFMA GEMM.  Both MFMA kernels
 * run the fp32 products on the bf16 matrix cores as three exact bf16
 * products each (fp32 accumulation; as accurate as an fp32 product).
 * workspace: sgq_linear_workspace_bytes(8, M, K, N) bytes, else
 * SGQ_ERR_WORKSPACE. */
int sgq_linear_int8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                    int scheme, const float* bias, float* y, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Replaces quantization::quantized_matmul_int4 (src/quantization.cpp:199-206)
 * and nn::QuantizedLinear4Bit::forward (include/sovereigngrad/nn.hpp:994-996).
 * scales: the reference-layout scales (used by the FLAT layout); devscales:
 * the device scales written by sgq_quantize_int4/sgq_pack_int4 (TILED layout).
 * Dispatch (sgq_linear_plan): the INT4 skinny bf16 MFMA kernel for the
 * batches of 5..32 rows it takes, else the GEMV for up to 16 rows (and up to
 * 128 rows with M * K * N <= 2^28), else the GEMM.  workspace:
 * sgq_linear_workspace_bytes(4, M, K, N) bytes, else SGQ_ERR_WORKSPACE. */
int sgq_linear_int4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                    const float* devscales, int64_t group_size, const float* bias, float* y, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* sgq_linear_int4 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * allocates nothing: the split-K partials (of the GEMM or the skinny kernel) go to a static device
 * array of 32 MiB per GPU (created when the library is loaded on that GPU
 * and held until the process ends).  Shapes whose sgq_linear_workspace_bytes
 * exceeds 32 MiB are refused with SGQ_ERR_UNSUPPORTED.  The stream must
 * belong to the calling thread's current device.  Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (two
 * streams, two threads) race and must be serialised by the caller; calls in
 * order on one stream are safe.  Same results as sgq_linear_int4 (the same
 * kernels and plan). */
int sgq_linear_int4_noalloc(const float* x, int64_t M, int64_t K, int64_t N, const void* packed, const float* scales,
                            const float* devscales, int64_t group_size, const float* bias, float* y, void* stream);

/* ---- gated MLP (caller-side fusion) ----------------------------------- */

/* Replaces the first three lines of nn::SwiGLU::forward
 * (include/sovereigngrad/nn.hpp:151-154) with quantized gate and up
 * projections:
 *   h[M,N] = silu(x . Wg + bias_gate) * (x . Wu + bias_up)
 * silu(v) = v / (1 + exp(-v)) as Tensor::silu (src/ops.cpp:561-575,
 * include/sovereigngrad/simd.hpp:103-108), * as mul (src/ops.cpp:239-253).
 * The two weights share K, N, scheme / group_size.  The batches the forward
 * runs on the GEMV or on the INT4 skinny MFMA kernel (above), with the tiled
 * layout, run both weights in one launch (x read once per strip pair, no
 * intermediate in HBM; a split K adds its reduce kernel); otherwise two
 * projections (the INT8 skinny kernel, the GEMM or flat INT4) and an
 * elementwise kernel, so that the sums are those of two forward calls.
 * Biases may be NULL.  workspace:
 * sgq_swiglu_workspace_bytes(bits, M, K, N, group_size) bytes (group_size is
 * ignored for bits 8), else SGQ_ERR_WORKSPACE. */
int64_t sgq_swiglu_workspace_bytes(int bits, int64_t M, int64_t K, int64_t N, int64_t group_size);
int sgq_swiglu_int8(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_gate,
                    const float* scales_gate, const float* bias_gate, const void* packed_up, const float* scales_up,
                    const float* bias_up, int scheme, float* h, void* workspace, int64_t workspace_bytes,
                    void* stream);
int sgq_swiglu_int4(const float* x, int64_t M, int64_t K, int64_t N, const void* packed_gate,
                    const float* scales_gate, const float* devscales_gate, const float* bias_gate,
                    const void* packed_up, const float* scales_up, const float* devscales_up, const float* bias_up,
                    int64_t group_size, float* h, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- quantized LLaMA block, one decode step ---------------------------- */

/* One INT4 projection in the tiled layout (written by sgq_quantize_int4 /
 * sgq_pack_int4), with its bias row (NULL: no bias add). */
typedef struct sgq_int4_linear {
    const void* packed;
    const float* devscales;
    const float* bias;
} sgq_int4_linear;

/* LLaMABlock (include/sovereigngrad/models.hpp:197-224) with every nn::Linear
 * a QuantizedLinear4Bit (nn.hpp:965-1001) of one group size:
 *   q, k, v, o: [D, D] (CausalSelfAttention, nn.hpp:503-553)
 *   gate, up: [D, H]; down: [H, D] (SwiGLU, nn.hpp:135-156)
 *   norm1, norm2: the RMSNorm weights [D] (nn.hpp:67-85), eps their epsilon
 *   attn_scale: CausalSelfAttention::scale, 1 / sqrt((float)(D / num_heads))
 *     (nn.hpp:518); the reference attends over the full width D.
 * D and H must be multiples of 8 and group_size a multiple of 8 (the tiled
 * layout), D <= 8192. */
typedef struct sgq_llama_block_int4 {
    int64_t D, H, group_size;
    float eps, attn_scale;
    const float* norm1;
    const float* norm2;
    sgq_int4_linear q, k, v, o, gate, up, down;
} sgq_llama_block_int4;

/* Workspace bytes of sgq_llama_block_decode_int4 for B sequences, widths D
 * and H, and at most max_len keys per sequence in the step. */
int64_t sgq_llama_decode_workspace_bytes(int64_t B, int64_t D, int64_t H, int64_t max_len);

/* One decode step of the block for B sequences, one new token each.
 * Replaces LLaMABlock::forward (models.hpp:217-222) on the last row of each
 * sequence: the reference reruns the whole sequence (NanoLLaMA::generate,
 * models.hpp:270-302); here the keys and values of earlier positions are kept
 * in a cache, so the step computes
 *   h   = x + o(attention(q(n1), K, V)),          n1 = rms_norm(x, norm1)
 *   out = h + down(silu(gate(n2)) * up(n2)),       n2 = rms_norm(h, norm2)
 * where attention is CausalSelfAttention's last row (nn.hpp:545-552): softmax
 * over positions 0..pos[b] of (q . k_j) * attn_scale, applied to v_j.
 *   x, out:    [B, D]; out may be x (in-place update of the hidden state).
 *   k_cache, v_cache: [B][max_tokens][D] fp32, 16-byte aligned; rows 0..pos[b]-1
 *              hold the keys/values of earlier positions.  The step writes
 *              row pos[b] (this token's key and value).
 *   pos:       [B] int32 on the device: tokens already cached per sequence.
 *              The caller advances it after the step (every layer of one step
 *              uses the same positions).
 *   max_len:   host bound on pos[b] + 1 for this step (sizes the launch),
 *              1 <= max_len <= max_tokens.  A sequence whose pos[b] is
 *              negative or >= min(max_len, max_tokens) gets a NaN output row
 *              and no cache write.
 *   workspace: sgq_llama_decode_workspace_bytes(B, D, H, max_len) bytes,
 *              16-byte aligned.
 * Batches the forward runs on the GEMV (B <= 16, or up to 128 when every
 * projection's B * K * N <= 2^28) run every projection on it (q, k, v in one
 * launch; the RMSNorms folded in; the residual adds in the epilogues), except
 * that 5..16 rows run the norm-fused q/k/v and gate/up launches on the skinny
 * bf16 MFMA kernel where its plan takes the projection's total width (e.g.
 * the NanoLLaMA shape); larger B on the MFMA GEMM.  fp32 results throughout;
 * outputs match the reference's full-sequence forward within 1e-5 relative. */
int sgq_llama_block_decode_int4(const sgq_llama_block_int4* block, const float* x, float* out, int64_t B,
                                float* k_cache, float* v_cache, int64_t max_tokens, const int32_t* pos,
                                int64_t max_len, void* workspace, int64_t workspace_bytes, void* stream);

/* Replaces embedding (src/ops.cpp:2624-2650): out[i, :] = weight[(int)indices[i], :]
 * for the n fp32 token ids in `indices` (truncated to int, as the reference
 * reads them), a zero row for an id outside [0, num_embeddings). */
int sgq_embedding(const float* indices, int64_t n, const float* weight, int64_t num_embeddings,
                  int64_t embedding_dim, float* out, void* stream);

/* Replaces rms_norm (src/ops.cpp:1532-1556) for rows of [rows, D]:
 * out = x * (1 / sqrt(sum(x^2) / D + eps)) * g.  out may be x. */
int sgq_rms_norm(const float* x, int64_t rows, int64_t D, const float* g, float eps, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SGQ_H */
