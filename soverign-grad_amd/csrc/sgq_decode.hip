// sgq_decode.hip -- the non-projection kernels of one LLaMA block decode step:
// RMSNorm, attention of one new token per sequence over its key/value cache,
// and residual adds.  The projections are the quantized GEMV/GEMM kernels of
// sgq_linear.hip.
//
// Reference: LLaMABlock::forward (include/sovereigngrad/models.hpp:217-222)
// with CausalSelfAttention::forward (include/sovereigngrad/nn.hpp:533-553) and
// rms_norm (src/ops.cpp:1532-1556).  The reference recomputes attention over
// the whole sequence each step; here the keys and values of earlier positions
// stay in a cache, so a step reads them once and computes only the new row,
// which is the last row of the reference's causal attention.
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over the workgroup's kBlock threads; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) t += red[w];
    return t;
}

// out[i, :] = x[i, :] * inv_rms * g, inv_rms = 1 / sqrt(sum(x^2) / D + eps)
// (rms_norm, src/ops.cpp:1532-1556).  One workgroup per row.
__global__ __launch_bounds__(kBlock) void k_rms_norm(const float* __restrict__ x, int64_t D,
                                                     const float* __restrict__ g, float eps,
                                                     float* __restrict__ out) {
    __shared__ float red[kBlock / 64];
    const float* xr = x + (int64_t)blockIdx.x * D;
    float* orow = out + (int64_t)blockIdx.x * D;
    float ss = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += kBlock) ss = fmaf(xr[d], xr[d], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    for (int64_t d = threadIdx.x; d < D; d += kBlock) orow[d] = (xr[d] * inv) * g[d];
}

// y[i] = a[i] + b[i]: the block's residual connections (equal-shape add,
// src/ops.cpp:142-148).
__global__ __launch_bounds__(kBlock) void k_add(const float* __restrict__ a, const float* __restrict__ b,
                                                float* __restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        y[i] = a[i] + b[i];
}

// Sequence b's keys this step: positions 0 .. pos[b] (pos[b] were cached
// before, the new one is pos[b]).  Invalid when pos[b] is negative or does
// not fit the cache or the caller's bound.
__device__ __forceinline__ int seq_keys(const int32_t* pos, int b, int64_t max_tokens, int64_t max_len) {
    const int p = pos[b];
    return (p < 0 || p >= max_tokens || p >= max_len) ? -1 : p + 1;
}

// One workgroup per (chunk c of CS keys, sequence b):
//   s_j = (q . k_j) * scale           for the chunk's keys j
//   m_c = max s_j, l_c = sum exp(s_j - m_c), o_c = sum exp(s_j - m_c) v_j
// k_j, v_j come from the cache for j < pos[b] and from the new row for
// j == pos[b]; the workgroup whose chunk holds pos[b] also stores the new row
// into the cache.  With a single chunk (direct) the workgroup writes
// ctx = o_c / l_c; otherwise (o_c, m_c, l_c) go to part[b][c] for
// k_attn_combine.  D % 4 == 0; rows 16-byte aligned.
__global__ __launch_bounds__(kBlock) void k_attn_partial(const float* __restrict__ q, const float* __restrict__ knew,
                                                         const float* __restrict__ vnew, int64_t ldq, int64_t D,
                                                         float* __restrict__ kc, float* __restrict__ vc,
                                                         int64_t max_tokens, const int32_t* __restrict__ pos,
                                                         int64_t max_len, int CS, float scale,
                                                         float* __restrict__ part, float* __restrict__ ctx) {
    extern __shared__ float smem[];  // q row (D floats), then CS scores
    float* qs = smem;
    float* sc = smem + D;
    const int b = blockIdx.y, c = blockIdx.x, nc = gridDim.x;
    const int T = seq_keys(pos, b, max_tokens, max_len);
    const int j0 = c * CS;
    if (T < 0 || j0 >= T) return;  // combine reads only chunks below ceil(T / CS)
    const int j1 = min(j0 + CS, T);
    const int p = T - 1;  // the new position
    const float* qrow = q + (int64_t)b * ldq;
    const float* kn = knew + (int64_t)b * ldq;
    const float* vn = vnew + (int64_t)b * ldq;
    float* kcb = kc + (int64_t)b * max_tokens * D;
    float* vcb = vc + (int64_t)b * max_tokens * D;
    const int64_t D4 = D / 4;

    for (int64_t i = threadIdx.x; i < D4; i += kBlock) ((float4*)qs)[i] = ((const float4*)qrow)[i];
    if (p >= j0 && p < j1) {  // this chunk holds the new position: append it to the cache
        for (int64_t i = threadIdx.x; i < D4; i += kBlock) {
            ((float4*)(kcb + (int64_t)p * D))[i] = ((const float4*)kn)[i];
            ((float4*)(vcb + (int64_t)p * D))[i] = ((const float4*)vn)[i];
        }
    }
    __syncthreads();

    // Scores: one wavefront per key.
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int j = j0 + wave; j < j1; j += kBlock / 64) {
        const float* kr = (j == p) ? kn : kcb + (int64_t)j * D;
        float acc = 0.0f;
        for (int64_t i = lane; i < D4; i += 64) {
            const float4 kv = ((const float4*)kr)[i];
            const float4 qv = ((const float4*)qs)[i];
            acc = fmaf(qv.x, kv.x, acc);
            acc = fmaf(qv.y, kv.y, acc);
            acc = fmaf(qv.z, kv.z, acc);
            acc = fmaf(qv.w, kv.w, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) sc[j - j0] = acc * scale;
    }
    __syncthreads();

    const int n = j1 - j0;
    float m = -INFINITY;
    for (int t = 0; t < n; ++t) m = fmaxf(m, sc[t]);
    __syncthreads();
    for (int t = threadIdx.x; t < n; t += kBlock) sc[t] = expf(sc[t] - m);
    __syncthreads();
    float l = 0.0f;
    for (int t = 0; t < n; ++t) l += sc[t];

    // o_c[d] = sum_j e_j v_j[d], four dims per thread per step.
    const bool direct = nc == 1;
    float* dst = direct ? ctx + (int64_t)b * D : part + ((int64_t)b * nc + c) * (D + 4);
    const float inv_l = 1.0f / l;
    for (int64_t i = threadIdx.x; i < D4; i += kBlock) {
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int t = 0; t < n; ++t) {
            const int j = j0 + t;
            const float4 vv = ((const float4*)((j == p) ? vn : vcb + (int64_t)j * D))[i];
            const float e = sc[t];
            o.x = fmaf(e, vv.x, o.x);
            o.y = fmaf(e, vv.y, o.y);
            o.z = fmaf(e, vv.z, o.z);
            o.w = fmaf(e, vv.w, o.w);
        }
        if (direct) {
            o.x = o.x * inv_l;
            o.y = o.y * inv_l;
            o.z = o.z * inv_l;
            o.w = o.w * inv_l;
        }
        ((float4*)dst)[i] = o;
    }
    if (!direct && threadIdx.x == 0) {
        dst[D] = m;
        dst[D + 1] = l;
    }
}

// ctx[b] = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M) over the chunks
// that hold keys (M = max_c m_c).  Grid (ceil(D / (4 * kBlock)), B).  A
// sequence with an invalid position gets a NaN row.
__global__ __launch_bounds__(kBlock) void k_attn_combine(const float* __restrict__ part, int nc, int CS, int64_t D,
                                                         const int32_t* __restrict__ pos, int64_t max_tokens,
                                                         int64_t max_len, float* __restrict__ ctx) {
    const int b = blockIdx.y;
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;  // float4 index
    if (i * 4 >= D) return;
    float4* out = (float4*)(ctx + (int64_t)b * D) + i;
    const int T = seq_keys(pos, b, max_tokens, max_len);
    if (T < 0) {
        *out = make_float4(NAN, NAN, NAN, NAN);
        return;
    }
    const int used = (T + CS - 1) / CS;
    const float* pb = part + (int64_t)b * nc * (D + 4);
    float M = -INFINITY;
    for (int c = 0; c < used; ++c) M = fmaxf(M, pb[(int64_t)c * (D + 4) + D]);
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c = 0; c < used; ++c) {
        const float* pc = pb + (int64_t)c * (D + 4);
        const float w = expf(pc[D] - M);
        L = fmaf(pc[D + 1], w, L);
        const float4 v = ((const float4*)pc)[i];
        o.x = fmaf(v.x, w, o.x);
        o.y = fmaf(v.y, w, o.y);
        o.z = fmaf(v.z, w, o.z);
        o.w = fmaf(v.w, w, o.w);
    }
    const float inv = 1.0f / L;
    *out = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// Poisons the output rows of sequences with an invalid position (so the
// error is visible in the result rather than silently wrong).
__global__ __launch_bounds__(kBlock) void k_poison_rows(const int32_t* __restrict__ pos, int64_t max_tokens,
                                                        int64_t max_len, int64_t D, float* __restrict__ out) {
    const int b = blockIdx.y;
    if (seq_keys(pos, b, max_tokens, max_len) >= 0) return;
    for (int64_t d = blockIdx.x * (int64_t)kBlock + threadIdx.x; d < D; d += (int64_t)gridDim.x * kBlock)
        out[(int64_t)b * D + d] = NAN;
}

}  // namespace

hipError_t launch_rms_norm(const float* x, int64_t rows, int64_t D, const float* g, float eps, float* out,
                           hipStream_t s) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    k_rms_norm<<<(unsigned)rows, kBlock, 0, s>>>(x, D, g, eps, out);
    return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, float* y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = ceil_div(n, kBlock);
    if (blocks > 4096) blocks = 4096;
    k_add<<<(unsigned)blocks, kBlock, 0, s>>>(a, b, y, n);
    return hipGetLastError();
}

AttnPlan attn_plan(int64_t B, int64_t max_len) {
    AttnPlan p;
    // About 512 workgroups over all sequences, at least 8 and at most
    // kAttnMaxChunk keys per chunk.
    int64_t cs = ceil_div(max_len * B, 512);
    cs = cs < 8 ? 8 : (cs > kAttnMaxChunk ? kAttnMaxChunk : cs);
    p.CS = (int)cs;
    p.NC = (int)ceil_div(max_len, cs);
    return p;
}

int64_t attn_workspace_floats(int64_t B, int64_t D, int64_t max_len) {
    const AttnPlan p = attn_plan(B, max_len);
    return p.NC > 1 ? B * p.NC * (D + 4) : 0;
}

hipError_t launch_attention_decode(const float* q, const float* knew, const float* vnew, int64_t ldq, int64_t B,
                                   int64_t D, float* kc, float* vc, int64_t max_tokens, const int32_t* pos,
                                   int64_t max_len, float scale, float* part, float* ctx, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    const AttnPlan p = attn_plan(B, max_len);
    const size_t lds = (size_t)(D + kAttnMaxChunk) * sizeof(float);
    k_attn_partial<<<dim3((unsigned)p.NC, (unsigned)B), kBlock, lds, s>>>(q, knew, vnew, ldq, D, kc, vc, max_tokens,
                                                                        pos, max_len, p.CS, scale, part, ctx);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.NC > 1) {
        k_attn_combine<<<dim3((unsigned)ceil_div(D, 4 * kBlock), (unsigned)B), kBlock, 0, s>>>(
            part, p.NC, p.CS, D, pos, max_tokens, max_len, ctx);
    } else {
        k_poison_rows<<<dim3((unsigned)ceil_div(D, kBlock), (unsigned)B), kBlock, 0, s>>>(pos, max_tokens, max_len, D,
                                                                                       ctx);
    }
    return hipGetLastError();
}

}  // namespace sgq
