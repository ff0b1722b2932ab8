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
#include "sgq_lanes.h"

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

// out[i, :] = w[(int)idx[i], :], or zeros for an id outside [0, V)
// (embedding, src/ops.cpp:2624-2650: ids are fp32 values truncated to int).
__global__ __launch_bounds__(kBlock) void k_embedding(const float* __restrict__ idx, const float* __restrict__ w,
                                                      int64_t V, int64_t E, float* __restrict__ out) {
    const float f = idx[blockIdx.x];
    // (int) of a float outside int's range is undefined in C++; such ids are
    // out of [0, V) anyway, so they are tested as floats first.
    const bool ok = f > -1.0f && f < (float)V;
    const int64_t id = ok ? (int64_t)(int)f : -1;
    float* o = out + (int64_t)blockIdx.x * E;
    const float* r = w + (id >= 0 && id < V ? id : 0) * E;
    for (int64_t e = threadIdx.x; e < E; e += kBlock) o[e] = (id >= 0 && id < V) ? r[e] : 0.0f;
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
//
// Latency, not bandwidth, bounds a decode step's attention (a few keys per
// workgroup), so every phase issues all of its loads before using any: the
// scores split D over the four wavefronts (each lane holds its slice of q and
// loads its slice of all CS keys at once), and the value sum loads KB keys'
// rows per batch.  Cached keys and values are read once per step: their loads
// take the non-temporal cache policy (ld_stream4), so they do not displace
// the step's weights and activations.
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float* row, int64_t i) {
    const f32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(row) + i);
    return make_float4(v.x, v.y, v.z, v.w);
}
template <int CS>
__global__ __launch_bounds__(kBlock) void k_attn_partial(const float* __restrict__ q, const float* __restrict__ knew,
                                                         const float* __restrict__ vnew, int64_t ldq, int64_t D,
                                                         float* __restrict__ kc, float* __restrict__ vc,
                                                         int64_t max_tokens, const int32_t* __restrict__ pos,
                                                         int64_t max_len, float scale,
                                                         float* __restrict__ part, float* __restrict__ ctx) {
    constexpr int NWV = kBlock / 64;
    __shared__ float red[NWV][CS];
    __shared__ float ex[CS];
    const int b = blockIdx.y, c = blockIdx.x, nc = gridDim.x;
    const int T = seq_keys(pos, b, max_tokens, max_len);
    const int j0 = c * CS;
    if (T < 0 || j0 >= T) return;  // combine reads only chunks below ceil(T / CS)
    const int n = min(CS, T - j0);
    const int p = T - 1;  // the new position
    const float* kn = knew + (int64_t)b * ldq;
    const float* vn = vnew + (int64_t)b * ldq;
    const float* kcb = kc + (int64_t)b * max_tokens * D;
    const float* vcb = vc + (int64_t)b * max_tokens * D;
    const int64_t D4 = D / 4;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // Scores: wavefront w sums dims [w * D4 / 4, (w + 1) * D4 / 4) (float4
    // units) of every key; lanes stride over that slice, KB keys' loads at a
    // time.  Keys past the chunk's n read the new row (always written memory)
    // and their scores are never used.
    constexpr int KB = CS < 8 ? CS : 8;
    // The first KB value rows of this thread's first PC float4 columns are
    // loaded now, so their latency overlaps the scores and the softmax.
    constexpr int PC = 2;
    float4 vpre[PC][KB];
#pragma unroll
    for (int ci = 0; ci < PC; ++ci) {
        const int64_t i = threadIdx.x + ci * kBlock;
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int j = j0 + u;
            const float* vr = (u >= n || j == p) ? vn : vcb + (int64_t)j * D;
            vpre[ci][u] = i < D4 ? ld_stream4(vr, i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    const int64_t s0 = wave * ((D4 + NWV - 1) / NWV), s1 = min(D4, s0 + (D4 + NWV - 1) / NWV);
    const float4* q4 = (const float4*)(q + (int64_t)b * ldq);
    for (int t0 = 0; t0 < n; t0 += KB) {
        float acc[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) acc[u] = 0.0f;
        for (int64_t i = s0 + lane; i < s1; i += 64) {
            const float4 qv = q4[i];
            float4 kv[KB];
#pragma unroll
            for (int u = 0; u < KB; ++u) {
                const int t = t0 + u, j = j0 + t;
                const float* kr = (t >= n || j == p) ? kn : kcb + (int64_t)j * D;
                kv[u] = ld_stream4(kr, i);
            }
#pragma unroll
            for (int u = 0; u < KB; ++u) {
                acc[u] = fmaf(qv.x, kv[u].x, acc[u]);
                acc[u] = fmaf(qv.y, kv[u].y, acc[u]);
                acc[u] = fmaf(qv.z, kv[u].z, acc[u]);
                acc[u] = fmaf(qv.w, kv[u].w, acc[u]);
            }
        }
        // Halving butterfly over the wavefront (DPP / permlane steps): lane
        // group `base` ends with the total of key t0 + base.
        int base = 0;
        lane_reduce<KB, 0>(acc, lane, base);
        if ((lane & red_dup_mask(KB)) == 0) red[wave][t0 + base] = acc[0];
    }
    // The chunk holding the new position appends it to the cache (no other
    // workgroup reads that row: they take it from knew / vnew).
    if (p >= j0 && p < j0 + n) {
        float4* kd = (float4*)(kc + ((int64_t)b * max_tokens + p) * D);
        float4* vd = (float4*)(vc + ((int64_t)b * max_tokens + p) * D);
        for (int64_t i = threadIdx.x; i < D4; i += kBlock) {
            kd[i] = ((const float4*)kn)[i];
            vd[i] = ((const float4*)vn)[i];
        }
    }
    __syncthreads();
    if (threadIdx.x < CS) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) v += red[w][threadIdx.x];
        red[0][threadIdx.x] = v * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int t = 0; t < n; ++t) m = fmaxf(m, red[0][t]);
    if (threadIdx.x < CS) ex[threadIdx.x] = threadIdx.x < n ? expf(red[0][threadIdx.x] - m) : 0.0f;
    __syncthreads();
    float l = 0.0f;
    for (int t = 0; t < n; ++t) l += ex[t];

    // o_c[d] = sum_j e_j v_j[d]: each thread owns float4 columns i, keys in
    // batches of KB with all of a batch's loads issued first.
    const bool direct = nc == 1;
    float* dst = direct ? ctx + (int64_t)b * D : part + ((int64_t)b * nc + c) * (D + 4);
    const float inv_l = 1.0f / l;
    // Column i of o_c: batch t0 of KB value rows is vv (loaded by the caller).
    auto fma_batch = [&](float4& o, const float4* vv, int t0) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            if (t0 + u < n) {  // uniform over the workgroup
                const float e = ex[t0 + u];
                o.x = fmaf(e, vv[u].x, o.x);
                o.y = fmaf(e, vv[u].y, o.y);
                o.z = fmaf(e, vv[u].z, o.z);
                o.w = fmaf(e, vv[u].w, o.w);
            }
        }
    };
    auto rest_and_store = [&](float4 o, int64_t i, int t_start) {
        for (int t0 = t_start; t0 < n; t0 += KB) {
            float4 vv[KB];
#pragma unroll
            for (int u = 0; u < KB; ++u) {
                const int t = t0 + u, j = j0 + t;
                const float* vr = (t >= n || j == p) ? vn : vcb + (int64_t)j * D;
                vv[u] = ld_stream4(vr, i);
            }
            fma_batch(o, vv, t0);
        }
        if (direct) {
            o.x = o.x * inv_l;
            o.y = o.y * inv_l;
            o.z = o.z * inv_l;
            o.w = o.w * inv_l;
        }
        ((float4*)dst)[i] = o;
    };
#pragma unroll
    for (int ci = 0; ci < PC; ++ci) {
        const int64_t i = threadIdx.x + ci * kBlock;
        if (i < D4) {
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            fma_batch(o, vpre[ci], 0);
            rest_and_store(o, i, KB);
        }
    }
    for (int64_t i = threadIdx.x + PC * kBlock; i < D4; i += kBlock)
        rest_and_store(make_float4(0.f, 0.f, 0.f, 0.f), i, 0);
    if (!direct && threadIdx.x == 0) {
        dst[D] = m;
        dst[D + 1] = l;
    }
}

// ctx[b] = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M) over the chunks
// that hold keys (M = max_c m_c).  Grid (ceil(D / (4 * kCombCols)), B): a
// workgroup owns kCombCols float4 columns of one sequence, and its
// kBlock / kCombCols thread groups split the chunks (group g takes chunks g,
// g + groups, ...), so each thread's loads of a batch are all in flight and
// many workgroups share the work even for one long sequence.  The chunk
// weights exp(m_c - M) go to LDS first; the group partial sums are added in
// group order through LDS (deterministic).  A sequence with an invalid
// position gets a NaN row.
constexpr int kCombCols = 16;
constexpr int kCombGroups = kBlock / kCombCols;  // 16
__global__ __launch_bounds__(kBlock) void k_attn_combine(const float* __restrict__ part, int nc, int CS, int64_t D,
                                                         const int32_t* __restrict__ pos, int64_t max_tokens,
                                                         int64_t max_len, float* __restrict__ ctx) {
    __shared__ float wgt[kAttnMaxChunks];
    __shared__ float4 grp[kCombGroups][kCombCols];
    __shared__ float red[kBlock / 64];
    __shared__ float lred[kBlock / 64];
    const int b = blockIdx.y;
    const int g = threadIdx.x / kCombCols, col = threadIdx.x % kCombCols;
    const int64_t D4 = D / 4;
    const int64_t i = (int64_t)blockIdx.x * kCombCols + col;  // float4 column
    const bool ok = i < D4;
    const int T = seq_keys(pos, b, max_tokens, max_len);
    if (T < 0) {
        if (g == 0 && ok) ((float4*)(ctx + (int64_t)b * D))[i] = make_float4(NAN, NAN, NAN, NAN);
        return;
    }
    const int used = (T + CS - 1) / CS;
    const float* pb = part + (int64_t)b * nc * (D + 4);
    // The first batch of this thread's chunk values loads now, under the
    // weight computation.
    constexpr int CB = 8;  // chunks per thread per batch
    float4 v0[CB];
#pragma unroll
    for (int u = 0; u < CB; ++u) {
        const int cc = g + u * kCombGroups;
        v0[u] = (ok && cc < used) ? ((const float4*)(pb + (int64_t)cc * (D + 4)))[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mx = -INFINITY;
    for (int cc = threadIdx.x; cc < used; cc += kBlock) {
        const float v = pb[(int64_t)cc * (D + 4) + D];
        wgt[cc] = v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) M = fmaxf(M, red[w]);
    float lp = 0.0f;  // this thread's share of L = sum_c l_c w_c, in chunk order per thread
    for (int cc = threadIdx.x; cc < used; cc += kBlock) {
        const float w = expf(wgt[cc] - M);
        wgt[cc] = w;
        lp = fmaf(pb[(int64_t)cc * (D + 4) + D + 1], w, lp);
    }
    lp = wave_sum(lp);
    if ((threadIdx.x & 63) == 0) lred[threadIdx.x >> 6] = lp;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) L += lred[w];
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = 0; c0 < used; c0 += CB * kCombGroups) {
        float4 v[CB];
#pragma unroll
        for (int u = 0; u < CB; ++u) {
            const int cc = c0 + g + u * kCombGroups;
            v[u] = c0 == 0 ? v0[u]
                           : ((ok && cc < used) ? ((const float4*)(pb + (int64_t)cc * (D + 4)))[i]
                                                : make_float4(0.f, 0.f, 0.f, 0.f));
        }
#pragma unroll
        for (int u = 0; u < CB; ++u) {
            const int cc = c0 + g + u * kCombGroups;
            if (cc < used) {
                const float w = wgt[cc];
                o.x = fmaf(v[u].x, w, o.x);
                o.y = fmaf(v[u].y, w, o.y);
                o.z = fmaf(v[u].z, w, o.z);
                o.w = fmaf(v[u].w, w, o.w);
            }
        }
    }
    grp[g][col] = o;
    __syncthreads();
    if (g == 0 && ok) {
        float4 t = grp[0][col];
#pragma unroll
        for (int gg = 1; gg < kCombGroups; ++gg) {
            const float4 u = grp[gg][col];
            t.x += u.x, t.y += u.y, t.z += u.z, t.w += u.w;
        }
        const float inv = 1.0f / L;
        ((float4*)(ctx + (int64_t)b * D))[i] = make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv);
    }
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

hipError_t launch_embedding(const float* idx, int64_t n, const float* w, int64_t V, int64_t E, float* out,
                            hipStream_t s) {
    if (n <= 0 || E <= 0) return hipSuccess;
    k_embedding<<<(unsigned)n, kBlock, 0, s>>>(idx, w, V, E, out);
    return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, float* y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = ceil_div(n, kBlock);
    if (blocks > 4096) blocks = 4096;
    k_add<<<(unsigned)blocks, kBlock, 0, s>>>(a, b, y, n);
    return hipGetLastError();
}

#ifndef SGQ_ATTN_WGS
#define SGQ_ATTN_WGS 2048
#endif
AttnPlan attn_plan(int64_t B, int64_t max_len) {
    // Up to SGQ_ATTN_WGS workgroups over all sequences; chunks of 8, 16, 32 or
    // 64 keys (kAttnMaxChunk), at most kAttnMaxChunks chunks per sequence.
    // Short chunks keep every load of a workgroup's phase in flight at once
    // (a chunk of 8 keys is one batch); the combine kernel splits the chunks
    // over thread groups, so many chunks cost it little.
    int64_t cs = 8;
    while (cs < kAttnMaxChunk &&
           (ceil_div(max_len, cs) * B > SGQ_ATTN_WGS || ceil_div(max_len, cs) > kAttnMaxChunks))
        cs *= 2;
    AttnPlan p;
    p.CS = (int)cs;
    p.NC = (int)ceil_div(max_len, cs);
    return p;
}

int64_t attn_max_len() { return kAttnMaxChunk * kAttnMaxChunks; }

int64_t attn_workspace_floats(int64_t B, int64_t D, int64_t max_len) {
    const AttnPlan p = attn_plan(B, max_len);
    return p.NC > 1 ? B * p.NC * (D + 4) : 0;
}

hipError_t launch_attention_decode(const float* q, const float* knew, const float* vnew, int64_t ldq, int64_t B,
                                   int64_t D, float* kc, float* vc, int64_t max_tokens, const int32_t* pos,
                                   int64_t max_len, float scale, float* part, float* ctx, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (max_len > attn_max_len()) return hipErrorInvalidValue;
    const AttnPlan p = attn_plan(B, max_len);
    const dim3 grid((unsigned)p.NC, (unsigned)B);
#define SGQ_ATTN(CS_)                                                                                                 \
    case CS_:                                                                                                         \
        k_attn_partial<CS_><<<grid, kBlock, 0, s>>>(q, knew, vnew, ldq, D, kc, vc, max_tokens, pos, max_len, scale, \
                                                    part, ctx);                                                       \
        break;
    switch (p.CS) {
        SGQ_ATTN(8)
        SGQ_ATTN(16)
        SGQ_ATTN(32)
        SGQ_ATTN(64)
        default:
            return hipErrorInvalidValue;
    }
#undef SGQ_ATTN
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.NC > 1) {
        k_attn_combine<<<dim3((unsigned)ceil_div(D, 4 * kCombCols), (unsigned)B), kBlock, 0, s>>>(
            part, p.NC, p.CS, D, pos, max_tokens, max_len, ctx);
    } else {
        k_poison_rows<<<dim3((unsigned)ceil_div(D, kBlock), (unsigned)B), kBlock, 0, s>>>(pos, max_tokens, max_len, D,
                                                                                       ctx);
    }
    return hipGetLastError();
}

}  // namespace sgq
