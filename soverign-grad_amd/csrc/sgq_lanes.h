// sgq_lanes.h -- cross-lane reductions within a 64-lane wavefront (gfx950),
// shared by the device code of libsgq.so.  Device-only; include from .hip files.
#pragma once

#include <hip/hip_runtime.h>

namespace sgq {
namespace {

// Value of `v` held by the lane whose index differs from this lane's in bit O,
// with VALU-latency cross-lane ops where gfx950 has them: DPP quad_perm for
// bits 0-1, ds_swizzle (xor mode) for bits 2-3, v_permlane16/32_swap for bits
// 4-5.  All lanes of the wavefront must be active.
template <int O>
__device__ __forceinline__ float xor_lane(float v, int lane) {
    const int iv = __float_as_int(v);
    if constexpr (O == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, true));  // quad_perm [1,0,3,2]
    } else if constexpr (O == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, true));  // quad_perm [2,3,0,1]
    } else if constexpr (O == 4 || O == 8) {
        return __int_as_float(__builtin_amdgcn_ds_swizzle(iv, (O << 10) | 0x1F));  // xor O within 32 lanes
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
        return __int_as_float((lane & 16) ? r[0] : r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        return __int_as_float((lane & 32) ? r[0] : r[1]);
    }
}

// Halving step across lane bit O (16 or 32) with v_permlane16/32_swap, two
// VALU ops per pair of values: swapping (x, y) = (v[i], v[i+h]) between the
// two lane halves leaves, in a lane with bit O clear, its own v[i] and the
// partner's v[i]; with bit O set, the partner's v[i+h] and its own.  Either
// way x + y is the pair total of the index that lane keeps (i or i+h).
template <int O>
__device__ __forceinline__ float swap_add(float x, float y) {
    const int xi = __float_as_int(x), yi = __float_as_int(y);
    if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(xi, yi, false, false);
        return __int_as_float(r[0]) + __int_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(xi, yi, false, false);
        return __int_as_float(r[0]) + __int_as_float(r[1]);
    }
}

// Lane bits in the order the reduction consumes them: cheapest exchange per
// pair first (permlane swaps, 2 ops; then DPP, then ds_swizzle, 4 ops),
// because the first steps move the most values.
constexpr int red_bit(int i) { return i == 0 ? 32 : i == 1 ? 16 : i == 2 ? 1 : i == 3 ? 2 : i == 4 ? 4 : 8; }

// Sums v[0..H) (H a power of two) over the 64 lanes of a wavefront.  While a
// lane carries more than one value, each step halves them: the lane with bit
// O set keeps the upper half plus its partner's upper half, the other keeps
// the lower half (every value is exchanged once).  With one value left, the
// remaining bits are plain butterflies.  On return v[0..red_left(H)) holds
// the totals of indices base + i.
template <int H, int I>
__device__ __forceinline__ void lane_reduce(float* v, int lane, int& base) {
    static_assert((H & (H - 1)) == 0, "halving needs a power of two");
    if constexpr (I < 6) {
        constexpr int O = red_bit(I);
        if constexpr (H > 1) {
            constexpr int h = H / 2;
            const bool upper = (lane & O) != 0;
            if constexpr (O >= 16) {
#pragma unroll
                for (int i = 0; i < h; ++i) v[i] = swap_add<O>(v[i], v[i + h]);
            } else {
#pragma unroll
                for (int i = 0; i < h; ++i) {
                    const float send = upper ? v[i] : v[i + h];
                    const float keep = upper ? v[i + h] : v[i];
                    v[i] = keep + xor_lane<O>(send, lane);
                }
            }
            if (upper) base += h;
            lane_reduce<h, I + 1>(v, lane, base);
        } else {
            v[0] += xor_lane<O>(v[0], lane);
            lane_reduce<1, I + 1>(v, lane, base);
        }
    }
}

// As lane_reduce, but a one-value step on lane bit 4 or 8 is a DPP row_shr
// accumulation (v += v of lane - O within the 16-lane row, zero below the row
// start) instead of an xor butterfly through ds_swizzle: VALU latency instead
// of an LDS round trip per step.  The totals are then only in the lanes with
// those bits set (the last lanes of each row); red_tail_writer(H) tells which
// lanes hold a total (once).
template <int H, int I>
__device__ __forceinline__ void lane_reduce_tail(float* v, int lane, int& base) {
    static_assert((H & (H - 1)) == 0, "halving needs a power of two");
    if constexpr (I < 6) {
        constexpr int O = red_bit(I);
        if constexpr (H > 1) {
            constexpr int h = H / 2;
            const bool upper = (lane & O) != 0;
            if constexpr (O >= 16) {
#pragma unroll
                for (int i = 0; i < h; ++i) v[i] = swap_add<O>(v[i], v[i + h]);
            } else {
#pragma unroll
                for (int i = 0; i < h; ++i) {
                    const float send = upper ? v[i] : v[i + h];
                    const float keep = upper ? v[i + h] : v[i];
                    v[i] = keep + xor_lane<O>(send, lane);
                }
            }
            if (upper) base += h;
            lane_reduce_tail<h, I + 1>(v, lane, base);
        } else if constexpr (O == 4 || O == 8) {
            v[0] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[0]), 0x110 + O, 0xF, 0xF, true));
            lane_reduce_tail<1, I + 1>(v, lane, base);
        } else {
            v[0] += xor_lane<O>(v[0], lane);
            lane_reduce_tail<1, I + 1>(v, lane, base);
        }
    }
}

// Lanes holding a total after lane_reduce_tail<H>: (lane & mask) == value.
// Bits 4 and 8 reduced by row_shr must be set; bits reduced by a butterfly
// must be clear (their lanes hold copies).
struct LaneSel {
    int mask, value;
};
constexpr LaneSel red_tail_writer(int H) {
    LaneSel s{0, 0};
    for (int i = 0; i < 6; ++i) {
        const int o = red_bit(i);
        if (H > 1) {
            H /= 2;
        } else {
            s.mask |= o;
            if (o == 4 || o == 8) s.value |= o;
        }
    }
    return s;
}

// Values a lane holds after lane_reduce, and the lane bits whose lanes then
// hold identical totals.
constexpr int red_left(int H) { return H >= 64 ? H / 64 : 1; }
constexpr int red_dup_mask(int H) {
    int m = 0;
    for (int i = 0; i < 6; ++i) {
        if (H > 1)
            H /= 2;
        else
            m |= red_bit(i);
    }
    return m;
}

}  // namespace
}  // namespace sgq
