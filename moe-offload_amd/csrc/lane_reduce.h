// Cross-lane reductions for 64-wide gfx950 waves without LDS traffic.
//
// Steps inside a 16-lane row are DPP moves (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror); the two 32-lane steps are v_permlane16_swap (row pairs 0-1 and 2-3) and
// v_permlane32_swap (the wave halves).  Each step hands every lane the partial of its partner
// lane group, and both partners add the same two operands (fp addition commutes), so every lane
// of a group ends with the bit-identical result.  A __shfl_xor step instead costs a
// ds_bpermute round trip through the LDS unit, waited for before the next step.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lanes {

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// The value of the partner lane for a butterfly step of width W (1, 2, 4, 8: inside 16-lane
// rows) as the two operands (mine, partner).
template <int W>
__device__ __forceinline__ uint32_t partner(uint32_t v) {
    static_assert(W == 1 || W == 2 || W == 4 || W == 8, "DPP steps cover widths 1..8");
    if constexpr (W == 1) return dpp<0xB1>(v);       // lane ^ 1
    else if constexpr (W == 2) return dpp<0x4E>(v);  // lane ^ 2
    else if constexpr (W == 4) return dpp<0x141>(v); // row_half_mirror: 7 - i inside 8 lanes
    else return dpp<0x140>(v);                       // row_mirror: 15 - i inside 16 lanes
}

// Sum over aligned groups of N lanes (N = 1, 2, 4, ..., 64); every lane of a group gets the sum.
// The mirror steps are valid butterflies because by then every lane of each half holds the same
// partial.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
    if constexpr (N >= 2) v += __uint_as_float(partner<1>(__float_as_uint(v)));
    if constexpr (N >= 4) v += __uint_as_float(partner<2>(__float_as_uint(v)));
    if constexpr (N >= 8) v += __uint_as_float(partner<4>(__float_as_uint(v)));
    if constexpr (N >= 16) v += __uint_as_float(partner<8>(__float_as_uint(v)));
    if constexpr (N >= 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if constexpr (N >= 64) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

// (value of the lower wave half, value of the upper wave half) for the same lane offset.
__device__ __forceinline__ void halves(float v, float& lo, float& hi) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(p[0]);
    hi = __uint_as_float(p[1]);
}

__device__ __forceinline__ double f64_from(uint32_t lo, uint32_t hi) {
    return __hiloint2double((int)hi, (int)lo);
}

template <int W>
__device__ __forceinline__ double partner_f64(double v) {
    const uint32_t lo = (uint32_t)__double2loint(v), hi = (uint32_t)__double2hiint(v);
    return f64_from(partner<W>(lo), partner<W>(hi));
}

// fp64 reductions over the whole wave (sum or max); every lane gets the result.
template <bool MAX>
__device__ __forceinline__ double wave_reduce_f64(double v) {
    auto op = [](double a, double b) { return MAX ? fmax(a, b) : a + b; };
    v = op(v, partner_f64<1>(v));
    v = op(v, partner_f64<2>(v));
    v = op(v, partner_f64<4>(v));
    v = op(v, partner_f64<8>(v));
    {
        const uint32_t lo = (uint32_t)__double2loint(v), hi = (uint32_t)__double2hiint(v);
        const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        v = op(f64_from(pl[0], ph[0]), f64_from(pl[1], ph[1]));
    }
    {
        const uint32_t lo = (uint32_t)__double2loint(v), hi = (uint32_t)__double2hiint(v);
        const auto pl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto ph = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        v = op(f64_from(pl[0], ph[0]), f64_from(pl[1], ph[1]));
    }
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) { return wave_reduce_f64<false>(v); }
__device__ __forceinline__ double wave_max_f64(double v) { return wave_reduce_f64<true>(v); }

}  // namespace lanes
