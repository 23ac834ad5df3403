// Q2 (2-bit affine, group 64) dot products shared by the decode kernels (gfx950).
//
// One 16-byte load is one group (64 codes) of one weight row; the (scale, bias) pair is one
// 32-bit word.  Codes are expanded without integer->float conversions: OR-ing a code pair into
// the mantissa of fp16 1024.0 gives the exact halves 1024 + c*4^p, which feed v_dot2_f32_f16
// against the matching activation pair.  With 5 accumulators (one per power 4^p):
//     sum_i c_i x_i = sum_p 4^-p A_p - 1024 * sum_i x_i 4^-p(i)
// and the second term is a per-(vector, group) constant computed once when the activation
// vector is staged (stage_pairs).
#pragma once
#include <hip/hip_fp16.h>

#include "lane_reduce.h"

namespace q2dot {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

constexpr uint32_t kMagic = 0x64006400u;   // fp16 1024.0 in both halves

// Dot of one group (4 words = 64 codes) with 32 activation pairs laid out as
// P[8*w + j] = (a[16w + j], a[16w + j + 8]), j = 0..7.
__device__ __forceinline__ float q2_group_dot(uint4 c, const h2_t* P) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f;
    const uint32_t words[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t v = words[w];
        const uint32_t v2 = v >> 10;
        const h2_t* p = P + 8 * w;
        a0 = __builtin_amdgcn_fdot2(as_h2((v & 0x00030003u) | kMagic), p[0], a0, false);
        a1 = __builtin_amdgcn_fdot2(as_h2((v & 0x000C000Cu) | kMagic), p[1], a1, false);
        a2 = __builtin_amdgcn_fdot2(as_h2((v & 0x00300030u) | kMagic), p[2], a2, false);
        a3 = __builtin_amdgcn_fdot2(as_h2((v & 0x00C000C0u) | kMagic), p[3], a3, false);
        a4 = __builtin_amdgcn_fdot2(as_h2((v & 0x03000300u) | kMagic), p[4], a4, false);
        a0 = __builtin_amdgcn_fdot2(as_h2((v2 & 0x00030003u) | kMagic), p[5], a0, false);
        a1 = __builtin_amdgcn_fdot2(as_h2((v2 & 0x000C000Cu) | kMagic), p[6], a1, false);
        a2 = __builtin_amdgcn_fdot2(as_h2((v2 & 0x00300030u) | kMagic), p[7], a2, false);
    }
    return a0 + 0.25f * a1 + 0.0625f * a2 + 0.015625f * a3 + 0.00390625f * a4;
}

// Weight of input position j (0..15) inside a word in the offset constant: 4^-class.
__device__ __forceinline__ float pos_weight(int j) {
    int p = j & 7;
    int cls = (p <= 4) ? p : p - 5;
    return 1.0f / (float)(1 << (2 * cls));
}

__device__ __forceinline__ float sb_apply(uint32_t sb, float dot, float cst, float sum) {
    float sc = __half2float(__ushort_as_half((uint16_t)(sb & 0xFFFFu)));
    float bi = __half2float(__ushort_as_half((uint16_t)(sb >> 16)));
    return sc * (dot - cst) + bi * sum;
}

// Stage one 16-value unit of an fp16 vector (lo = values 0-7, hi = 8-15 of unit w of a group of
// 64) as its 8 dot2 pairs P[8w + p] = (a[16w + p], a[16w + p + 8]) and add its share of the
// group's constants.  The 4 units of a group sit on 4 adjacent lanes, which sum the constants
// with two DPP steps, so every lane of the wave must call this (store masks the writes).
// A group's 8 pair vectors sit at slots i ^ swz (swz = group & 7): lanes reading vector i of
// different groups then hit different LDS banks instead of all the same ones (a group is 128
// bytes, a full bank cycle).
__device__ __forceinline__ void stage_pairs(uint4 lo4, uint4 hi4, bool store, uint4* grp_pairs, float* grp_c, int w,
                                            int swz) {
    const uint32_t lo[4] = {lo4.x, lo4.y, lo4.z, lo4.w};
    const uint32_t hi[4] = {hi4.x, hi4.y, hi4.z, hi4.w};
    uint32_t pr[8];
    float cc = 0.f, ss = 0.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        pr[p] = __builtin_amdgcn_perm(hi[p >> 1], lo[p >> 1], (p & 1) ? 0x07060302u : 0x05040100u);
        const h2_t v = as_h2(pr[p]);
        const float f = (float)v.x + (float)v.y;
        ss += f;
        cc += pos_weight(p) * f;
    }
    cc = lanes::group_sum<4>(cc);
    ss = lanes::group_sum<4>(ss);
    if (store) {
        grp_pairs[(2 * w) ^ swz] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        grp_pairs[(2 * w + 1) ^ swz] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
        if (w == 0) {
            grp_c[0] = 1024.0f * cc;
            grp_c[1] = ss;
        }
    }
}


}  // namespace q2dot
