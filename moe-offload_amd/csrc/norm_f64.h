// fp64 RMSNorm of an fp32 vector by one block of 256 threads, shared by the router's prologue,
// the standalone RMSNorm and the codebook up-projection's prologue, so all three round the same
// way: x = fp16(h / sqrt(mean(h^2) + eps) * w), the sum of squares in fp64 (per-thread chunks,
// then wave sums, then the 4 wave partials in order), one rounding to fp16.
//
// Thread tid owns elements 4 (c * 256 + tid) + 0..3 of chunk c (hidden is a multiple of 8, at
// most 4096).  The caller issues the chunk loads itself, ahead of its weight loads (loads retire
// in issue order), so the normalisation overlaps the weights' flight.
#pragma once

#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "route_select.h"

namespace norm64 {

constexpr int kThreads = 256;
constexpr int kMaxHidden = 4096;
constexpr int kChunks = kMaxHidden / (4 * kThreads);

struct NormIn {
    float4 hv[kChunks];      // 4 consecutive fp32 of h per chunk
    uint2 w2[kChunks];       // the matching 4 fp16 norm weights
};

// The chunk loads, unconditional from clamped in-range addresses (chunks past the end reread the
// last 4 elements and are ignored by finish()).  Without norm weights, h is read in their place.
__device__ __forceinline__ void load(NormIn& in, const float* __restrict__ h_in, const __half* __restrict__ norm_w,
                                     int hidden) {
    const __half* wsrc = norm_w ? norm_w : reinterpret_cast<const __half*>(h_in);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int i = 4 * (c * kThreads + (int)threadIdx.x);
        const int ic = i < hidden ? i : hidden - 4;
        in.hv[c] = *reinterpret_cast<const float4*>(h_in + ic);
        in.w2[c] = *reinterpret_cast<const uint2*>(wsrc + ic);
    }
}

// Normalises into xs (fp16 bits in LDS, [hidden]) and, when x_out is given, global memory.
// Contains one __syncthreads (the block reduction); xs is complete only after the caller's next
// barrier.  red: 4 doubles of LDS.
__device__ inline void finish(const NormIn& in, bool has_w, float eps, int hidden, uint16_t* xs, __half* x_out,
                              double* red) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        if (4 * (c * kThreads + tid) >= hidden) continue;
        const double a = in.hv[c].x, b = in.hv[c].y, d = in.hv[c].z, e = in.hv[c].w;
        ss += a * a;
        ss += b * b;
        ss += d * d;
        ss += e * e;
    }
    ss = lanes::wave_sum_f64(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double denom = sqrt(tot / hidden + (double)eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int i = 4 * (c * kThreads + tid);
        if (i >= hidden) continue;
        const float hh[4] = {in.hv[c].x, in.hv[c].y, in.hv[c].z, in.hv[c].w};
        const uint32_t ww[2] = {in.w2[c].x, in.w2[c].y};
        uint16_t b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            double v = (double)hh[j] / denom;
            if (has_w) v *= (double)__half2float(__ushort_as_half((uint16_t)(ww[j >> 1] >> (16 * (j & 1)))));
            b[j] = route::f64_to_f16_bits(v);
        }
        const uint2 packed = make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
        *reinterpret_cast<uint2*>(&xs[i]) = packed;
        if (x_out) *reinterpret_cast<uint2*>(x_out + i) = packed;
    }
}

// The checkpoint form (bf16 model): the same sum of squares and normalisation with bf16 norm
// weights, x rounded once from fp64 to bf16 (x_bf16, the 8-bit router's input) and that bf16 value
// converted to fp16 (x_f16, the expert kernels' input: exact in fp16's normal range).  Every
// thread writes its own elements to whichever outputs are given: x_bf16 / x_f16 in global memory,
// xf (LDS, [hidden]) the bf16 value as fp32 for a router that multiplies in this block.  One
// __syncthreads (the block reduction); xf is complete only after the caller's next barrier.
__device__ inline void finish_bf16(const NormIn& in, bool has_w, float eps, int hidden, uint16_t* __restrict__ x_bf16,
                                   __half* __restrict__ x_f16, double* red, float* __restrict__ xf = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        if (4 * (c * kThreads + tid) >= hidden) continue;
        const double a = in.hv[c].x, b = in.hv[c].y, d = in.hv[c].z, e = in.hv[c].w;
        ss += a * a;
        ss += b * b;
        ss += d * d;
        ss += e * e;
    }
    ss = lanes::wave_sum_f64(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double denom = sqrt(tot / hidden + (double)eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int i = 4 * (c * kThreads + tid);
        if (i >= hidden) continue;
        const float hh[4] = {in.hv[c].x, in.hv[c].y, in.hv[c].z, in.hv[c].w};
        const uint32_t ww[2] = {in.w2[c].x, in.w2[c].y};
        uint16_t b[4], f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            double v = (double)hh[j] / denom;
            if (has_w) v *= (double)route::bf16_to_f32((ww[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            b[j] = route::f64_to_bf16_bits(v);
            f[j] = __half_as_ushort(__float2half_rn(route::bf16_to_f32(b[j])));
        }
        if (x_bf16)
            *reinterpret_cast<uint2*>(x_bf16 + i) =
                make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
        if (x_f16)
            *reinterpret_cast<uint2*>(x_f16 + i) =
                make_uint2((uint32_t)f[0] | ((uint32_t)f[1] << 16), (uint32_t)f[2] | ((uint32_t)f[3] << 16));
        if (xf)
            *reinterpret_cast<float4*>(xf + i) = make_float4(route::bf16_to_f32(b[0]), route::bf16_to_f32(b[1]),
                                                             route::bf16_to_f32(b[2]), route::bf16_to_f32(b[3]));
    }
}

}  // namespace norm64
