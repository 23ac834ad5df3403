// One decode token through every layer of a stack whose experts are all resident in HBM, in a
// single cooperative launch (gfx950).
//
// Reference semantics, per layer (mlx-qwen38/loader.py:903-908,948-965; the RMSNorm between
// layers is the stack's own glue):
//     x_l   = l == 0 ? x_0 : fp16(RMSNorm(y_{l-1}) * norm_w[l-1])
//     ids, scores = top-k(softmax(W_l x_l))                       (ascending gate, renormalised)
//     y_l   = x_l + sum_j s_j down_j(silu(gate_j x_l) * up_j x_l)  (fp32)
// with the arithmetic of the per-layer kernels (router.hip, q2_gemv.hip) step for step: fp64
// router dot products and RMSNorm rounded once to fp16, the same selection code, the same Q2
// dot products and the same cross-wave reduction order, so every id, score, x and y is
// bit-identical to the launch-per-kernel path.
//
// Why one launch: at batch 1 each layer moves 9.8 MB of expert weights (1.2 us at 8 TB/s), while
// each kernel boundary costs ~3.5-4 us.  Inside one launch the blocks hand data to each other
// through device memory instead: every published 32/64-bit word carries the token's epoch in its
// high bits, so a consumer needs no separate flag or counter -- it re-reads until every word it
// needs carries the current epoch (a 32/64-bit store is single-copy atomic).  Three hand-offs per
// layer remain (logits, h, y), each ~2.5 us on MI355X; the weight loads of a layer (gate/up and
// down together) are issued as soon as its experts are known, and the next layer's router rows
// and norm weights are prefetched before the layer's waits.
//
// Work split over G = hidden / 8 blocks (256 at hidden 2048: one block per CU): block b computes
// router rows [R b, R b + R), gate/up units (expert, intermediate row) [U b, U b + U) with the
// gate row on lanes 0-31 and the up row on lanes 32-63, and output rows [8 b, 8 b + 8) of the
// down product for every selected expert (one wave instruction per expert: 8 rows x 8 groups).
//
// Every wait is bounded: a timeout records (layer, phase) in the status word, raises the abort
// flag that every other waiter polls, and all waves leave the kernel.  Cooperative launch
// guarantees that the blocks are co-resident, so the waits do end in normal operation.
#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "moe_common.h"
#include "q2_dot.h"
#include "route_select.h"

namespace {

using namespace q2dot;

constexpr int kThreads = 256;
constexpr int kDownRows = 8;            // output rows per block
constexpr int kMaxUnitsPerWave = 8;     // gate/up units per wave
constexpr unsigned kSpinLimit = 1u << 22;

// Workspace (32-bit words): line 0 = the last token's epoch, line 1 = status, line 2 = abort flag,
// then per layer: logits [kLgWords] u32, h [kHxWords] u32, y [kYxWords] u64.
constexpr int kLine = 64;
constexpr int kWsEpoch = 0, kWsStatus = kLine, kWsAbort = 2 * kLine, kWsHeader = 4 * kLine;
constexpr int kLgWords = route::kMaxExperts;            // n_exp <= 1024
constexpr int kHxWords = MOE_MAX_K * 512;              // k * inter <= 8192
constexpr int kYxWords = 2048;                          // hidden <= 2048 (u64 words)
constexpr size_t kLayerWords = kLgWords + kHxWords + 2 * (size_t)kYxWords;

struct ResidentArgs {
    const __half* x0;          // [H] token input
    const __half* router_w;    // [L][E][H]
    const __half* norm_w;      // [L][H]  (the norm after layer l)
    const uint64_t* pools;     // [L] device addresses of blob pools holding every expert
    uint64_t stride;           // bytes per blob in the pools
    int n_layers, n_exp, k;
    float eps;
    BlobLayout lay;
    uint32_t* ids_out;         // [L][k]
    __half* scores_out;        // [L][k]
    __half* xs_out;            // [L + 1][H]
    float* hs_out;             // [L][H]
    uint32_t* ws;
};

__device__ __forceinline__ uint32_t ld32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t* layer_lg(uint32_t* ws, int l) { return ws + kWsHeader + (size_t)l * kLayerWords; }
__device__ __forceinline__ uint32_t* layer_hx(uint32_t* ws, int l) { return layer_lg(ws, l) + kLgWords; }
__device__ __forceinline__ uint64_t* layer_yx(uint32_t* ws, int l) {
    return reinterpret_cast<uint64_t*>(layer_hx(ws, l) + kHxWords);
}

// Record a timeout (first one wins) and raise the abort flag.
__device__ void fail(uint32_t* ws, int layer, int phase) {
    unsigned expected = 0;
    __hip_atomic_compare_exchange_strong(ws + kWsStatus, &expected, 0x80000000u | ((unsigned)layer << 8) | (unsigned)phase,
                                         __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    st32(ws + kWsAbort, 1u);
}

// y_{l-1} (fp32 words of the exchange) -> x_l = fp16(y / sqrt(mean(y^2) + eps) * w) into LDS xs,
// the arithmetic and summation order of the router's RMSNorm prologue.  Thread tid owns elements
// 4 (c 256 + tid) + 0..3 for chunks c = 0, 1.  Returns false on timeout / abort (block-uniform).
template <int H>
__device__ bool input_norm(uint32_t* ws, int l, unsigned ep, const uint2 (&w2)[2], float eps, uint16_t* xs,
                           double* red, __half* x_out) {
    constexpr int NCH = H / (4 * kThreads);
    static_assert(NCH >= 1 && NCH <= 2 && H % (4 * kThreads) == 0, "hidden must be 1024 or 2048");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint64_t* yx = layer_yx(ws, l - 1);
    float h[NCH][4];
    for (unsigned it = 0;; ++it) {
        bool mine = true;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint64_t v = ld64(yx + 4 * (c * kThreads + tid) + e);
                mine &= (uint32_t)(v >> 32) == ep;
                h[c][e] = __uint_as_float((uint32_t)v);
            }
        if (__syncthreads_and(mine)) break;
        if ((it & 63) == 63 && __syncthreads_or(tid == 0 ? (int)ld32(ws + kWsAbort) : 0)) return false;
        if (it >= kSpinLimit) {
            if (tid == 0) fail(ws, l, 1);
            return false;
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const double a = h[c][0], b = h[c][1], d = h[c][2], e = h[c][3];
        ss += a * a;
        ss += b * b;
        ss += d * d;
        ss += e * e;
    }
    ss = lanes::wave_sum_f64(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double denom = sqrt(tot / H + (double)eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int i = 4 * (c * kThreads + tid);
        uint16_t b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            double v = (double)h[c][j] / denom;
            v *= (double)__half2float(__ushort_as_half((uint16_t)(((j & 2) ? w2[c].y : w2[c].x) >> (16 * (j & 1)))));
            b[j] = route::f64_to_f16_bits(v);
        }
        const uint2 packed = make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
        *reinterpret_cast<uint2*>(&xs[i]) = packed;
        if (x_out) *reinterpret_cast<uint2*>(x_out + i) = packed;
    }
    __syncthreads();
    return true;
}

// RR: router rows per block (n_exp <= RR * G).
template <int GPR, int IPR, int RR>
__global__ __launch_bounds__(kThreads) void k_resident_token(ResidentArgs a) {
    constexpr int H = GPR * 64, I = IPR * 64;
    constexpr int G = H / kDownRows;                      // the grid (checked at launch)
    constexpr int LQ = RR * G / 64;                       // logits per lane of the polling wave
    static_assert(GPR == 32, "gate/up lanes: one 32-group row per half-wave");
    static_assert(IPR * kDownRows == 64, "down: 8 rows x IPR groups per wave instruction");
    constexpr int RU = H / 8 / kThreads;                  // router uint4 per thread and row
    static_assert(RU >= 1, "hidden >= 2048 / 1");
    constexpr int MAXJ = (MOE_MAX_K + 3) / 4;             // down experts per wave
    constexpr int HUNITS = MOE_MAX_K * I / 16;            // 16-value units of h at the largest k
    constexpr int HU_ITERS = (HUNITS + kThreads - 1) / kThreads;

    __shared__ __align__(16) uint16_t xs[H];
    __shared__ uint4 xp[GPR][8];
    __shared__ float xc[GPR][2];
    __shared__ uint4 hp[MOE_MAX_K][IPR][8];
    __shared__ float hc[MOE_MAX_K][IPR][2];
    __shared__ uint32_t keys[route::kMaxExperts];
    __shared__ float lraw_s[route::kMaxExperts];
    __shared__ double red[4], redm[4], reds[4];
    __shared__ double rred[4][RR];
    __shared__ uint32_t sel[MOE_MAX_K];
    __shared__ float sel_sc[MOE_MAX_K];
    __shared__ float dred[4][kDownRows];
    __shared__ int s_ok;

    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x;
    const int L = a.n_layers, E = a.n_exp, K = a.k;
    const int UPB = (K * I + G - 1) / G;                  // gate/up units per block
    uint32_t* ws = a.ws;
    // A workspace left by a timed-out launch holds words of an epoch that never completed: do
    // nothing until the caller re-zeroes it (moe_resident_status reports the failure).
    if (ld32(ws + kWsStatus) != 0u) return;
    const unsigned ep = (ld32(ws + kWsEpoch) % 65535u) + 1u;

    // ---- preloads for layer 0: router rows and (for the input norm of layer 1) norm weights --
    uint4 rq[RR][RU];
    auto load_router = [&](int l) {
        const __half* W = a.router_w + (size_t)l * E * H;
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            int row = b * RR + i;
            row = row < E ? row : E - 1;
#pragma unroll
            for (int u = 0; u < RU; ++u)
                rq[i][u] = *reinterpret_cast<const uint4*>(W + (size_t)row * H + 8 * (u * kThreads + tid));
        }
    };
    uint2 nw2[2];
    auto load_norm = [&](int l) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int i = 4 * (c * kThreads + tid);
            nw2[c] = *reinterpret_cast<const uint2*>(a.norm_w + (size_t)l * H + (i < H ? i : 0));
        }
    };
    load_router(0);
    load_norm(0);

    for (int l = 0; l < L; ++l) {
        // ---- 1. the layer's input x_l -> xs (LDS) ------------------------------------------------
        if (l == 0) {
            for (int i = tid; i < H / 8; i += kThreads)
                reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(a.x0)[i];
            if (b == 0)
                for (int i = tid; i < H / 8; i += kThreads)
                    reinterpret_cast<uint4*>(a.xs_out)[i] = reinterpret_cast<const uint4*>(a.x0)[i];
            __syncthreads();
        } else {
            uint2 w_prev[2] = {nw2[0], nw2[1]};
            if (!input_norm<H>(ws, l, ep, w_prev, a.eps, xs, red, b == 0 ? a.xs_out + (size_t)l * H : nullptr)) return;
        }

        // ---- 2. this block's router rows -> logits (epoch | fp16) --------------------------------
        {
            double acc[RR];
#pragma unroll
            for (int i = 0; i < RR; ++i) {
                acc[i] = 0.0;
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    const int off = 8 * (u * kThreads + tid);
                    const uint4 xq = *reinterpret_cast<const uint4*>(&xs[off]);
                    const __half* hw = reinterpret_cast<const __half*>(&rq[i][u]);
                    const __half* hx = reinterpret_cast<const __half*>(&xq);
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[i] += (double)(__half2float(hw[j]) * __half2float(hx[j]));
                }
                acc[i] = lanes::wave_sum_f64(acc[i]);
            }
            if (lane == 0)
#pragma unroll
                for (int i = 0; i < RR; ++i) rred[wv][i] = acc[i];
            __syncthreads();
            if (tid < RR && b * RR + tid < E) {
                const double s = rred[0][tid] + rred[1][tid] + rred[2][tid] + rred[3][tid];
                st32(layer_lg(ws, l) + b * RR + tid, ((uint32_t)ep << 16) | route::f64_to_f16_bits(s));
            }
        }

        // ---- 3. every logit of the layer (wave 0 polls), then the selection ----------------------
        if (wv == 0) {
            const uint32_t* lg = layer_lg(ws, l);
            bool ok = false;
            for (unsigned it = 0; it < kSpinLimit; ++it) {
                bool mine = true;
                uint32_t wds[LQ];
#pragma unroll
                for (int q = 0; q < LQ; ++q) {
                    const int e = lane + 64 * q;
                    wds[q] = ld32(lg + (e < E ? e : 0));
                    mine &= (e >= E) || (wds[q] >> 16) == ep;
                }
                if (__all(mine)) {
#pragma unroll
                    for (int q = 0; q < LQ; ++q) {
                        const int e = lane + 64 * q;
                        if (e < E) lraw_s[e] = __half2float(__ushort_as_half((uint16_t)(wds[q] & 0xFFFFu)));
                    }
                    ok = true;
                    break;
                }
                if ((it & 63) == 63 && ld32(ws + kWsAbort)) break;
            }
            if (!ok && lane == 0 && !ld32(ws + kWsAbort)) fail(ws, l, 2);
            if (lane == 0) s_ok = ok;
        }
        __syncthreads();
        if (!s_ok) return;
        {
            float lraw[route::kPer];
#pragma unroll
            for (int i = 0; i < route::kPer; ++i) {
                const int e = tid + route::kThreads * i;
                lraw[i] = lraw_s[e < E ? e : 0];
            }
            route::gate_keys(lraw, E, keys, redm, reds);
            if (wv == 0) {
                uint32_t id;
                __half sc;
                const int pos = route::select_topk(keys, ((E + 63) / 64) * 64, K, lane, id, sc);
                if (pos >= 0) {
                    sel[pos] = id;
                    sel_sc[pos] = __half2float(sc);
                    if (b == 0) {
                        a.ids_out[(size_t)l * K + pos] = id;
                        a.scores_out[(size_t)l * K + pos] = sc;
                    }
                }
            }
            __syncthreads();
        }

        // ---- 4. every weight load of the layer, then the next layer's router and norm rows ------
        const uint8_t* pool = reinterpret_cast<const uint8_t*>(a.pools[l]);
        const BlobLayout& Ly = a.lay;
        const int proj = lane >> 5, gg = lane & 31;
        uint4 gc[kMaxUnitsPerWave];
        uint32_t gsb[kMaxUnitsPerWave];
        const int upw = (UPB + 3) / 4;                        // units per wave (<= kMaxUnitsPerWave)
#pragma unroll
        for (int q = 0; q < kMaxUnitsPerWave; ++q) {
            int u = b * UPB + wv + 4 * q;
            const bool valid = q < upw && (wv + 4 * q) < UPB && u < K * I;
            u = valid ? u : 0;
            const int j = u / I, r = u % I;
            const uint8_t* blob = pool + (size_t)sel[j] * a.stride;
            gc[q] = *reinterpret_cast<const uint4*>(blob + (proj ? Ly.up_codes : Ly.gate_codes) + (size_t)r * GPR * 16 + gg * 16);
            gsb[q] = reinterpret_cast<const uint32_t*>(blob + (proj ? Ly.up_sb : Ly.gate_sb))[(size_t)r * GPR + gg];
        }
        const int dg = lane % IPR, drl = lane / IPR;
        const int drow = b * kDownRows + drl;
        uint4 dc[MAXJ];
        uint32_t dsb[MAXJ];
#pragma unroll
        for (int q = 0; q < MAXJ; ++q) {
            const int j = wv + 4 * q;
            const uint8_t* blob = pool + (size_t)sel[j < K ? j : K - 1] * a.stride;
            dc[q] = *reinterpret_cast<const uint4*>(blob + Ly.down_codes + (size_t)drow * IPR * 16 + dg * 16);
            dsb[q] = reinterpret_cast<const uint32_t*>(blob + Ly.down_sb)[(size_t)drow * IPR + dg];
        }
        if (l + 1 < L) load_router(l + 1);
        load_norm(l);

        // ---- 5. gate/up units -> h (epoch | fp16) -----------------------------------------------
        {
            // x as dot2 pairs (every lane takes part in the DPP sums; stores masked)
            const int n_units = GPR * 4;
            const int uc = tid < n_units ? tid : 0;
            const uint4 xlo = reinterpret_cast<const uint4*>(xs)[2 * uc];
            const uint4 xhi = reinterpret_cast<const uint4*>(xs)[2 * uc + 1];
            stage_pairs(xlo, xhi, tid < n_units, xp[uc >> 2], xc[uc >> 2], uc & 3, (uc >> 2) & 7);
            __syncthreads();
            h2_t P[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = xp[gg][i ^ (gg & 7)];
                P[4 * i] = as_h2(v.x);
                P[4 * i + 1] = as_h2(v.y);
                P[4 * i + 2] = as_h2(v.z);
                P[4 * i + 3] = as_h2(v.w);
            }
            const float cst = xc[gg][0], sum = xc[gg][1];
            uint32_t* hx = layer_hx(ws, l);
#pragma unroll
            for (int q = 0; q < kMaxUnitsPerWave; ++q) {
                if (q >= upw) break;
                const int ul = wv + 4 * q;
                const int u = b * UPB + ul;
                float part = sb_apply(gsb[q], q2_group_dot(gc[q], P), cst, sum);
                part = lanes::group_sum<GPR>(part);
                float gt, up;
                lanes::halves(part, gt, up);
                if (lane == 0 && ul < UPB && u < K * I) {
                    const float hval = gt / (1.0f + __expf(-gt)) * up;
                    st32(hx + u, ((uint32_t)ep << 16) | __half_as_ushort(__float2half_rn(hval)));
                }
            }
        }

        // ---- 6. every h of the layer -> LDS pairs; down rows + residual -> y ----------------------
        {
            const uint32_t* hx = layer_hx(ws, l);
            const int n_units = K * IPR * 4;                   // 16-value units of h
            uint32_t hw[HU_ITERS][16];
            for (unsigned it = 0;; ++it) {
                bool mine = true;
#pragma unroll
                for (int ui = 0; ui < HU_ITERS; ++ui) {
                    const int u = tid + kThreads * ui;
                    const int uc = u < n_units ? u : 0;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        hw[ui][e] = ld32(hx + 16 * uc + e);
                        mine &= (hw[ui][e] >> 16) == ep;
                    }
                }
                if (__syncthreads_and(mine)) break;
                if ((it & 63) == 63 && __syncthreads_or(tid == 0 ? (int)ld32(ws + kWsAbort) : 0)) return;
                if (it >= kSpinLimit) {
                    if (tid == 0) fail(ws, l, 3);
                    return;
                }
            }
#pragma unroll
            for (int ui = 0; ui < HU_ITERS; ++ui) {
                const int u = tid + kThreads * ui;
                if (kThreads * ui >= n_units) break;           // block-uniform
                const int uc = u < n_units ? u : 0;
                const int jj = uc / (IPR * 4), g2 = (uc >> 2) % IPR;
                uint32_t pk[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) pk[e] = (hw[ui][2 * e] & 0xFFFFu) | (hw[ui][2 * e + 1] << 16);
                stage_pairs(make_uint4(pk[0], pk[1], pk[2], pk[3]), make_uint4(pk[4], pk[5], pk[6], pk[7]), u < n_units,
                            hp[jj][g2], hc[jj][g2], uc & 3, g2 & 7);
            }
            __syncthreads();
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q < MAXJ; ++q) {
                const int j = wv + 4 * q;
                if (j >= K) break;
                h2_t P[32];
                const uint4* src = hp[j][dg];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint4 v = src[i ^ (dg & 7)];
                    P[4 * i] = as_h2(v.x);
                    P[4 * i + 1] = as_h2(v.y);
                    P[4 * i + 2] = as_h2(v.z);
                    P[4 * i + 3] = as_h2(v.w);
                }
                float part = sb_apply(dsb[q], q2_group_dot(dc[q], P), hc[j][dg][0], hc[j][dg][1]);
                part = lanes::group_sum<IPR>(part);
                acc += sel_sc[j] * part;
            }
            if (dg == 0) dred[wv][drl] = acc;
            __syncthreads();
            if (tid < kDownRows) {
                const int row = b * kDownRows + tid;
                float y = ((dred[0][tid] + dred[1][tid]) + dred[2][tid]) + dred[3][tid];
                y += __half2float(__ushort_as_half(xs[row]));
                a.hs_out[(size_t)l * H + row] = y;
                st64(layer_yx(ws, l) + row, ((uint64_t)ep << 32) | __float_as_uint(y));
            }
        }
    }

    // ---- the last layer's output through its norm (block 0), then the epoch -----------------------
    if (b == 0) {
        uint2 w_last[2] = {nw2[0], nw2[1]};
        if (!input_norm<H>(ws, L, ep, w_last, a.eps, xs, red, a.xs_out + (size_t)L * H)) return;
        if (tid == 0) st32(ws + kWsEpoch, ep);
    }
}

}  // namespace

uint64_t resident_workspace_bytes(int n_layers) {
    return ((uint64_t)kWsHeader + (uint64_t)n_layers * kLayerWords) * sizeof(uint32_t);
}

int launch_resident_token(const __half* x0, const __half* router_w, const __half* norm_w, const uint64_t* pools,
                          size_t stride, int n_layers, int hidden, int n_exp, int k, int inter, int group, float eps,
                          uint32_t* ids_out, __half* scores_out, __half* xs_out, float* hs_out, uint32_t* ws,
                          hipStream_t s) {
    if (hidden != 2048 || inter != 512 || group != 64) {
        moe_set_error("resident_token: hidden=%d inter=%d group=%d (this kernel takes 2048 / 512 / 64)", hidden, inter, group);
        return -1;
    }
    const int G = hidden / kDownRows;
    if (n_layers <= 0 || n_layers > MOE_MAX_LAYERS || k <= 0 || k > MOE_MAX_K || n_exp <= 0 || n_exp > 4 * G ||
        k > n_exp || ((k * inter + G - 1) / G + 3) / 4 > kMaxUnitsPerWave) {
        moe_set_error("resident_token: n_layers=%d n_exp=%d k=%d out of range", n_layers, n_exp, k);
        return -1;
    }
    if (!x0 || !router_w || !norm_w || !pools || !ids_out || !scores_out || !xs_out || !hs_out || !ws) {
        moe_set_error("resident_token: null pointer argument");
        return -1;
    }
    BlobLayout L = blob_layout(hidden, inter, group);
    if (stride < L.bytes) { moe_set_error("resident_token: stride %zu < blob bytes %zu", stride, L.bytes); return -1; }
    const bool four = n_exp > 2 * G;                    // router rows per block: 2 or 4
    const void* kern = four ? (const void*)k_resident_token<32, 8, 4> : (const void*)k_resident_token<32, 8, 2>;
    int dev = 0, n_cu = 0;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    int per_cu = 0;
    HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, 0));
    if (per_cu * n_cu < G) {
        moe_set_error("resident_token: %d blocks cannot be co-resident (%d CUs x %d)", G, n_cu, per_cu);
        return -1;
    }
    ResidentArgs a;
    a.x0 = x0;
    a.router_w = router_w;
    a.norm_w = norm_w;
    a.pools = pools;
    a.stride = stride;
    a.n_layers = n_layers;
    a.n_exp = n_exp;
    a.k = k;
    a.eps = eps;
    a.lay = L;
    a.ids_out = ids_out;
    a.scores_out = scores_out;
    a.xs_out = xs_out;
    a.hs_out = hs_out;
    a.ws = ws;
    void* args[] = {&a};
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (kt_enabled()) kt_events(TK_RESIDENT, &e0, &e1);
    if (e0) HIP_TRY(hipEventRecord(e0, s));
    HIP_TRY(hipLaunchCooperativeKernel(kern, dim3(G), dim3(kThreads), args, 0, s));
    if (e1) HIP_TRY(hipEventRecord(e1, s));
    return 0;
}

int read_resident_status(const uint32_t* ws, hipStream_t s, uint32_t* out) {
    HIP_TRY(hipMemcpyAsync(out, ws + kWsStatus, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return 0;
}
