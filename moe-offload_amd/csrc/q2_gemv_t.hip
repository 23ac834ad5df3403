// Q2 gather-GEMV (SwitchGLU decode) over experts addressed as tensors, at any hidden / intermediate
// size that is a multiple of 64 (gfx950).
//
// Reference semantics: mlx-qwen38/loader.py:557-564,964-965 (gather_qmm x3 + SwiGLU + the
// score-weighted sum), cpp/src/layers.cpp:343-362.  The reference keeps a layer's slot pool as 9
// tensors (loader.py:332-406): per projection (gate, up, down) a code pool [cap][out][in/16] u32 and
// scale and bias pools [cap][out][in/64] (bf16 in its checkpoints).  Here each projection is
// addressed by three base addresses with their own bytes per slot, and scale/bias by an element
// step (2: separate arrays, 4: the interleaved (scale, bias) words of a blob), so the same kernels
// read the reference's 9 pools in place, bf16 or fp16, and blob pools of any shape.  The real
// model's layer (hidden 2560, intermediate 640: 40 and 10 groups per row) runs here.
//
// Arithmetic: the Q2 dot of q2_dot.h (codes expanded by the fp16 1024-offset trick, v_dot2 against
// activation pairs staged in LDS), fp32 accumulation, W = scale * q + bias per group of 64.
//   k_q2t_gate_up: LPR = 8, 16 or 32 lanes per row, each lane looping over the row's groups
//                  g = l, l + LPR, ...; gate rows on lanes 0-31, up rows on lanes 32-63.
//   k_q2t_down:    16 lanes per output row (one group each: intermediate <= 1024), 8 rows per
//                  block, the block's 8 waves split the experts; fixed-order cross-wave sum.
#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "moe_common.h"
#include "q2_dot.h"
#include "route_select.h"

namespace {

using namespace q2dot;

constexpr int kTMaxGroups = 64;         // hidden <= 4096
constexpr int kTMaxPasses = 8;          // groups per lane of a gate/up row
constexpr int kTDownRows = 8;           // output rows per down block
constexpr int kTDownWaves = 8;          // waves per down block (1-2 of the top-10 experts each)
static_assert((kTDownRows & (kTDownRows - 1)) == 0, "the epilogue row of a thread is tid & (kTDownRows - 1)");
constexpr int kTDownLanes = 16;         // lanes per down row: intermediate <= 1024

// Block index -> row block, keeping consecutive row blocks on one XCD (blocks are dealt to the 8
// XCDs round robin): a down row's scales and biases (2 bytes per group) share 128-byte lines with
// the neighbouring rows, which another XCD's L2 would fetch again.
__device__ __forceinline__ int xcd_rank(int b, int nb) {
    const int per = nb / 8, rem = nb % 8, x = b % 8, i = b / 8;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

template <bool BF16>
__device__ __forceinline__ float half_bits(uint16_t v) {
    if constexpr (BF16) return __uint_as_float((uint32_t)v << 16);
    else return __half2float(__ushort_as_half(v));
}

// Rows of gate and up for one selected expert.  ROUTED: the block first selects the top-k experts
// itself from the logits of the checkpoint's router (bf16, moe_router_q8's rule in bf16, the same
// code: route_select.h) over a pool holding every expert (slot = id); block (0, 0) also writes the
// ids and bf16 scores, after its weight loads are issued.
template <bool BF16, int LPR, bool ROUTED>
__device__ __forceinline__ void q2t_gate_up_body(const __half* __restrict__ x, const Q2Experts& E,
                                                 const uint32_t* __restrict__ slots, int n_slots, int hidden,
                                                 int inter, __half* __restrict__ h_out,
                                                 const uint16_t* __restrict__ logits, int k,
                                                 uint32_t* __restrict__ ids_out, uint16_t* __restrict__ scores_out) {
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = blockIdx.y;
    const int GPR = hidden >> 6;
    constexpr int RPW = 32 / LPR;                       // rows per projection and wave
    const int passes = (GPR + LPR - 1) / LPR;
    const int proj = lane >> 5, rl = (lane & 31) / LPR, l8 = lane & (LPR - 1);
    const int row = (blockIdx.x * 4 + wv) * RPW + rl;
    __shared__ uint4 xp[kTMaxGroups][8];
    __shared__ float xc[kTMaxGroups][2];

    // the activation units first (one 16-value unit per thread), then every weight load
    const int n_units = hidden >> 4;
    const int uc = tid < n_units ? tid : 0;
    const uint4 xlo = reinterpret_cast<const uint4*>(x)[2 * uc];
    const uint4 xhi = reinterpret_cast<const uint4*>(x)[2 * uc + 1];
    uint32_t slot;
    uint32_t top_key = 0;                                 // routed, wave 0: lane r's r-th largest key
    if constexpr (ROUTED) {
        __builtin_amdgcn_sched_barrier(0);
        __shared__ uint32_t keys[route::kMaxExperts];
        __shared__ double redm[4], reds[4];
        __shared__ uint32_t sel[MOE_MAX_K];
        float lraw[route::kPer];
#pragma unroll
        for (int i = 0; i < route::kPer; ++i) {
            const int e = tid + route::kThreads * i;
            lraw[i] = route::bf16_to_f32(logits[e < n_slots ? e : 0]);
        }
        route::gate_keys<true>(lraw, n_slots, keys, redm, reds);
        if (wv == 0) {
            top_key = route::wave_topn(keys, 0, ((n_slots + 63) / 64) * 64, k, lane);
            if (lane < k) sel[k - 1 - lane] = top_key & 0xFFFFu;
        }
        __syncthreads();
        slot = sel[j];
    } else {
        slot = slots[j];
    }
    const bool ok = slot < (uint32_t)n_slots;             // an invalid slot yields h = 0
    const size_t s = ok ? slot : 0;
    const int rowc = row < inter ? row : inter - 1;
    const Q2Proj& Pg = E.p[0];
    const Q2Proj& Pu = E.p[1];
    const uint8_t* wb = proj ? Pu.w + s * Pu.w_stride : Pg.w + s * Pg.w_stride;
    const uint8_t* sb = proj ? Pu.s + s * Pu.s_stride : Pg.s + s * Pg.s_stride;
    const uint8_t* bb = proj ? Pu.b + s * Pu.b_stride : Pg.b + s * Pg.b_stride;
    const int step = proj ? Pu.sb_step : Pg.sb_step;
    wb += (size_t)rowc * (hidden >> 2);
    sb += (size_t)rowc * GPR * step;
    bb += (size_t)rowc * GPR * step;
    uint4 c[kTMaxPasses];
    uint16_t sc[kTMaxPasses], bi[kTMaxPasses];
#pragma unroll
    for (int t = 0; t < kTMaxPasses; ++t) {
        if (t >= passes) break;                           // wave-uniform
        int g = l8 + LPR * t;
        g = g < GPR ? g : GPR - 1;
        c[t] = *reinterpret_cast<const uint4*>(wb + (size_t)g * 16);
        sc[t] = *reinterpret_cast<const uint16_t*>(sb + (size_t)g * step);
        bi[t] = *reinterpret_cast<const uint16_t*>(bb + (size_t)g * step);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ROUTED) {
        if (wv == 0 && blockIdx.x == 0 && blockIdx.y == 0) {
            uint32_t id;
            uint16_t scb;
            const int pos = route::topk_score_bits<true>(top_key, k, lane, id, scb);
            if (pos >= 0) {
                ids_out[pos] = id;
                scores_out[pos] = scb;
            }
        }
    }
    stage_pairs(xlo, xhi, tid < n_units, xp[uc >> 2], xc[uc >> 2], uc & 3, (uc >> 2) & 7);
    __syncthreads();

    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < kTMaxPasses; ++t) {
        if (t >= passes) break;
        const int g = l8 + LPR * t;
        if (g < GPR) {
            h2_t P[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = xp[g][i ^ (g & 7)];
                P[4 * i] = as_h2(v.x);
                P[4 * i + 1] = as_h2(v.y);
                P[4 * i + 2] = as_h2(v.z);
                P[4 * i + 3] = as_h2(v.w);
            }
            const float dot = q2_group_dot(c[t], P);
            acc += half_bits<BF16>(sc[t]) * (dot - xc[g][0]) + half_bits<BF16>(bi[t]) * xc[g][1];
        }
    }
    acc = lanes::group_sum<LPR>(acc);
    float gt, up;
    lanes::halves(acc, gt, up);
    if (proj == 0 && l8 == 0 && row < inter) {
        const float hval = ok ? gt / (1.0f + __expf(-gt)) * up : 0.0f;
        h_out[(size_t)j * inter + row] = __float2half_rn(hval);
    }
}

template <bool BF16, int LPR>
__global__ __launch_bounds__(256) void k_q2t_gate_up(const __half* __restrict__ x, Q2Experts E,
                                                     const uint32_t* __restrict__ slots, int n_slots, int hidden,
                                                     int inter, __half* __restrict__ h_out) {
    q2t_gate_up_body<BF16, LPR, false>(x, E, slots, n_slots, hidden, inter, h_out, nullptr, 0, nullptr, nullptr);
}

template <bool BF16, int LPR>
__global__ __launch_bounds__(256) void k_q2t_gate_up_routed(const __half* __restrict__ x, Q2Experts E,
                                                            const uint16_t* __restrict__ logits, int n_exp, int k,
                                                            int hidden, int inter, uint32_t* __restrict__ ids_out,
                                                            uint16_t* __restrict__ scores_out,
                                                            __half* __restrict__ h_out) {
    q2t_gate_up_body<BF16, LPR, true>(x, E, nullptr, n_exp, hidden, inter, h_out, logits, k, ids_out, scores_out);
}

template <bool BF16>
__global__ __launch_bounds__(64 * kTDownWaves) void k_q2t_down(const __half* __restrict__ h, Q2Experts E,
                                                  const uint32_t* __restrict__ slots, int n_slots,
                                                  const __half* __restrict__ scores, int k, int hidden, int inter,
                                                  const __half* __restrict__ residual, float* __restrict__ y_out,
                                                  int per_expert) {
    constexpr int RPI = 64 / kTDownLanes;                 // rows per wave instruction
    constexpr int ITERS = kTDownRows / RPI;
    constexpr int MAXJ = (MOE_MAX_K + kTDownWaves - 1) / kTDownWaves;
    constexpr int kUnitIters = (MOE_MAX_K * 1024 / 16 + 64 * kTDownWaves - 1) / (64 * kTDownWaves);
    __shared__ uint4 hp[MOE_MAX_K][kTDownLanes][8];
    __shared__ float hc[MOE_MAX_K][kTDownLanes][2];
    __shared__ float red[kTDownWaves][kTDownRows];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int IPR = inter >> 6;
    const int g = lane & (kTDownLanes - 1), rl = lane / kTDownLanes;
    const int gc = g < IPR ? g : IPR - 1;
    const int row0 = xcd_rank(blockIdx.x, gridDim.x) * kTDownRows;

    const int n_units = k * IPR * 4;
    uint4 hv[kUnitIters][2];
#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kTDownWaves * ui;
        const int uc = u < n_units ? u : 0;
        hv[ui][0] = reinterpret_cast<const uint4*>(h + (size_t)uc * 16)[0];
        hv[ui][1] = reinterpret_cast<const uint4*>(h + (size_t)uc * 16)[1];
    }
    const Q2Proj& Pd = E.p[2];
    uint32_t slot_q[MAXJ];
    uint4 c[MAXJ][ITERS];
    uint16_t sc[MAXJ][ITERS], bi[MAXJ][ITERS];
#pragma unroll
    for (int q = 0; q < MAXJ; ++q) {
        const int jq = wv + kTDownWaves * q;
        slot_q[q] = slots[jq < k ? jq : k - 1];
        const size_t s = slot_q[q] < (uint32_t)n_slots ? slot_q[q] : 0u;
        const uint8_t* wb = Pd.w + s * Pd.w_stride;
        const uint8_t* sb = Pd.s + s * Pd.s_stride;
        const uint8_t* bb = Pd.b + s * Pd.b_stride;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            int row = row0 + it * RPI + rl;
            row = row < hidden ? row : hidden - 1;
            c[q][it] = *reinterpret_cast<const uint4*>(wb + (size_t)row * (inter >> 2) + (size_t)gc * 16);
            sc[q][it] = *reinterpret_cast<const uint16_t*>(sb + ((size_t)row * IPR + gc) * Pd.sb_step);
            bi[q][it] = *reinterpret_cast<const uint16_t*>(bb + ((size_t)row * IPR + gc) * Pd.sb_step);
        }
    }
    const bool weighted = scores != nullptr;
    const uint16_t s_bits = __half_as_ushort((weighted ? scores : h)[lane < k ? lane : 0]);
    const float s_lane = E.scores_bf16 ? __uint_as_float((uint32_t)s_bits << 16) : __half2float(__ushort_as_half(s_bits));
    // the epilogue's operands, loaded now (as in k_q2_down): y_out's current value for mode 2, the
    // residual row for mode 0 (without a residual, y_out's first bytes, unused)
    const int erow = row0 + (tid & (kTDownRows - 1)) < hidden ? row0 + (tid & (kTDownRows - 1)) : hidden - 1;
    const float y_prev = y_out[erow];
    const __half r_prev = (residual ? residual : reinterpret_cast<const __half*>(y_out))[erow];

#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kTDownWaves * ui;
        if (64 * kTDownWaves * ui >= n_units) break;      // block-uniform
        const int uc = u < n_units ? u : 0;
        const int jj = uc / (IPR * 4), gg = (uc >> 2) % IPR;
        stage_pairs(hv[ui][0], hv[ui][1], u < n_units, hp[jj][gg], hc[jj][gg], uc & 3, gg & 7);
    }
    __syncthreads();

    float acc[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) acc[it] = 0.f;
#pragma unroll
    for (int q = 0; q < MAXJ; ++q) {
        const int jq = wv + kTDownWaves * q;
        if (jq >= k) break;
        h2_t P[32];
        const uint4* src = hp[jq][gc];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = src[i ^ (gc & 7)];
            P[4 * i] = as_h2(v.x);
            P[4 * i + 1] = as_h2(v.y);
            P[4 * i + 2] = as_h2(v.z);
            P[4 * i + 3] = as_h2(v.w);
        }
        const float cst = hc[jq][gc][0], sum = hc[jq][gc][1];
        const bool ok = slot_q[q] < (uint32_t)n_slots && g < IPR;
        const float sj = weighted ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s_lane), jq)) : 1.0f;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            float part = ok ? half_bits<BF16>(sc[q][it]) * (q2_group_dot(c[q][it], P) - cst) +
                                  half_bits<BF16>(bi[q][it]) * sum
                            : 0.0f;
            part = lanes::group_sum<kTDownLanes>(part);
            const int rloc = it * RPI + rl;
            if (per_expert == 1) {
                const int row = row0 + rloc;
                if (g == 0 && row < hidden) y_out[(size_t)jq * hidden + row] = part;
            } else {
                acc[it] += sj * part;
            }
        }
    }
    if (per_expert == 1) return;
#pragma unroll
    for (int it = 0; it < ITERS; ++it)
        if (g == 0) red[wv][it * RPI + rl] = acc[it];
    __syncthreads();
    if (tid < kTDownRows) {
        const int row = row0 + tid;
        if (row < hidden) {
            float y = red[0][tid];                      // the waves' sums in a fixed order
#pragma unroll
            for (int w = 1; w < kTDownWaves; ++w) y += red[w][tid];
            if (per_expert == 2) {
                y_out[row] = y_prev + y;
            } else {
                if (residual) y += __half2float(r_prev);
                y_out[row] = y;
            }
        }
    }
}

// The down product's sums (modes 0 and 2) with every lane on one (row, group) pair: a wave covers
// R = 64 / IPR rows at once (IPR = inter / 64 groups per row; 6 rows and 4 idle lanes at inter
// 640, where k_q2t_down's 16-lane rows leave 6 of 16 lanes idle), a block kRDIters such row sets
// (2R rows) for all k experts.  The block's (expert, row set) items are dealt to its waves in turn
// (k = 10: 3 or 2 per wave).  A lane accumulates s_j * (its group's part of row r of expert j)
// over its items in registers; the block then sums over waves and over the row's groups once, in a
// fixed order (run-to-run identical).  With hidden 2560 that is 214 blocks, one per CU, so no CU
// multiplies twice the rows of another.
constexpr int kRDWaves = 8;
constexpr int kRDIters = 2;                                  // row sets per block
constexpr int kRDMaxItems = (MOE_MAX_K * kRDIters + kRDWaves - 1) / kRDWaves;

template <bool BF16>
__global__ __launch_bounds__(64 * kRDWaves) void k_q2t_down_rows(const __half* __restrict__ h, Q2Experts E,
                                                               const uint32_t* __restrict__ slots, int n_slots,
                                                               const __half* __restrict__ scores, int k, int hidden,
                                                               int inter, const __half* __restrict__ residual,
                                                               float* __restrict__ y_out, bool add) {
    constexpr int kUnitIters = (MOE_MAX_K * 1024 / 16 + 64 * kRDWaves - 1) / (64 * kRDWaves);
    __shared__ uint4 hp[MOE_MAX_K][kTDownLanes][8];
    __shared__ float hc[MOE_MAX_K][kTDownLanes][2];
    __shared__ float red[kRDWaves][kRDIters][64];
    __shared__ float red2[kRDIters][64];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int IPR = inter >> 6;
    const int R = 64 / IPR;                                  // rows per row set
    const int rl = lane / IPR, g = lane - rl * IPR;
    const bool lane_ok = rl < R;
    const int rlc = lane_ok ? rl : R - 1;
    const int RB = R * kRDIters;
    const int row0 = xcd_rank(blockIdx.x, gridDim.x) * RB;
    const int n_items = k * kRDIters;

    // h (as in k_q2t_down), then every item's weights, unconditional from clamped addresses
    const int n_units = k * IPR * 4;
    uint4 hv[kUnitIters][2];
#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kRDWaves * ui;
        const int uc = u < n_units ? u : 0;
        hv[ui][0] = reinterpret_cast<const uint4*>(h + (size_t)uc * 16)[0];
        hv[ui][1] = reinterpret_cast<const uint4*>(h + (size_t)uc * 16)[1];
    }
    const Q2Proj& Pd = E.p[2];
    uint32_t slot_q[kRDMaxItems];
    uint4 c[kRDMaxItems];
    uint16_t sc[kRDMaxItems], bi[kRDMaxItems];
#pragma unroll
    for (int q = 0; q < kRDMaxItems; ++q) {
        const int i = wv + kRDWaves * q;
        const int ic = i < n_items ? i : n_items - 1;
        const int j = ic / kRDIters, it = ic - j * kRDIters;
        slot_q[q] = slots[j];
        const size_t s = slot_q[q] < (uint32_t)n_slots ? slot_q[q] : 0u;
        int row = row0 + it * R + rlc;
        row = row < hidden ? row : hidden - 1;
        c[q] = *reinterpret_cast<const uint4*>(Pd.w + s * Pd.w_stride + (size_t)row * (inter >> 2) + (size_t)g * 16);
        sc[q] = *reinterpret_cast<const uint16_t*>(Pd.s + s * Pd.s_stride + ((size_t)row * IPR + g) * Pd.sb_step);
        bi[q] = *reinterpret_cast<const uint16_t*>(Pd.b + s * Pd.b_stride + ((size_t)row * IPR + g) * Pd.sb_step);
    }
    const bool weighted = scores != nullptr;
    const uint16_t s_bits = __half_as_ushort((weighted ? scores : h)[lane < k ? lane : 0]);
    const float s_lane = E.scores_bf16 ? __uint_as_float((uint32_t)s_bits << 16) : __half2float(__ushort_as_half(s_bits));
    // the epilogue's operands (thread t < RB: row row0 + t): y's current value for mode 2, the
    // residual for mode 0 (without a residual, y's first bytes, unused)
    const int erow = row0 + tid < hidden ? row0 + tid : hidden - 1;
    const float y_prev = y_out[erow];
    const __half r_prev = (residual ? residual : reinterpret_cast<const __half*>(y_out))[erow];

#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kRDWaves * ui;
        if (64 * kRDWaves * ui >= n_units) break;      // block-uniform
        const int uc = u < n_units ? u : 0;
        const int jj = uc / (IPR * 4), gg = (uc >> 2) % IPR;
        stage_pairs(hv[ui][0], hv[ui][1], u < n_units, hp[jj][gg], hc[jj][gg], uc & 3, gg & 7);
    }
    __syncthreads();

    float acc0 = 0.f, acc1 = 0.f;
    static_assert(kRDIters == 2, "one accumulator per row set");
#pragma unroll
    for (int q = 0; q < kRDMaxItems; ++q) {
        const int i = wv + kRDWaves * q;
        if (i >= n_items) break;                          // wave-uniform
        const int j = i / kRDIters, it = i - j * kRDIters;
        h2_t P[32];
        const uint4* src = hp[j][g];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint4 v = src[e ^ (g & 7)];
            P[4 * e] = as_h2(v.x);
            P[4 * e + 1] = as_h2(v.y);
            P[4 * e + 2] = as_h2(v.z);
            P[4 * e + 3] = as_h2(v.w);
        }
        const float cst = hc[j][g][0], sum = hc[j][g][1];
        const bool ok = slot_q[q] < (uint32_t)n_slots && lane_ok;
        const float sj = weighted ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s_lane), j)) : 1.0f;
        const float part = ok ? half_bits<BF16>(sc[q]) * (q2_group_dot(c[q], P) - cst) + half_bits<BF16>(bi[q]) * sum
                              : 0.0f;
        if (it == 0) acc0 += sj * part;
        else acc1 += sj * part;
    }
    red[wv][0][lane] = acc0;
    red[wv][1][lane] = acc1;
    __syncthreads();
    if (tid < kRDIters * 64) {                           // over the waves, in order
        const int it = tid >> 6, ln = tid & 63;
        float v = red[0][it][ln];
#pragma unroll
        for (int w = 1; w < kRDWaves; ++w) v += red[w][it][ln];
        red2[it][ln] = v;
    }
    __syncthreads();
    if (tid < RB) {                                      // over the row's groups, in order
        const int it = tid / R, rr = tid - it * R;
        const int row = row0 + tid;
        if (row < hidden) {
            const float* rg = &red2[it][rr * IPR];
            float y = rg[0];
            for (int gi = 1; gi < IPR; ++gi) y += rg[gi];
            if (add) {
                y_out[row] = y_prev + y;
            } else {
                if (residual) y += __half2float(r_prev);
                y_out[row] = y;
            }
        }
    }
}

}  // namespace

bool q2t_shape_ok(const char* who, int k, int hidden, int inter, int group) {
    if (group != 64) { moe_set_error("%s: group=%d unsupported (kernels take group 64)", who, group); return false; }
    if (k <= 0 || k > MOE_MAX_K) { moe_set_error("%s: k=%d out of range 1..%d", who, k, MOE_MAX_K); return false; }
    if (hidden <= 0 || inter <= 0 || hidden % 64 || inter % 64 || hidden > 64 * kTMaxGroups || inter > 64 * kTDownLanes) {
        moe_set_error("%s: hidden=%d inter=%d (multiples of 64, hidden <= %d, inter <= %d)", who, hidden, inter,
                      64 * kTMaxGroups, 64 * kTDownLanes);
        return false;
    }
    return true;
}

Q2Experts q2_experts_from_blob(const uint8_t* pool, size_t stride, const BlobLayout& L) {
    Q2Experts E;
    const size_t w_off[3] = {L.gate_codes, L.up_codes, L.down_codes};
    const size_t sb_off[3] = {L.gate_sb, L.up_sb, L.down_sb};
    for (int p = 0; p < 3; ++p) {
        E.p[p].w = pool + w_off[p];
        E.p[p].s = pool + sb_off[p];
        E.p[p].b = pool + sb_off[p] + 2;
        E.p[p].w_stride = E.p[p].s_stride = E.p[p].b_stride = stride;
        E.p[p].sb_step = 4;
    }
    E.bf16 = 0;
    E.scores_bf16 = 0;
    return E;
}

namespace {

// Lanes per gate/up row: the widest of 32, 16 and 8 whose passes over the row's groups keep at
// least 80% of the lanes busy (one group per lane at hidden 2048: 5.5 us against 7.1 with 8
// lanes; 16 lanes at 2560, 40 groups: 8.0 us against 8.4 with 8 and 9.3 with 32).
template <class F>
void with_lanes_per_row(int hidden, F&& go) {
    const int gpr = hidden / 64;
    auto busy = [&](int lpr) { return 5 * gpr >= 4 * lpr * ((gpr + lpr - 1) / lpr); };
    if (busy(32)) go(std::integral_constant<int, 32>());
    else if (busy(16)) go(std::integral_constant<int, 16>());
    else go(std::integral_constant<int, 8>());
}

}  // namespace

int launch_q2t_gate_up(const __half* x, const Q2Experts& E, int n_slots, const uint32_t* slots, int k, int hidden,
                       int inter, __half* h_out, hipStream_t s) {
    if (!q2t_shape_ok("q2t_gate_up", k, hidden, inter, 64)) return -1;
    if (n_slots <= 0 || !slots || !x || !h_out) { moe_set_error("q2t_gate_up: empty pool or null pointer"); return -1; }
    auto go = [&](auto lc) {
        constexpr int L = decltype(lc)::value;
        constexpr int rpb = 4 * (32 / L);                 // rows per block and projection
        dim3 grid((inter + rpb - 1) / rpb, k);
        if (E.bf16) MOE_LAUNCH(TK_GATE_UP, (k_q2t_gate_up<true, L>), grid, dim3(256), 0, s, x, E, slots, n_slots, hidden, inter, h_out);
        else MOE_LAUNCH(TK_GATE_UP, (k_q2t_gate_up<false, L>), grid, dim3(256), 0, s, x, E, slots, n_slots, hidden, inter, h_out);
    };
    with_lanes_per_row(hidden, go);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_q2t_gate_up_routed(const __half* x, const Q2Experts& E, const uint16_t* logits, int n_exp, int k,
                              int hidden, int inter, uint32_t* ids_out, uint16_t* scores_out, __half* h_out,
                              hipStream_t s) {
    if (!q2t_shape_ok("q2t_gate_up_routed", k, hidden, inter, 64)) return -1;
    if (n_exp <= 0 || n_exp > route::kMaxExperts || k > n_exp) {
        moe_set_error("q2t_gate_up_routed: n_exp=%d (<= %d, >= k=%d)", n_exp, route::kMaxExperts, k);
        return -1;
    }
    if (!x || !logits || !ids_out || !scores_out || !h_out) { moe_set_error("q2t_gate_up_routed: null pointer"); return -1; }
    auto go = [&](auto lc) {
        constexpr int L = decltype(lc)::value;
        constexpr int rpb = 4 * (32 / L);
        dim3 grid((inter + rpb - 1) / rpb, k);
        if (E.bf16)
            MOE_LAUNCH(TK_GATE_UP, (k_q2t_gate_up_routed<true, L>), grid, dim3(256), 0, s, x, E, logits, n_exp, k, hidden,
                       inter, ids_out, scores_out, h_out);
        else
            MOE_LAUNCH(TK_GATE_UP, (k_q2t_gate_up_routed<false, L>), grid, dim3(256), 0, s, x, E, logits, n_exp, k, hidden,
                       inter, ids_out, scores_out, h_out);
    };
    with_lanes_per_row(hidden, go);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_q2t_down(const __half* h, const Q2Experts& E, int n_slots, const uint32_t* slots, const __half* scores,
                    int k, int hidden, int inter, const __half* residual, float* y_out, int per_expert, hipStream_t s) {
    if (!q2t_shape_ok("q2t_down", k, hidden, inter, 64)) return -1;
    if (per_expert < 0 || per_expert > 2) { moe_set_error("q2t_down: mode %d (0 sum, 1 per expert, 2 add)", per_expert); return -1; }
    if (n_slots <= 0 || !slots || !h || !y_out) { moe_set_error("q2t_down: empty pool or null pointer"); return -1; }
    hipStream_t st = s;
    if (per_expert != 1) {                 // the sums: every lane of a wave on a (row, group)
        const int ipr = inter >> 6, rb = (64 / ipr) * kRDIters;
        const dim3 grid((hidden + rb - 1) / rb);
        if (E.bf16)
            MOE_LAUNCH(TK_DOWN, (k_q2t_down_rows<true>), grid, dim3(64 * kRDWaves), 0, st, h, E, slots, n_slots, scores,
                       k, hidden, inter, residual, y_out, per_expert == 2);
        else
            MOE_LAUNCH(TK_DOWN, (k_q2t_down_rows<false>), grid, dim3(64 * kRDWaves), 0, st, h, E, slots, n_slots, scores,
                       k, hidden, inter, residual, y_out, per_expert == 2);
    } else {
        const dim3 grid((hidden + kTDownRows - 1) / kTDownRows);
        if (E.bf16)
            MOE_LAUNCH(TK_DOWN, (k_q2t_down<true>), grid, dim3(64 * kTDownWaves), 0, st, h, E, slots, n_slots, scores, k,
                       hidden, inter, residual, y_out, per_expert);
        else
            MOE_LAUNCH(TK_DOWN, (k_q2t_down<false>), grid, dim3(64 * kTDownWaves), 0, st, h, E, slots, n_slots, scores, k,
                       hidden, inter, residual, y_out, per_expert);
    }
    HIP_TRY(hipGetLastError());
    return 0;
}
