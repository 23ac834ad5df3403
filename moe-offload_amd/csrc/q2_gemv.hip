// Q2 (2-bit affine, group 64) gather-GEMV for batch-1 SwitchGLU decode on gfx950.
//
// Reference semantics: mlx-qwen38/loader.py:557-564,964-965 (`_slot_glu` = gather_qmm x3 over the
// slot pool + SwiGLU, then the score-weighted sum), cpp/src/layers.cpp:343-362,
// cpp/src/kernels.cpp:1027-1040,1090-1094:  y = sum_j s_j * D_j( silu(G_j x) * (U_j x) ),
// W = scale * q + bias per group of 64 inputs, q = 2-bit codes, 16 per uint32, LSB first.
//
// Data path.  One 16-byte load per lane is exactly one group (64 codes) of one weight row, so
// a wave reads whole rows with fully coalesced 128-bit loads; the matching (scale, bias) pair
// is one 32-bit load.  Codes are expanded in registers without integer->float conversions:
// OR-ing a code pair into the mantissa of fp16 1024.0 gives the exact halves 1024 + c*4^p,
// which feed v_dot2_f32_f16 against the matching activation pair.  Per 32-bit word that is
// 9 bit operations + 8 dot2 for 16 codes.  With 5 accumulators (one per power 4^p):
//     sum_i c_i x_i = sum_p 4^-p A_p - 1024 * sum_i x_i 4^-p(i)
// and the second term is a per-(vector, group) constant computed once.
// Accumulation is fp32; the activation vector is fp16 (x) or fp16-rounded (h).
//
// Kernels
//   k_q2_gate_up<GPR>: rows of gate and up for one selected expert; lanes 0-31 gate, 32-63 up,
//                      GPR = hidden/64 lanes per row.  Writes h = silu(g)*u as fp16 [k][inter].
//   k_q2_down<GPR>:    8 output rows per block x all k experts (8 waves split the experts);
//                      h is staged in LDS in dot2 pair order; the block reduces over experts in
//                      a fixed order and writes y = residual + sum_j s_j y_j (fp32, mode 0), the
//                      per-expert rows (mode 1), or adds sum_j s_j y_j to y (mode 2: the second
//                      half of a hit/miss split).
#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "moe_common.h"
#include "q2_dot.h"
#include "route_select.h"

namespace {

using namespace q2dot;

// Row iterations per wave (each covers 32/GPR rows of each projection).  The routed kernel takes 2:
// every block runs the selection, so fewer, larger blocks pay it less often (resident decode 1,301
// tok/s against 1,226 with 1).  The plain kernel takes 1: at top-10 its 5,120 waves give every
// SIMD of the 256 CUs the same count, where 2,560 leave some with 3 and others with 2 (4.35 ->
// 3.98 us back to back with the decode's inputs).
template <bool ROUTED>
constexpr int gu_rows_per_iter() { return ROUTED ? 2 : 1; }

// Rows of gate and up for one selected expert.  ROUTED: the block first selects the top-k
// experts from the router's logits itself (the router's rule, bit for bit) over a pool holding
// every expert (slot = id); block (0, 0) also writes the ids and scores.  The selection runs
// while the activation loads are in flight; it replaces the router's last-block hand-off
// (a device-scope counter and a second read of every logit) on the resident path.
template <int GPR, bool ROUTED>
__device__ __forceinline__ void gate_up_body(
    const __half* __restrict__ x, const uint8_t* __restrict__ pool, size_t stride,
    const uint32_t* __restrict__ slots, int n_slots, int inter, const BlobLayout& L, __half* __restrict__ h_out,
    const float* __restrict__ logits, int k, uint32_t* __restrict__ ids_out, __half* __restrict__ scores_out) {
    constexpr int RPI = 32 / GPR;                       // rows per wave instruction
    constexpr int kGuRowsPerIter = gu_rows_per_iter<ROUTED>();
    constexpr int ROWS_PER_WAVE = RPI * kGuRowsPerIter;
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = blockIdx.y;
    const int proj = lane >> 5, sub = lane & 31;
    const int rl = sub / GPR, g = sub % GPR;
    const int row_base = (blockIdx.x * 4 + wv) * ROWS_PER_WAVE;

    // The activation vector first, one 16-value unit per thread (hidden / 16 <= 256 units): it
    // comes from L2, and loads complete in issue order, so staging its pairs in LDS overlaps the
    // weight loads' flight instead of following them.  The block stages x once; every lane then
    // reads its group's 32 pairs from LDS.
    __shared__ uint4 xp[32][8];                         // per group of 64: 32 dot2 pairs
    __shared__ float xc[32][2];
    const int tid = threadIdx.x;
    const int n_units = GPR * 4;
    const int uc = tid < n_units ? tid : 0;
    const uint4 xlo = reinterpret_cast<const uint4*>(x)[2 * uc];
    const uint4 xhi = reinterpret_cast<const uint4*>(x)[2 * uc + 1];
    __builtin_amdgcn_sched_barrier(0);

    uint32_t slot;
    uint32_t top_key = 0;                              // routed, wave 0: lane r's r-th pick
    float lraw[route::kPer];
    __shared__ uint32_t keys[ROUTED ? route::kMaxExperts : 1];
    __shared__ double reds[4];
    __shared__ uint32_t sel[MOE_MAX_K];
    __shared__ uint32_t top1;
    __shared__ int clash;
    const int n_pad = ((n_slots + 63) / 64) * 64;
    if constexpr (ROUTED) {
        // rank by logit (k + 1 picks) so that the weight loads go out before the softmax
        // (route_select.h: spec_keys / spec_check)
#pragma unroll
        for (int i = 0; i < route::kPer; ++i) {
            const int e = tid + route::kThreads * i;
            lraw[i] = logits[e < n_slots ? e : 0];
        }
        route::spec_keys<false>(lraw, n_slots, keys);
        if (wv == 0) {
            top_key = route::wave_topn(keys, 0, n_pad, k + 1, lane);
            if (lane < k) sel[k - 1 - lane] = top_key & 0xFFFFu;
            if (lane == 0) top1 = top_key;
        }
        __syncthreads();
        slot = sel[j];
    } else {
        slot = slots[j];
    }
    const size_t row_bytes = (size_t)GPR * 16;

    // Every load is unconditional from a clamped in-range row; nothing is selected on arrival
    // (a load whose value is masked right away is sunk into a branch and waited for there).
    bool ok;
    uint4 c[kGuRowsPerIter];
    uint32_t sb[kGuRowsPerIter];
    auto load_w = [&](uint32_t sl) {
        ok = sl < (uint32_t)n_slots;                   // an invalid slot yields h = 0
        const uint8_t* blob = pool + (size_t)(ok ? sl : 0) * stride;
        const uint8_t* codes = blob + (proj ? L.up_codes : L.gate_codes);
        const uint32_t* sbv = reinterpret_cast<const uint32_t*>(blob + (proj ? L.up_sb : L.gate_sb));
#pragma unroll
        for (int it = 0; it < kGuRowsPerIter; ++it) {
            int row = row_base + it * RPI + rl;
            row = row < inter ? row : inter - 1;
            c[it] = *reinterpret_cast<const uint4*>(codes + (size_t)row * row_bytes + g * 16);
            sb[it] = sbv[(size_t)row * GPR + g];
        }
    };
    load_w(slot);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ROUTED) {
        // the rule's gates for the k + 1 picks while the weights fly; on a clash the full rule
        // (fallback_keys) and, if this block's expert changed, its weights again
        double lv[route::kPer], sum;
        uint32_t exact = 0;
        const double mx = (double)route::logit_from_order<false>(top1 >> 16);
        if (route::spec_check<false>(lraw, n_slots, k, top_key, mx, reds, &clash, lv, sum, exact)) {
            route::fallback_keys<false>(lv, sum, n_slots, keys);
            if (wv == 0) {
                exact = route::wave_topn(keys, 0, n_pad, k, lane);
                if (lane < k) sel[k - 1 - lane] = exact & 0xFFFFu;
            }
            __syncthreads();
            const uint32_t s2 = sel[j];
            if (s2 != slot) {                          // block-uniform
                slot = s2;
                load_w(slot);
            }
        }
        if (wv == 0 && blockIdx.x == 0 && blockIdx.y == 0) {
            uint32_t id;
            __half sc;
            const int pos = route::topk_scores(exact, k, lane, id, sc);
            if (pos >= 0) {
                ids_out[pos] = id;
                scores_out[pos] = sc;
            }
        }
    }

    stage_pairs(xlo, xhi, tid < n_units, xp[uc >> 2], xc[uc >> 2], uc & 3, (uc >> 2) & 7);
    __builtin_amdgcn_sched_barrier(0);                  // no weight use ahead of the barrier
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    h2_t P[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4 v = xp[g][i ^ (g & 7)];
        P[4 * i] = as_h2(v.x);
        P[4 * i + 1] = as_h2(v.y);
        P[4 * i + 2] = as_h2(v.z);
        P[4 * i + 3] = as_h2(v.w);
    }
    const float cst = xc[g][0], sum = xc[g][1];

    float part[kGuRowsPerIter];
#pragma unroll
    for (int it = 0; it < kGuRowsPerIter; ++it) part[it] = sb_apply(sb[it], q2_group_dot(c[it], P), cst, sum);
    // row sums over the GPR lanes of each row (DPP / permlane, no LDS round trips)
#pragma unroll
    for (int it = 0; it < kGuRowsPerIter; ++it) part[it] = lanes::group_sum<GPR>(part[it]);
#pragma unroll
    for (int it = 0; it < kGuRowsPerIter; ++it) {
        float gt, up;                                   // gate row (lanes 0-31), up row (32-63)
        lanes::halves(part[it], gt, up);
        const int row = row_base + it * RPI + rl;
        if (proj == 0 && g == 0 && row < inter) {
            const float hval = ok ? gt / (1.0f + __expf(-gt)) * up : 0.0f;
            h_out[(size_t)j * inter + row] = __float2half_rn(hval);
        }
    }
}

template <int GPR>
__global__ __launch_bounds__(256) void k_q2_gate_up(
    const __half* __restrict__ x, const uint8_t* __restrict__ pool, size_t stride,
    const uint32_t* __restrict__ slots, int n_slots, int inter, BlobLayout L, __half* __restrict__ h_out) {
    gate_up_body<GPR, false>(x, pool, stride, slots, n_slots, inter, L, h_out, nullptr, 0, nullptr, nullptr);
}

template <int GPR>
__global__ __launch_bounds__(256) void k_q2_gate_up_routed(
    const __half* __restrict__ x, const float* __restrict__ logits, int n_exp, int k, const uint8_t* __restrict__ pool,
    size_t stride, int inter, BlobLayout L, uint32_t* __restrict__ ids_out, __half* __restrict__ scores_out,
    __half* __restrict__ h_out) {
    gate_up_body<GPR, true>(x, pool, stride, nullptr, n_exp, inter, L, h_out, logits, k, ids_out, scores_out);
}

constexpr int kDownRows = 8;      // output rows per block (one wave instruction at GPR = 8)
// Waves per down block.  With 8, a wave multiplies 1-2 of the top-10 experts instead of 2-3: its
// chain of dependent dot products after the loads land is shorter (resident decode 1,294 tok/s
// against 1,254 with 4 waves; back to back, where one launch's tail hides under the next, both
// take 5.3-5.5 us).
constexpr int kDownWaves = 8;
static_assert((kDownRows & (kDownRows - 1)) == 0, "the epilogue row of a thread is tid & (kDownRows - 1)");

template <int GPR>
__global__ __launch_bounds__(64 * kDownWaves) void k_q2_down(
    const __half* __restrict__ h, const uint8_t* __restrict__ pool, size_t stride,
    const uint32_t* __restrict__ slots, int n_slots, const __half* __restrict__ scores, int k, int hidden,
    BlobLayout L, const __half* __restrict__ residual, float* __restrict__ y_out, int per_expert) {
    constexpr int LPR = GPR;                       // lanes per row
    constexpr int RPI = 64 / LPR;                  // rows per wave instruction
    constexpr int ITERS = (kDownRows + RPI - 1) / RPI;
    constexpr int MAXJ = (MOE_MAX_K + kDownWaves - 1) / kDownWaves;   // experts per wave
    constexpr int kUnits = MOE_MAX_K * GPR * 4;    // 16-value units of h at the largest k
    constexpr int kUnitIters = (kUnits + 64 * kDownWaves - 1) / (64 * kDownWaves);
    __shared__ uint4 hp[MOE_MAX_K][GPR][8];        // per (expert, group): 32 dot2 pairs
    __shared__ float hc[MOE_MAX_K][GPR][2];
    __shared__ float red[kDownWaves][kDownRows];

    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane % LPR, rl = lane / LPR;
    const int row0 = blockIdx.x * kDownRows;

    // h[k][inter] -> LDS as dot2 pairs plus the per-(expert, group) constants.  Unit u = 16
    // values 16w..16w+15 of group gg of expert jj (w = u % 4): two 16-byte loads give its 8
    // pairs (h[16w + p], h[16w + p + 8]); the 4 units of a group sit on 4 adjacent lanes, which
    // sum their partial constants with two DPP steps.
    const int n_units = k * GPR * 4;
    uint4 hv[kUnitIters][2];
#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kDownWaves * ui;
        const int uc = u < n_units ? u : 0;
        const __half* src = h + (size_t)uc * 16;          // units are contiguous in h
        hv[ui][0] = reinterpret_cast<const uint4*>(src)[0];
        hv[ui][1] = reinterpret_cast<const uint4*>(src)[1];
    }
    // This wave's weight loads (experts wv, wv + kDownWaves, ...), all unconditional from clamped
    // in-range addresses: a value loaded inside a branch and merged with another value at the
    // join is waited for in the branch, which would serialise the round trips.  A position past
    // k re-reads expert k-1's rows, which another wave of the block loads too (an L2 hit); the
    // scores are one lane load, read out after the staging barrier.
    uint32_t slot_q[MAXJ];
#pragma unroll
    for (int q = 0; q < MAXJ; ++q) {
        const int j = wv + kDownWaves * q;
        slot_q[q] = slots[j < k ? j : k - 1];
    }
    uint4 c[MAXJ][ITERS];
    uint32_t sb[MAXJ][ITERS];
#pragma unroll
    for (int q = 0; q < MAXJ; ++q) {
        const uint32_t slot = slot_q[q] < (uint32_t)n_slots ? slot_q[q] : 0u;
        const uint8_t* blob = pool + (size_t)slot * stride;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            int row = row0 + it * RPI + rl;
            row = row < hidden ? row : hidden - 1;
            c[q][it] = *reinterpret_cast<const uint4*>(blob + L.down_codes + (size_t)row * GPR * 16 + g * 16);
            sb[q][it] = reinterpret_cast<const uint32_t*>(blob + L.down_sb)[(size_t)row * GPR + g];
        }
    }
    const bool weighted = scores != nullptr;
    const float s_lane = __half2float((weighted ? scores : h)[lane < k ? lane : 0]);
    // The epilogue's operands, loaded here so that no round trip follows the reduction: y_out's
    // current value (mode 2 adds to it) and the residual row (mode 0).  Both unconditional from a
    // clamped row; without a residual the load reads y_out's first bytes and is not used.
    const int erow = row0 + (tid & (kDownRows - 1)) < hidden ? row0 + (tid & (kDownRows - 1)) : hidden - 1;
    const float y_prev = y_out[erow];
    const __half r_prev = (residual ? residual : reinterpret_cast<const __half*>(y_out))[erow];

#pragma unroll
    for (int ui = 0; ui < kUnitIters; ++ui) {
        const int u = tid + 64 * kDownWaves * ui;
        if (64 * kDownWaves * ui >= n_units) break;   // block-uniform: no lane of this pass is valid
        const int uc = u < n_units ? u : 0;
        const int jj = uc / (GPR * 4), gg = (uc >> 2) % GPR;
        stage_pairs(hv[ui][0], hv[ui][1], u < n_units, hp[jj][gg], hc[jj][gg], uc & 3, gg & 7);
    }
    __syncthreads();

    float acc[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) acc[it] = 0.f;
#pragma unroll
    for (int q = 0; q < MAXJ; ++q) {
        const int j = wv + kDownWaves * q;
        if (j >= k) break;
        h2_t P[32];
        const uint4* src = hp[j][g];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = src[i ^ (g & 7)];
            P[4 * i] = as_h2(v.x);
            P[4 * i + 1] = as_h2(v.y);
            P[4 * i + 2] = as_h2(v.z);
            P[4 * i + 3] = as_h2(v.w);
        }
        const float cst = hc[j][g][0], sum = hc[j][g][1];
        const bool ok = slot_q[q] < (uint32_t)n_slots;  // an invalid slot contributes 0
        const float sj = weighted ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s_lane), j)) : 1.0f;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            float part = ok ? sb_apply(sb[q][it], q2_group_dot(c[q][it], P), cst, sum) : 0.0f;
            part = lanes::group_sum<LPR>(part);
            const int rloc = it * RPI + rl;
            if (per_expert == 1) {
                const int row = row0 + rloc;
                if (g == 0 && rloc < kDownRows && row < hidden) y_out[(size_t)j * hidden + row] = part;
            } else {
                acc[it] += sj * part;
            }
        }
    }
    if (per_expert == 1) return;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int rloc = it * RPI + rl;
        if (g == 0 && rloc < kDownRows) red[wv][rloc] = acc[it];
    }
    __syncthreads();
    if (tid < kDownRows) {
        int row = row0 + tid;
        if (row < hidden) {
            float y = red[0][tid];                      // the waves' sums in a fixed order
#pragma unroll
            for (int w = 1; w < kDownWaves; ++w) y += red[w][tid];
            if (per_expert == 2) {
                y_out[row] = y_prev + y;
            } else {
                if (residual) y += __half2float(r_prev);
                y_out[row] = y;
            }
        }
    }
}

template <int GPR>
int gate_up_t(const __half* x, const uint8_t* pool, size_t stride, const uint32_t* slots, int n_slots, int k,
              int inter, BlobLayout L, __half* h_out, hipStream_t s) {
    constexpr int rows_per_block = 4 * (32 / GPR) * gu_rows_per_iter<false>();
    dim3 grid((inter + rows_per_block - 1) / rows_per_block, k);
    MOE_LAUNCH(TK_GATE_UP, (k_q2_gate_up<GPR>), grid, dim3(256), 0, s, x, pool, stride, slots, n_slots, inter, L, h_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int GPR>
int gate_up_routed_t(const __half* x, const float* logits, int n_exp, int k, const uint8_t* pool, size_t stride,
                     int inter, BlobLayout L, uint32_t* ids_out, __half* scores_out, __half* h_out, hipStream_t s) {
    constexpr int rows_per_block = 4 * (32 / GPR) * gu_rows_per_iter<true>();
    dim3 grid((inter + rows_per_block - 1) / rows_per_block, k);
    MOE_LAUNCH(TK_GATE_UP, (k_q2_gate_up_routed<GPR>), grid, dim3(256), 0, s, x, logits, n_exp, k, pool, stride, inter, L,
               ids_out, scores_out, h_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int GPR>
int down_t(const __half* h, const uint8_t* pool, size_t stride, const uint32_t* slots, int n_slots,
           const __half* scores, int k, int hidden, BlobLayout L, const __half* residual,
           float* y_out, int per_expert, hipStream_t s) {
    dim3 grid((hidden + kDownRows - 1) / kDownRows);
    MOE_LAUNCH(TK_DOWN, (k_q2_down<GPR>), grid, dim3(64 * kDownWaves), 0, s, h, pool, stride, slots, n_slots, scores, k,
                       hidden, L, residual, y_out, per_expert);
    HIP_TRY(hipGetLastError());
    return 0;
}

bool check_shape(const char* who, int k, int hidden, int inter, int group) {
    if (group != 64) { moe_set_error("%s: group=%d unsupported (kernels take group 64)", who, group); return false; }
    if (k <= 0 || k > MOE_MAX_K) { moe_set_error("%s: k=%d out of range 1..%d", who, k, MOE_MAX_K); return false; }
    if (hidden % 64 || inter % 64 || hidden <= 0 || inter <= 0) {
        moe_set_error("%s: hidden=%d inter=%d must be positive multiples of 64", who, hidden, inter);
        return false;
    }
    return true;
}

}  // namespace

int launch_q2_gate_up(const __half* x, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots,
                      int k, int hidden, int inter, int group, __half* h_out, hipStream_t s) {
    if (!check_shape("q2_gate_up", k, hidden, inter, group)) return -1;
    if (n_slots <= 0 || !pool || !slots || !x || !h_out) { moe_set_error("q2_gate_up: empty pool or null pointer"); return -1; }
    BlobLayout L = blob_layout(hidden, inter, group);
    if (stride < L.bytes) { moe_set_error("q2_gate_up: expert stride %zu < blob bytes %zu", stride, L.bytes); return -1; }
    switch (hidden / 64) {
        case 1: return gate_up_t<1>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        case 2: return gate_up_t<2>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        case 4: return gate_up_t<4>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        case 8: return gate_up_t<8>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        case 16: return gate_up_t<16>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        case 32: return gate_up_t<32>(x, pool, stride, slots, n_slots, k, inter, L, h_out, s);
        default:   // other multiples of 64: the tensor-form kernel over the blob's tensors
            return launch_q2t_gate_up(x, q2_experts_from_blob(pool, stride, L), n_slots, slots, k, hidden, inter, h_out, s);
    }
}

int launch_q2_gate_up_routed(const __half* x, const float* logits, int n_exp, int k, const uint8_t* pool,
                             size_t stride, int hidden, int inter, int group, uint32_t* ids_out, __half* scores_out,
                             __half* h_out, hipStream_t s) {
    if (!check_shape("q2_gate_up_routed", k, hidden, inter, group)) return -1;
    if (n_exp <= 0 || n_exp > route::kMaxExperts || k > n_exp) {
        moe_set_error("q2_gate_up_routed: n_exp=%d (<= %d, >= k=%d)", n_exp, route::kMaxExperts, k);
        return -1;
    }
    if (!pool || !x || !logits || !ids_out || !scores_out || !h_out) { moe_set_error("q2_gate_up_routed: null pointer"); return -1; }
    BlobLayout L = blob_layout(hidden, inter, group);
    if (stride < L.bytes) { moe_set_error("q2_gate_up_routed: expert stride %zu < blob bytes %zu", stride, L.bytes); return -1; }
    switch (hidden / 64) {
        case 1: return gate_up_routed_t<1>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        case 2: return gate_up_routed_t<2>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        case 4: return gate_up_routed_t<4>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        case 8: return gate_up_routed_t<8>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        case 16: return gate_up_routed_t<16>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        case 32: return gate_up_routed_t<32>(x, logits, n_exp, k, pool, stride, inter, L, ids_out, scores_out, h_out, s);
        default: moe_set_error("q2_gate_up_routed: hidden=%d unsupported (64*{1,2,4,8,16,32})", hidden); return -1;
    }
}

int launch_q2_down(const __half* h, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots,
                   const __half* scores, int k, int hidden, int inter, int group,
                   const __half* residual, float* y_out, int per_expert, hipStream_t s) {
    if (!check_shape("q2_down", k, hidden, inter, group)) return -1;
    if (per_expert < 0 || per_expert > 2) { moe_set_error("q2_down: mode %d (0 sum, 1 per expert, 2 add)", per_expert); return -1; }
    if (n_slots <= 0 || !pool || !slots || !h || !y_out) { moe_set_error("q2_down: empty pool or null pointer"); return -1; }
    BlobLayout L = blob_layout(hidden, inter, group);
    if (stride < L.bytes) { moe_set_error("q2_down: expert stride %zu < blob bytes %zu", stride, L.bytes); return -1; }
    switch (inter / 64) {
        case 1: return down_t<1>(h, pool, stride, slots, n_slots, scores, k, hidden, L, residual, y_out, per_expert, s);
        case 2: return down_t<2>(h, pool, stride, slots, n_slots, scores, k, hidden, L, residual, y_out, per_expert, s);
        case 4: return down_t<4>(h, pool, stride, slots, n_slots, scores, k, hidden, L, residual, y_out, per_expert, s);
        case 8: return down_t<8>(h, pool, stride, slots, n_slots, scores, k, hidden, L, residual, y_out, per_expert, s);
        case 16: return down_t<16>(h, pool, stride, slots, n_slots, scores, k, hidden, L, residual, y_out, per_expert, s);
        default:   // other multiples of 64: the tensor-form kernel over the blob's tensors
            return launch_q2t_down(h, q2_experts_from_blob(pool, stride, L), n_slots, slots, scores, k, hidden, inter,
                                   residual, y_out, per_expert, s);
    }
}
