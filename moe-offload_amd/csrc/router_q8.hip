// The real checkpoint's router and next-layer predictor on gfx950: 8-bit affine quantized linear
// layers (bits 8, group 64: W = scale * q + bias per 64 inputs, q a byte, 4 per u32 LSB first;
// scales and biases bf16) over a bf16 hidden vector, then the router rule in bf16.
//
// Reference: loader.py:903-908 (gate -> softmax(precise) -> top-k -> renormalise), loader.py:
// 237-242 + 950-958 (predictor: top-m sorted by descending logit), cpp/src/kernels.cpp:997-1019
// (QLinear::forward: quantized_matmul, affine, the layer's bits and group size).
//
// Logits are accumulated in fp64 and rounded to bf16 once (a correctly rounded quantized dot
// product; MLX's own kernel accumulates in fp32 and rounds one logit of the reference fixture
// one ulp lower).  Per 16-code unit u of a row: d_u = sum_i x_i q_i (fp64, exact for the inputs'
// exponent spreads of a hidden vector), logit += s_g d_u + b_g sx_u with sx_u = sum_i x_i of
// that unit (fp64, computed once per launch by the block).
//
// Selection (the block that finishes last, as in k_router): route mode (k > 0) gates =
// bf16(softmax in fp64), the top k by (gate bits, id) with equal gates ordered by id, scores =
// bf16(g / s) with s the left-to-right bf16-rounded sum in ascending order; predict mode (m > 0)
// the top m logits sorted by descending value, equal values by ascending id.
#include <hip/hip_runtime.h>

#include "lane_reduce.h"
#include "moe_common.h"
#include "moe_offload.h"
#include "norm_f64.h"
#include "route_select.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRows = kThreads / 64;          // one wave per weight row
constexpr int kMaxHidden = 4096;
constexpr int kMaxUnits = kMaxHidden / 16;    // 16-code units per row

using route::bf16_to_f32;
using route::f32_to_bf16_bits;
using route::f64_to_bf16_bits;
// Order-preserving map of a bf16 value to 16 bits (-0 folded onto +0).
__device__ __forceinline__ uint32_t bf16_order(uint32_t b) {
    if (b == 0x8000u) b = 0;
    return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

// NORM: the input is the previous layer's output h (fp32), normalised by every block (the bf16
// RMSNorm of norm_f64.h, bit-identical to moe_rmsnorm_bf16) while its weight loads fly; block 0
// also writes x as bf16 and as fp16 (the expert kernels' input and residual).  A compile-time
// choice, so that no branch lets the compiler sink the input loads behind the weight loads.
template <int NU, bool NORM>
__global__ __launch_bounds__(kThreads) void k_router_q8(
    const uint16_t* __restrict__ x, const float* __restrict__ h_in, const uint16_t* __restrict__ norm_w, float eps,
    uint16_t* __restrict__ xb_out, __half* __restrict__ xh_out,
    const uint32_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, int hidden, int n_rows, int k, int m, float* __restrict__ scratch,
    unsigned* __restrict__ counter, uint32_t* __restrict__ ids_out, uint16_t* __restrict__ scores_out,
    int32_t* __restrict__ pred_out, uint16_t* __restrict__ logits_out) {
    __shared__ __align__(16) float xf[kMaxHidden];
    __shared__ double sx[kMaxUnits];
    __shared__ double redn[kThreads / 64];
    __shared__ int is_last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int units = hidden / 16, groups = hidden / 64;
    const int row = blockIdx.x * kRows + wv;
    const int rc = row < n_rows ? row : n_rows - 1;             // a row past the end reads the last

    norm64::NormIn nin;
    if constexpr (NORM) norm64::load(nin, h_in, reinterpret_cast<const __half*>(norm_w), hidden);
    __builtin_amdgcn_sched_barrier(0);                            // the input loads ahead of the weights

    // weight loads first (unconditional, clamped): unit u = lane + 64 c of row rc
    uint4 q[NU];
    uint32_t sb[NU];
#pragma unroll
    for (int c = 0; c < NU; ++c) {
        const int u = lane + 64 * c, uc = u < units ? u : units - 1;
        q[c] = reinterpret_cast<const uint4*>(codes + (size_t)rc * (hidden / 4))[uc];
        const size_t gi = (size_t)rc * groups + uc / 4;
        sb[c] = (uint32_t)scales[gi] | ((uint32_t)biases[gi] << 16);
    }
    __builtin_amdgcn_sched_barrier(0);                            // every weight load issued before anything waits
    // the input, as fp32 (exact), and each unit's input sum
    if constexpr (NORM) {
        const bool first = blockIdx.x == 0;
        norm64::finish_bf16(nin, norm_w != nullptr, eps, hidden, first ? xb_out : nullptr, first ? xh_out : nullptr,
                            redn, xf);
    } else {
        for (int i = tid; i < hidden; i += kThreads) xf[i] = bf16_to_f32(x[i]);
    }
    __syncthreads();
    for (int u = tid; u < units; u += kThreads) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += (double)xf[16 * u + i];
        sx[u] = s;
    }
    __syncthreads();

    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < NU; ++c) {
        const int u = lane + 64 * c;
        if (u >= units) continue;
        const uint32_t w4[4] = {q[c].x, q[c].y, q[c].z, q[c].w};
        double d = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b) d += (double)xf[16 * u + 4 * j + b] * (double)((w4[j] >> (8 * b)) & 0xFFu);
        acc += (double)bf16_to_f32(sb[c] & 0xFFFFu) * d + (double)bf16_to_f32(sb[c] >> 16) * sx[u];
    }
    acc = lanes::wave_sum_f64(acc);
    if (lane == 0 && row < n_rows) {
        const uint16_t lb = f64_to_bf16_bits(acc);
        if (logits_out) logits_out[row] = lb;
        __hip_atomic_store(&scratch[row], bf16_to_f32(lb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (k <= 0 && m <= 0) return;

    // ---- the block that finishes last selects (see k_router) ---------------------------------
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) is_last = (__hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1);
    __syncthreads();
    if (!is_last) return;

    __shared__ uint32_t keys[route::kMaxExperts];
    __shared__ double redm[kThreads / 64], reds[kThreads / 64];
    constexpr int kPer = route::kPer;
    const int n_pad = ((n_rows + 63) / 64) * 64;
    float lraw[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        lraw[i] = __hip_atomic_load(&scratch[e < n_rows ? e : 0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (k > 0) {
        // gates = bf16(softmax in fp64), keys (gate bits << 16 | id), the top k, scores = bf16(g / s)
        // with s the left-to-right bf16-rounded sum in ascending order: the router rule in bf16,
        // the same code as the routed tensor-form gate/up (k_q2t_gate_up_routed)
        route::gate_keys<true>(lraw, n_rows, keys, redm, reds);
        if (wv == 0) {
            const uint32_t mine = route::wave_topn(keys, 0, n_pad, k, lane);   // lane j: j-th largest
            uint32_t id;
            uint16_t sc;
            const int pos = route::topk_score_bits<true>(mine, k, lane, id, sc);
            if (pos >= 0) {
                ids_out[pos] = id;
                scores_out[pos] = sc;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = tid + kThreads * i;
            if (e < n_pad)
                keys[e] = e < n_rows ? ((bf16_order(f32_to_bf16_bits(lraw[i])) << 16) | (uint32_t)e) : 0u;
        }
        __syncthreads();
        if (wv == 0) {
            const uint32_t mine = route::wave_topn(keys, 0, n_pad, m, lane);
            // descending (value, id); within a run of equal values the ids go ascending: lane r
            // takes the id of its mirror position in the run
            const uint32_t val = mine >> 16;
            int first = lane, last = lane;
            for (int q2 = 0; q2 < m; ++q2) {
                const uint32_t vq = (uint32_t)__builtin_amdgcn_readlane((int)val, q2);
                if (vq == val && q2 < first) first = q2;
                if (vq == val && q2 > last) last = q2;
            }
            const int id = __shfl((int)(mine & 0xFFFFu), first + last - lane, 64);
            if (lane < m) pred_out[lane] = id;
        }
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" uint64_t moe_router_q8_workspace_bytes(int n_rows) {
    return (uint64_t)(n_rows > 0 ? n_rows : 0) * sizeof(float) + 256;
}

namespace {

int launch_router_q8(const void* x, const float* h_in, const void* norm_w, float eps, void* xb_out, void* xh_out,
                     const uint32_t* codes, const void* scales, const void* biases, int hidden, int n_rows, int group,
                     int k, int m, void* workspace, uint32_t* ids_out, void* scores_out, int32_t* pred_out,
                     void* logits_out, void* stream) {
    const char* who = h_in ? "router_q8_norm" : "router_q8";
    if (group != 64 || hidden <= 0 || hidden % 64 || hidden > kMaxHidden) {
        moe_set_error("%s: hidden=%d group=%d (group 64, hidden a multiple of 64 up to %d)", who, hidden, group,
                      kMaxHidden);
        return -1;
    }
    if (n_rows <= 0 || n_rows > route::kMaxExperts) {
        moe_set_error("%s: %d rows (1..%d)", who, n_rows, route::kMaxExperts);
        return -1;
    }
    if ((k > 0) == (m > 0) && (k > 0 || m > 0)) {
        moe_set_error("%s: route (k > 0) or predict (m > 0), not both", who);
        return -1;
    }
    if (k > MOE_MAX_K || k > n_rows || m > 64 || m > n_rows) {
        moe_set_error("%s: k=%d m=%d for %d rows (k <= %d, m <= 64)", who, k, m, n_rows, MOE_MAX_K);
        return -1;
    }
    if ((!x && !h_in) || !codes || !scales || !biases || !workspace || (k > 0 && (!ids_out || !scores_out)) ||
        (m > 0 && !pred_out) || (k <= 0 && m <= 0 && !logits_out)) {
        moe_set_error("%s: null pointer", who);
        return -1;
    }
    float* scratch = (float*)workspace;
    unsigned* counter = (unsigned*)((uint8_t*)workspace + (size_t)n_rows * sizeof(float));
    const int units = hidden / 16, nu = (units + 63) / 64;
    const dim3 grid((n_rows + kRows - 1) / kRows);
    hipStream_t s = (hipStream_t)stream;
    auto go = [&](auto nuc, auto normc) {
        constexpr int NU = decltype(nuc)::value;
        constexpr bool NORM = decltype(normc)::value;
        MOE_LAUNCH(TK_ROUTER, (k_router_q8<NU, NORM>), grid, dim3(kThreads), 0, s, (const uint16_t*)x, h_in,
                   (const uint16_t*)norm_w, eps, (uint16_t*)xb_out, (__half*)xh_out, codes, (const uint16_t*)scales,
                   (const uint16_t*)biases, hidden, n_rows, k, m, scratch, counter, ids_out, (uint16_t*)scores_out,
                   pred_out, (uint16_t*)logits_out);
    };
    auto with_nu = [&](auto normc) {
        switch (nu) {
            case 1: go(std::integral_constant<int, 1>(), normc); break;
            case 2: go(std::integral_constant<int, 2>(), normc); break;
            case 3: go(std::integral_constant<int, 3>(), normc); break;
            default: go(std::integral_constant<int, 4>(), normc); break;
        }
    };
    if (h_in) with_nu(std::true_type());
    else with_nu(std::false_type());
    HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

extern "C" int moe_router_q8(const void* x, const uint32_t* codes, const void* scales, const void* biases, int hidden,
                             int n_rows, int group, int k, int m, void* workspace, uint32_t* ids_out, void* scores_out,
                             int32_t* pred_out, void* logits_out, void* stream) {
    if (!x) { moe_set_error("router_q8: null pointer"); return -1; }
    return launch_router_q8(x, nullptr, nullptr, 0.f, nullptr, nullptr, codes, scales, biases, hidden, n_rows, group, k,
                            m, workspace, ids_out, scores_out, pred_out, logits_out, stream);
}

extern "C" int moe_router_q8_norm(const float* h_in, const void* norm_w, float eps, void* x_bf16_out, void* x_f16_out,
                                  const uint32_t* codes, const void* scales, const void* biases, int hidden, int n_rows,
                                  int group, int k, int m, void* workspace, uint32_t* ids_out, void* scores_out,
                                  int32_t* pred_out, void* logits_out, void* stream) {
    if (!h_in) { moe_set_error("router_q8_norm: null pointer"); return -1; }
    if (hidden % 8) { moe_set_error("router_q8_norm: hidden=%d (a multiple of 8)", hidden); return -1; }
    return launch_router_q8(nullptr, h_in, norm_w, eps, x_bf16_out, x_f16_out, codes, scales, biases, hidden, n_rows,
                            group, k, m, workspace, ids_out, scores_out, pred_out, logits_out, stream);
}
