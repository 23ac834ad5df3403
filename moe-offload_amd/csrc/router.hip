// Fused router for gfx950: [RMSNorm] -> logits = x . W^T (and the next layer's W_next . x for
// the prefetch predictor) -> softmax -> top-k in ascending-gate order -> renormalise.
//
// Reference semantics: mlx-qwen38/loader.py:903-908 (router), :237-242 and :950-958 (next-layer
// top-m predictor), cpp/src/layers.cpp:311-341.  Ordering rule: the selected ids are the last k
// of a stable ascending sort of the gates (ascending gate, equal gates in ascending id; at the
// k boundary the higher id wins); scores = round(g / seqsum(g)) where the sum runs left to
// right over that order with every partial rounded to fp16.  The predictor selects by the same
// rule on the raw logits and emits descending value, equal values in ascending id.
//
// Arithmetic: fp16 x fp16 products are exact in fp32 and are accumulated in fp64; the sum is
// rounded once, directly, to fp16.  The softmax, renormalisation and RMSNorm run in fp64 and
// round once to fp16.  Rounded results therefore do not depend on summation order.
//
// Launch: one weight row per wave (4 per block), every wave's loads issued before the input
// vector is ready.  Every block writes its rounded logits to scratch, then counts itself done
// on a device-scope counter; the block that arrives last runs the selection (wave 0:
// softmax/top-k with DPP wave maxima, wave 1: predictor) and re-arms the counter, so no
// grid-wide wait is ever needed.
//
// Optionally the last block continues with the slot-table work of the decode path
// (expert_io.c:583-685 and 527-581): wave 0 runs the decode step of this layer's table with the
// selected ids, wave 1 the prefetch of the next layer's table with the prediction, so neither
// needs a launch of its own.
#include <hip/hip_fp16.h>

#include <mutex>

#include "lane_reduce.h"
#include "moe_common.h"
#include "norm_f64.h"
#include "route_select.h"
#include "slot_table_dev.h"

namespace {

using route::kMaxExperts;
using route::kThreads;
using route::f16_order;
using route::f64_to_f16_bits;
using route::round_f16;
using route::wave_topn;
using lanes::wave_sum_f64;
constexpr int kRowsPerBlock = 4;          // one weight row per wave
constexpr int kMaxHidden = 4096;

// A zeroed table, read (never written) by the last block in place of a missing one.
__device__ SlotTable g_no_table;

// The RMSNorm prologue (every block computes it) is norm64::finish over chunks this kernel loads
// itself, ahead of its weight loads.
using norm64::NormIn;
constexpr int kNormChunks = norm64::kChunks;
static_assert(norm64::kThreads == kThreads && norm64::kMaxHidden == kMaxHidden, "norm block shape");

// NC = 16-byte weight units per lane and row: hidden <= 512 * NC.  NORM: the input is h (fp32,
// normalised here) rather than x (fp16); a compile-time choice, so that no branch lets the
// compiler sink the input loads behind the weight loads.
template <int NC, bool NORM>
__global__ __launch_bounds__(kThreads) void k_router(
    const float* __restrict__ h_in, const __half* __restrict__ norm_w, float eps,
    const __half* __restrict__ x_in, __half* __restrict__ x_out,
    const __half* __restrict__ w, const __half* __restrict__ w_next,
    int hidden, int n_exp, int k, int m,
    float* __restrict__ scratch, unsigned* __restrict__ counter,
    uint32_t* __restrict__ ids_out, __half* __restrict__ scores_out, int32_t* __restrict__ pred_out,
    SlotTable* __restrict__ step_tab, uint32_t* __restrict__ slot_inds, SlotTable* __restrict__ pf_tab, int max_fetch) {
    __shared__ __align__(16) uint16_t xs[kMaxHidden];
    __shared__ double red[kThreads / 64];
    __shared__ int is_last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int total_rows = n_exp * (w_next ? 2 : 1);
    const int row = blockIdx.x * kRowsPerBlock + wv;
    const __half* wr = nullptr;
    if (row < total_rows) wr = (row < n_exp) ? (w + (size_t)row * hidden) : (w_next + (size_t)(row - n_exp) * hidden);

    // Loads first, nothing waits before all are issued: the input (h and the norm weights, or
    // x), then this wave's weight row.  Every load is unconditional from a clamped in-range
    // address and masked where it is used (a row past the end reads row 0; a unit past the
    // row's end reads its last unit).  The input is read as 16-byte units of whichever vector
    // is given (h: 4 fp32 per unit, x: 8 fp16), so no branch separates the two cases.
    NormIn nin;
    {
        const uint4* src = NORM ? reinterpret_cast<const uint4*>(h_in) : reinterpret_cast<const uint4*>(x_in);
        const int n_units = NORM ? hidden / 4 : hidden / 8;
        // without norm weights, read the input again in their place (in range; unused)
        const __half* wsrc = norm_w ? norm_w : reinterpret_cast<const __half*>(src);
#pragma unroll
        for (int c = 0; c < kNormChunks; ++c) {
            const int u = c * kThreads + tid;
            const uint4 v = src[u < n_units ? u : n_units - 1];
            nin.hv[c] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
            const int i = 4 * u;
            nin.w2[c] = *reinterpret_cast<const uint2*>(wsrc + (i < hidden ? i : hidden - 4));
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every input load ahead of the weight loads
    const __half* wrow = wr ? wr : w;
    uint4 q[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int off = c * 512 + lane * 8;
        q[c] = *reinterpret_cast<const uint4*>(wrow + (off < hidden ? off : hidden - 8));
    }
    __builtin_amdgcn_sched_barrier(0);   // every weight load issued before anything waits

    if constexpr (NORM) {
        norm64::finish(nin, norm_w != nullptr, eps, hidden, xs, (x_out && blockIdx.x == 0) ? x_out : nullptr, red);
    } else {
#pragma unroll
        for (int c = 0; c < kNormChunks; ++c) {
            const int i = 8 * (c * kThreads + tid);
            if (i < hidden) {
                const float4 v = nin.hv[c];
                *reinterpret_cast<uint4*>(&xs[i]) =
                    make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w));
            }
        }
    }
    __syncthreads();

    if (wr) {
        double acc = 0.0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int off = c * 512 + lane * 8;
            if (off >= hidden) continue;
            const uint4 wq = q[c];
            const uint4 xq = *reinterpret_cast<const uint4*>(&xs[off]);
            const __half* hw = reinterpret_cast<const __half*>(&wq);
            const __half* hx = reinterpret_cast<const __half*>(&xq);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc += (double)(__half2float(hw[j]) * __half2float(hx[j]));
        }
        acc = wave_sum_f64(acc);
        // publish with an agent-scope atomic store (written through to the device coherence
        // point), so the only ordering needed before counting in is this wave's store completion;
        // without a counter the logits are the output (read by a later kernel: a plain store)
        if (lane == 0) {
            if (counter) __hip_atomic_store(&scratch[row], round_f16(acc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else scratch[row] = round_f16(acc);
        }
    }
    if (!counter) return;                 // logits only: the consumer selects

    // ---- the last block to finish selects ---------------------------------------------------
    // Every logit store of this block has completed (vmcnt(0)) before the block counts itself
    // done; the last block reads the logits with agent-scope atomic loads.  No L2 write-back
    // or invalidate is needed for data that only ever moves through agent-scope atomics.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) is_last = (__hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1);
    __syncthreads();
    if (!is_last) return;

    __shared__ uint32_t keys[kMaxExperts];
    __shared__ uint32_t pkeys[kMaxExperts];
    __shared__ uint32_t sel_ids[MOE_MAX_K];
    __shared__ int32_t sel_pred[MOE_MAX_PREFETCH];
    __shared__ double redm[kThreads / 64], reds[kThreads / 64];
    const int n_pad = ((n_exp + 63) / 64) * 64;
    const bool predict = w_next && m > 0;
    // softmax over the logits in fp64, spread over the whole block.  Every logit load is issued
    // first, unconditionally from a clamped index (scratch holds 2 * n_exp values), and masked
    // afterwards: a load merged with a default value at a branch join is waited for inside the
    // branch, one round trip per load.
    constexpr int kPer = route::kPer;
    float lraw[kPer], praw[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        const int ec = e < n_exp ? e : 0;
        lraw[i] = __hip_atomic_load(&scratch[ec], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        praw[i] = __hip_atomic_load(&scratch[n_exp + ec], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The slot tables, in the same round trip: wave 0 reads the step's table, wave 1 the
    // prefetch's; the other waves read one of them again (unused), so that the address is
    // chosen without a branch and no wait lands inside one.
    const SlotTable* any_tab = step_tab ? step_tab : (pf_tab ? pf_tab : &g_no_table);
    const SlotTable* my_tab = (wv == 1 && pf_tab) ? pf_tab : ((wv == 0 && step_tab) ? step_tab : any_tab);
    const slot_dev::TabRegs tab = slot_dev::fetch_table(my_tab, lane);
    if (predict) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = tid + kThreads * i;
            if (e < n_pad)
                pkeys[e] = (e < n_exp) ? ((f16_order(__half_as_ushort(__float2half_rn(praw[i]))) << 16) | (uint32_t)e) : 0u;
        }
    }
    route::gate_keys(lraw, n_exp, keys, redm, reds);

    // the selection on wave 0, the predictor on wave 2
    if (wv == 0) {
        uint32_t id;
        __half sc;
        const int pos = route::select_topk(keys, n_pad, k, lane, id, sc);
        if (pos >= 0) {
            ids_out[pos] = id;
            sel_ids[pos] = id;
            scores_out[pos] = sc;
        }
    } else if (wv == 2 && predict) {
        const uint32_t mine = wave_topn(pkeys, 0, n_pad, m, lane);
        // lanes 0..m-1 hold descending (value, id); equal values must come out in ascending id:
        // within a run of equal values, lane r takes the id of its mirror position in the run
        const uint32_t val = mine >> 16;
        int first = lane, last = lane;
        for (int q2 = 0; q2 < m; ++q2) {
            uint32_t vq = (uint32_t)__builtin_amdgcn_readlane((int)val, q2);
            if (vq == val && q2 < first) first = q2;
            if (vq == val && q2 > last) last = q2;
        }
        const int src = first + last - lane;
        const int id = __shfl((int)(mine & 0xFFFFu), src, 64);
        if (lane < m) {
            pred_out[lane] = id;
            sel_pred[lane] = id;
        }
    }
    if (step_tab || pf_tab) {
        __shared__ slot_dev::LdsTable tabs[2];
        __syncthreads();
        if (wv == 0 && step_tab)
            slot_dev::dev_slot_step(step_tab, tabs[0], tab, lane < k ? sel_ids[lane] : 0u, k, slot_inds, lane);
        if (wv == 1 && pf_tab && predict) slot_dev::dev_slot_prefetch(pf_tab, tabs[1], tab, sel_pred, m, max_fetch, lane);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Standalone RMSNorm (one block): x_out = fp16(h / sqrt(mean(h^2) + eps) * w), fp64 math,
// one rounding; the same arithmetic as the router's prologue.
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float* __restrict__ h_in, const __half* __restrict__ norm_w,
                                                       float eps, int hidden, __half* __restrict__ x_out) {
    __shared__ __align__(16) uint16_t xs[kMaxHidden];
    __shared__ double red[kThreads / 64];
    NormIn nin;
    norm64::load(nin, h_in, norm_w, hidden);
    norm64::finish(nin, norm_w != nullptr, eps, hidden, xs, x_out, red);
}

__global__ __launch_bounds__(kThreads) void k_rmsnorm_bf16(const float* __restrict__ h_in, const uint16_t* __restrict__ norm_w,
                                                            float eps, int hidden, uint16_t* __restrict__ x_bf16,
                                                            __half* __restrict__ x_f16) {
    __shared__ double red[kThreads / 64];
    NormIn nin;
    norm64::load(nin, h_in, reinterpret_cast<const __half*>(norm_w), hidden);
    norm64::finish_bf16(nin, norm_w != nullptr, eps, hidden, x_bf16, x_f16, red);
}

__global__ void k_f64_to_f16(const double* __restrict__ in, uint16_t* __restrict__ out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f64_to_f16_bits(in[i]);
}

__global__ void k_zero_u32(uint32_t* __restrict__ p, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// ---- the router without a caller workspace ------------------------------------------------------
// Logits of the router and the predictor (2 * kMaxExperts floats), then the arrival counter on a
// 256-byte line of its own.  Fixed offsets, so calls with different expert counts share one
// counter.  Each GPU the library runs on holds its own copy until the process ends.
constexpr size_t kStaticLogitBytes = 2 * (size_t)kMaxExperts * sizeof(float);
constexpr size_t kStaticScratchBytes = kStaticLogitBytes + 256;
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

// Device address of this device's copy of `scratch`, resolved once per device with that device
// current.  The counter is cleared then (a fill kernel on the caller's stream, not a memset: the
// first call may be under graph capture); every router launch leaves it at zero again.
static int static_scratch(hipStream_t s, uint8_t** out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        moe_set_error("router_noalloc: device %d beyond the %d devices the library tracks", dev, kMaxDevices);
        return -1;
    }
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) {
            moe_set_error("router_noalloc: no device address for the static scratch on device %d", dev);
            return -1;
        }
        hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(64), 0, s, (uint32_t*)((uint8_t*)p + kStaticLogitBytes), 64);
        HIP_TRY(hipGetLastError());
        g_scratch_ptr[dev] = (uint8_t*)p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

int launch_router_noalloc(const float* h_in, const __half* norm_w, float eps, const __half* x_in, __half* x_out,
                          const __half* w, const __half* w_next, int hidden, int n_exp, int k, int m, uint32_t* ids_out,
                          __half* scores_out, int32_t* pred_out, hipStream_t s) {
    if (n_exp <= 0 || n_exp > kMaxExperts) {
        moe_set_error("router_noalloc: n_exp=%d exceeds the static scratch (at most %d experts, %zu bytes)", n_exp,
                      kMaxExperts, kStaticScratchBytes);
        return -1;
    }
    uint8_t* base = nullptr;
    if (static_scratch(s, &base)) return -1;
    return launch_router(h_in, norm_w, eps, x_in, x_out, w, w_next, hidden, n_exp, k, m, (float*)base,
                         (unsigned*)(base + kStaticLogitBytes), ids_out, scores_out, pred_out, nullptr, nullptr,
                         nullptr, 0, s);
}

int launch_f64_to_f16(const double* in, uint16_t* out, int n, hipStream_t s) {
    if (n <= 0 || !in || !out) { moe_set_error("f64_to_f16: bad arguments"); return -1; }
    hipLaunchKernelGGL(k_f64_to_f16, dim3((n + 255) / 256), dim3(256), 0, s, in, out, n);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_rmsnorm(const float* h_in, const __half* norm_w, float eps, int hidden, __half* x_out, hipStream_t s) {
    if (!h_in || !x_out || hidden <= 0 || hidden > kMaxHidden || hidden % 8) {
        moe_set_error("rmsnorm: hidden=%d (multiple of 8, <= %d) or null pointer", hidden, kMaxHidden);
        return -1;
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kThreads), 0, s, h_in, norm_w, eps, hidden, x_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_rmsnorm_bf16(const float* h_in, const uint16_t* norm_w, float eps, int hidden, uint16_t* x_bf16,
                        __half* x_f16, hipStream_t s) {
    if (!h_in || !x_bf16 || !x_f16 || hidden <= 0 || hidden > kMaxHidden || hidden % 8) {
        moe_set_error("rmsnorm_bf16: hidden=%d (multiple of 8, <= %d) or null pointer", hidden, kMaxHidden);
        return -1;
    }
    hipLaunchKernelGGL(k_rmsnorm_bf16, dim3(1), dim3(kThreads), 0, s, h_in, norm_w, eps, hidden, x_bf16, x_f16);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_router_logits(const float* h_in, const __half* norm_w, float eps, const __half* x_in, __half* x_out,
                         const __half* w, int hidden, int n_exp, float* logits_out, hipStream_t s) {
    if (hidden <= 0 || hidden > kMaxHidden || hidden % 8 != 0) {
        moe_set_error("router_logits: hidden=%d unsupported (multiple of 8, <= %d)", hidden, kMaxHidden);
        return -1;
    }
    if (n_exp <= 0 || n_exp > kMaxExperts) { moe_set_error("router_logits: n_exp=%d unsupported", n_exp); return -1; }
    if (!w || !logits_out || (!h_in && !x_in)) { moe_set_error("router_logits: null pointer argument"); return -1; }
    const int grid = (n_exp + kRowsPerBlock - 1) / kRowsPerBlock;
    auto go = [&](auto nc, auto norm) {
        constexpr int NC = decltype(nc)::value;
        constexpr bool NORM = decltype(norm)::value;
        MOE_LAUNCH(TK_ROUTER, (k_router<NC, NORM>), dim3(grid), dim3(kThreads), 0, s, h_in, norm_w, eps, x_in, x_out, w,
                   nullptr, hidden, n_exp, 1, 0, logits_out, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                   nullptr, 0);
    };
    using N4 = std::integral_constant<int, 4>;
    using N8 = std::integral_constant<int, 8>;
    if (h_in) {
        if (hidden <= 2048) go(N4(), std::true_type());
        else go(N8(), std::true_type());
    } else {
        if (hidden <= 2048) go(N4(), std::false_type());
        else go(N8(), std::false_type());
    }
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_router(const float* h_in, const __half* norm_w, float eps, const __half* x_in,
                  __half* x_out, const __half* w, const __half* w_next, int hidden, int n_exp,
                  int k, int m, float* scratch, unsigned* counter, uint32_t* ids_out,
                  __half* scores_out, int32_t* pred_out, SlotTable* step_tab, uint32_t* slot_inds,
                  SlotTable* pf_tab, int max_fetch, hipStream_t s) {
    if (hidden <= 0 || hidden > kMaxHidden || hidden % 8 != 0) {
        moe_set_error("router: hidden=%d unsupported (multiple of 8, <= %d)", hidden, kMaxHidden);
        return -1;
    }
    if (n_exp <= 0 || n_exp > kMaxExperts || k <= 0 || k > MOE_MAX_K || k > n_exp) {
        moe_set_error("router: n_exp=%d k=%d unsupported", n_exp, k);
        return -1;
    }
    if (w_next && (m <= 0 || m > MOE_MAX_PREFETCH || m > n_exp)) {
        moe_set_error("router: predictor m=%d unsupported", m);
        return -1;
    }
    if (!w || !scratch || !counter || !ids_out || !scores_out || (!h_in && !x_in) || (w_next && !pred_out) ||
        (step_tab && !slot_inds)) {
        moe_set_error("router: null pointer argument");
        return -1;
    }
    int rows = n_exp * (w_next ? 2 : 1);
    int grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;      // one row per wave
    auto go = [&](auto nc, auto norm) {
        constexpr int NC = decltype(nc)::value;
        constexpr bool NORM = decltype(norm)::value;
        MOE_LAUNCH(TK_ROUTER, (k_router<NC, NORM>), dim3(grid), dim3(kThreads), 0, s, h_in, norm_w, eps, x_in, x_out,
                           w, w_next, hidden, n_exp, k, w_next ? m : 0, scratch, counter, ids_out,
                           scores_out, pred_out, step_tab, slot_inds, pf_tab, max_fetch);
    };
    using N4 = std::integral_constant<int, 4>;
    using N8 = std::integral_constant<int, 8>;
    if (h_in) {
        if (hidden <= 2048) go(N4(), std::true_type());
        else go(N8(), std::true_type());
    } else {
        if (hidden <= 2048) go(N4(), std::false_type());
        else go(N8(), std::false_type());
    }
    HIP_TRY(hipGetLastError());
    return 0;
}
