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
// Launch: one block per 16 weight rows (4 waves x 4 rows).  Every block writes its rounded
// logits to scratch, then counts itself done on a device-scope counter; the block that
// arrives last runs the selection (wave 0: softmax/top-k, wave 1: predictor) and re-arms the
// counter, so no grid-wide wait is ever needed.
#include <hip/hip_fp16.h>

#include "moe_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 4;
constexpr int kRowsPerBlock = 4 * kRowsPerWave;
constexpr int kMaxHidden = 4096;
constexpr int kMaxExperts = 1024;

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}

// One rounding, f64 -> f16 (round to nearest even); never through f32, which would round twice.
__device__ __forceinline__ uint16_t f16_bits(double v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ float round_f16(double v) {
    return (float)(_Float16)v;
}

// Order-preserving map of an fp16 value to uint16 (signed values; -0 folded onto +0).
__device__ __forceinline__ uint32_t f16_order(float v) {
    uint16_t b = f16_bits(v == 0.0f ? 0.0 : (double)v);
    return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

__global__ __launch_bounds__(kThreads) void k_router(
    const float* __restrict__ h_in, const __half* __restrict__ norm_w, float eps,
    const __half* __restrict__ x_in, __half* __restrict__ x_out,
    const __half* __restrict__ w, const __half* __restrict__ w_next,
    int hidden, int n_exp, int k, int m,
    float* __restrict__ scratch, unsigned* __restrict__ counter,
    uint32_t* __restrict__ ids_out, __half* __restrict__ scores_out, int32_t* __restrict__ pred_out) {
    __shared__ float xs[kMaxHidden];
    __shared__ double red[kThreads / 64];
    __shared__ int is_last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    // ---- input vector (exact fp16 values held as float) -------------------------------------
    if (h_in) {
        double ss = 0.0;
        for (int i = tid; i < hidden; i += kThreads) {
            double v = h_in[i];
            ss += v * v;
        }
        ss = wave_sum_f64(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        double tot = red[0] + red[1] + red[2] + red[3];
        double denom = sqrt(tot / hidden + (double)eps);
        for (int i = tid; i < hidden; i += kThreads) {
            double v = (double)h_in[i] / denom;
            if (norm_w) v *= (double)__half2float(norm_w[i]);
            float r = round_f16(v);
            xs[i] = r;
            if (x_out && blockIdx.x == 0) x_out[i] = __ushort_as_half(f16_bits(v));
        }
    } else {
        for (int i = tid; i < hidden; i += kThreads) xs[i] = __half2float(x_in[i]);
    }
    __syncthreads();

    // ---- logits: 4 rows per wave, 16 bytes per lane per 512 columns -------------------------
    const int total_rows = n_exp * (w_next ? 2 : 1);
    const int row0 = blockIdx.x * kRowsPerBlock + wv * kRowsPerWave;
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
        int row = row0 + rr;
        if (row >= total_rows) break;
        const __half* wr = (row < n_exp) ? (w + (size_t)row * hidden) : (w_next + (size_t)(row - n_exp) * hidden);
        double acc = 0.0;
        for (int c0 = lane * 8; c0 < hidden; c0 += 512) {
            uint4 q = *reinterpret_cast<const uint4*>(wr + c0);
            const __half* hv = reinterpret_cast<const __half*>(&q);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc += (double)(__half2float(hv[j]) * xs[c0 + j]);
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) scratch[row] = round_f16(acc);
    }

    // ---- last block selects -----------------------------------------------------------------
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(counter, 1u);
        is_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    const int per_lane = (n_exp + 63) / 64;

    if (wv == 0) {
        // softmax over n_exp logits in fp64, gates rounded to fp16
        double lv[kMaxExperts / 64];
        double mx = -1e300;
        for (int i = 0; i < per_lane; ++i) {
            int e = lane + 64 * i;
            lv[i] = (e < n_exp) ? (double)__hip_atomic_load(&scratch[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -1e300;
            mx = fmax(mx, lv[i]);
        }
        mx = wave_max_f64(mx);
        double sum = 0.0;
        for (int i = 0; i < per_lane; ++i) {
            int e = lane + 64 * i;
            lv[i] = (e < n_exp) ? exp(lv[i] - mx) : 0.0;
            sum += lv[i];
        }
        sum = wave_sum_f64(sum);
        uint32_t key[kMaxExperts / 64];
        for (int i = 0; i < per_lane; ++i) {
            int e = lane + 64 * i;
            // gates are >= 0, so fp16 bit patterns order like the values; id breaks ties upward
            key[i] = (e < n_exp) ? (((uint32_t)f16_bits(lv[i] / sum) << 16) | (uint32_t)e) : 0u;
        }
        uint32_t picked[MOE_MAX_K];
        for (int r = 0; r < k; ++r) {
            uint32_t best = 0;
            for (int i = 0; i < per_lane; ++i) best = max(best, key[i]);
            best = wave_max_u32(best);
            for (int i = 0; i < per_lane; ++i)
                if (key[i] == best) key[i] = 0;
            picked[r] = best;
        }
        if (lane == 0) {
            // ascending order = reverse of extraction order
            double gsel[MOE_MAX_K];
            double s = 0.0;
            for (int j = 0; j < k; ++j) {
                uint32_t kk = picked[k - 1 - j];
                ids_out[j] = kk & 0xFFFFu;
                gsel[j] = (double)__half2float(__ushort_as_half((uint16_t)(kk >> 16)));
                s = (double)round_f16(s + gsel[j]);
            }
            for (int j = 0; j < k; ++j) scores_out[j] = __ushort_as_half(f16_bits(gsel[j] / s));
        }
    } else if (wv == 1 && w_next && m > 0) {
        uint32_t key[kMaxExperts / 64];
        for (int i = 0; i < per_lane; ++i) {
            int e = lane + 64 * i;
            float v = (e < n_exp) ? __hip_atomic_load(&scratch[n_exp + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
            key[i] = (e < n_exp) ? ((f16_order(v) << 16) | (uint32_t)e) : 0u;
        }
        uint32_t picked[MOE_MAX_PREFETCH];
        for (int r = 0; r < m; ++r) {
            uint32_t best = 0;
            for (int i = 0; i < per_lane; ++i) best = max(best, key[i]);
            best = wave_max_u32(best);
            for (int i = 0; i < per_lane; ++i)
                if (key[i] == best) key[i] = 0;
            picked[r] = best;
        }
        if (lane == 0) {
            // picked is descending by (value, id); equal values must come out in ascending id
            int i = 0;
            while (i < m) {
                int j = i;
                while (j + 1 < m && (picked[j + 1] >> 16) == (picked[i] >> 16)) ++j;
                for (int a = i, b = j; a < b; ++a, --b) {
                    uint32_t t = picked[a];
                    picked[a] = picked[b];
                    picked[b] = t;
                }
                i = j + 1;
            }
            for (int r = 0; r < m; ++r) pred_out[r] = (int32_t)(picked[r] & 0xFFFFu);
        }
    }
    if (tid == 0) atomicExch(counter, 0u);
}

// Standalone RMSNorm (one block): x_out = fp16(h / sqrt(mean(h^2) + eps) * w), fp64 math,
// one rounding; the same arithmetic as the router's prologue.
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float* __restrict__ h_in, const __half* __restrict__ norm_w,
                                                       float eps, int hidden, __half* __restrict__ x_out) {
    __shared__ double red[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    double ss = 0.0;
    for (int i = tid; i < hidden; i += kThreads) {
        double v = h_in[i];
        ss += v * v;
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    double tot = red[0] + red[1] + red[2] + red[3];
    double denom = sqrt(tot / hidden + (double)eps);
    for (int i = tid; i < hidden; i += kThreads) {
        double v = (double)h_in[i] / denom;
        if (norm_w) v *= (double)__half2float(norm_w[i]);
        x_out[i] = __ushort_as_half(f16_bits(v));
    }
}

}  // namespace

int launch_rmsnorm(const float* h_in, const __half* norm_w, float eps, int hidden, __half* x_out, hipStream_t s) {
    if (!h_in || !x_out || hidden <= 0) { moe_set_error("rmsnorm: bad arguments"); return -1; }
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kThreads), 0, s, h_in, norm_w, eps, hidden, x_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_router(const float* h_in, const __half* norm_w, float eps, const __half* x_in,
                  __half* x_out, const __half* w, const __half* w_next, int hidden, int n_exp,
                  int k, int m, float* scratch, unsigned* counter, uint32_t* ids_out,
                  __half* scores_out, int32_t* pred_out, hipStream_t s) {
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
    if (!w || !scratch || !counter || !ids_out || !scores_out || (!h_in && !x_in) || (w_next && !pred_out)) {
        moe_set_error("router: null pointer argument");
        return -1;
    }
    int rows = n_exp * (w_next ? 2 : 1);
    int grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(k_router, dim3(grid), dim3(kThreads), 0, s, h_in, norm_w, eps, x_in, x_out,
                       w, w_next, hidden, n_exp, k, w_next ? m : 0, scratch, counter, ids_out,
                       scores_out, pred_out);
    HIP_TRY(hipGetLastError());
    return 0;
}
