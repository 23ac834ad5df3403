// Expert selection of the router (loader.py:903-908; cpp/src/layers.cpp:311-325), shared by the
// router's last block and the resident-path gate/up kernel, which therefore select bit for bit
// alike.  Input: the n_exp logits, already rounded to fp16 (held as floats).
//   gates = fp16(softmax in fp64), keys = (gate bits << 16 | id): gates are >= 0, so the bit
//   pattern orders like the value and equal gates order by id (the higher id wins at the k
//   boundary); the top k keys in ascending order are the selected ids; scores = fp16(g / s) with
//   s the left-to-right fp16-rounded sum over that order.
#pragma once
#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "moe_common.h"

namespace route {

constexpr int kThreads = 256;                  // the selection runs on a block of 256 threads
constexpr int kMaxExperts = 1024;
constexpr int kPer = kMaxExperts / kThreads;   // logits per thread

// Wave-wide max of a uint32: DPP butterflies inside each 16-lane row, then the row pairs and the
// wave halves exchanged with v_permlane16_swap / v_permlane32_swap, so every lane ends with the
// maximum in a vector register (no readlane -> scalar -> vector round trip in a selection round).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, lanes::partner<1>(v));
    v = max(v, lanes::partner<2>(v));
    v = max(v, lanes::partner<4>(v));
    v = max(v, lanes::partner<8>(v));
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)p[0], (uint32_t)p[1]);
    p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)p[0], (uint32_t)p[1]);
}

// Wave-wide min of a uint32, the same butterflies.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, lanes::partner<1>(v));
    v = min(v, lanes::partner<2>(v));
    v = min(v, lanes::partner<4>(v));
    v = min(v, lanes::partner<8>(v));
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = min((uint32_t)p[0], (uint32_t)p[1]);
    p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return min((uint32_t)p[0], (uint32_t)p[1]);
}


// f64 -> f16 with a single round-to-nearest-even: truncate to f32, set the sticky bit when
// inexact (round-to-odd with 24 >= 11 + 2 bits), then let the f32 -> f16 conversion round.
__device__ __forceinline__ uint16_t f64_to_f16_bits(double d) {
    float f = __double2float_rz(d);
    if ((double)f != d) f = __uint_as_float(__float_as_uint(f) | 1u);
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float round_f16(double v) {
    return __half2float(__ushort_as_half(f64_to_f16_bits(v)));
}

// f64 -> bf16 bits with one round-to-nearest-even: f32 by round-to-odd (sticky bit when inexact;
// 24 >= 8 + 2 bits), then the f32 -> bf16 rounding.
__device__ __forceinline__ uint16_t f64_to_bf16_bits(double d) {
    float f = __double2float_rz(d);
    if ((double)f != d) f = __uint_as_float(__float_as_uint(f) | 1u);
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// The rule's 16-bit format: fp16 (the workload's fp16 router, loader.py:903-908 at fp16) or bf16
// (the real checkpoint's router, whose gates, sums and scores are bf16).
template <bool BF16>
__device__ __forceinline__ uint16_t rule_from_f64(double d) { return BF16 ? f64_to_bf16_bits(d) : f64_to_f16_bits(d); }
template <bool BF16>
__device__ __forceinline__ float rule_to_f32(uint32_t b) {
    return BF16 ? bf16_to_f32(b) : __half2float(__ushort_as_half((uint16_t)b));
}
template <bool BF16>
__device__ __forceinline__ uint16_t rule_from_f32(float f) {
    return BF16 ? f32_to_bf16_bits(f) : __half_as_ushort(__float2half_rn(f));
}

// The n largest keys of keys[lo, hi) (LDS; distinct, 0 = empty) by one wave: lane r < n gets
// the r-th largest (0 once the range runs out).  KPL keys per lane cover the range.  The keys
// are distinct except for zeros (padding, and a zero gate of expert 0), so round r > 0 picks the
// largest key below the previous pick b: with d = (b - 1) - key in unsigned arithmetic, every key
// below b gives d < b and every other key d >= b, so the pick is b - 1 - (wave minimum of d).  A
// pick of 0 stays 0 (all later ranks are 0 keys).  No key is rewritten, so a round is one
// subtraction per key, a minimum tree and the wave minimum.  When no key is left below the pick
// (more ranks than keys), the pick is 0, as once the keys run out.
template <int KPL>
__device__ __forceinline__ uint32_t wave_topn_k(const uint32_t* keys, int lo, int hi, int n, int lane) {
    uint32_t key[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
        const int idx = lo + lane + 64 * i;
        key[i] = idx < hi ? keys[idx] : 0u;
    }
    uint32_t best = key[0];
#pragma unroll
    for (int i = 1; i < KPL; ++i) best = max(best, key[i]);
    best = wave_max_u32(best);
    uint32_t mine = lane == 0 ? best : 0u;
    for (int r = 1; r < n; ++r) {
        const uint32_t bm1 = best - 1u;
        uint32_t d = bm1 - key[0];
#pragma unroll
        for (int i = 1; i < KPL; ++i) d = min(d, bm1 - key[i]);
        d = wave_min_u32(d);
        best = (best == 0u || d >= best) ? 0u : bm1 - d;      // d >= best: no key left below
        if (lane == r) mine = best;
    }
    return mine;
}

// wave_topn_k with KPL fixed at compile time for the range size (up to kMaxExperts keys): a
// runtime bound would turn every key operation into a masked select.
__device__ __forceinline__ uint32_t wave_topn(const uint32_t* keys, int lo, int hi, int n, int lane) {
    const int kpl = (hi - lo + 63) / 64;                    // wave-uniform
    if (kpl <= 1) return wave_topn_k<1>(keys, lo, hi, n, lane);
    if (kpl <= 2) return wave_topn_k<2>(keys, lo, hi, n, lane);
    if (kpl <= 4) return wave_topn_k<4>(keys, lo, hi, n, lane);
    if (kpl <= 8) return wave_topn_k<8>(keys, lo, hi, n, lane);
    return wave_topn_k<kMaxExperts / 64>(keys, lo, hi, n, lane);
}

// Order-preserving map of an fp16 value to uint16 (signed values; -0 folded onto +0).
__device__ __forceinline__ uint32_t f16_order(uint16_t b) {
    if (b == 0x8000u) b = 0;
    return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

// Block-wide: the gate keys of the logits this thread holds (lraw[i] = logit tid + kThreads i,
// any value where that index is >= n_exp) into keys[0, n_pad) (n_pad = n_exp rounded up to 64;
// padding keys 0).  Gates rounded to fp16, or to bf16 with BF16.  Ends with a barrier.
template <bool BF16 = false>
__device__ __forceinline__ void gate_keys(const float (&lraw)[kPer], int n_exp, uint32_t* keys, double* redm,
                                          double* reds) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n_pad = ((n_exp + 63) / 64) * 64;
    double lv[kPer];
    double mx = -1e300;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        lv[i] = e < n_exp ? (double)lraw[i] : -1e300;
        mx = fmax(mx, lv[i]);
    }
    mx = lanes::wave_max_f64(mx);
    if (lane == 0) redm[wv] = mx;
    __syncthreads();
    mx = fmax(fmax(redm[0], redm[1]), fmax(redm[2], redm[3]));
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        int e = tid + kThreads * i;
        lv[i] = (e < n_exp) ? exp(lv[i] - mx) : 0.0;
        sum += lv[i];
    }
    sum = lanes::wave_sum_f64(sum);
    if (lane == 0) reds[wv] = sum;
    __syncthreads();
    sum = (reds[0] + reds[1]) + (reds[2] + reds[3]);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        int e = tid + kThreads * i;
        if (e < n_pad) keys[e] = (e < n_exp) ? (((uint32_t)rule_from_f64<BF16>(lv[i] / sum) << 16) | (uint32_t)e) : 0u;
    }
    __syncthreads();
}

// ---- the resident gate/up's selection, the weight loads first ----------------------------------
// Gates are a monotone function of the logits (exp, one division by the same sum, one rounding), so
// ordering by (logit, id) gives the rule's order -- (gate, id) -- unless two different logits round
// to one gate among the first k + 1.  The fp16 resident gate/up (k_q2_gate_up_routed) therefore
// ranks by logit first (no softmax: spec_keys + wave_topn of k + 1 rounds), issues its weight loads
// for that ranking, and only then computes the k + 1 gates (spec_check); when they decide the same
// ranking the exact keys follow from them, otherwise the block runs the full rule (fallback_keys +
// wave_topn) and reloads if its expert changed.  Ids, order and scores are the rule's in both cases.
// The bf16 rule (the checkpoint's router) keeps the softmax first: its coarser gates tie at the k
// boundary for 13-20% of tokens, and those fallbacks cost more than the head start saves.

// Order-preserving 16-bit key of a logit held as a float that is exactly a value of the rule's
// format (-0 folded onto +0), and its inverse.
template <bool BF16>
__device__ __forceinline__ uint32_t logit_order(float v) {
    uint32_t b = rule_from_f32<BF16>(v);
    if (b == 0x8000u) b = 0;
    return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
template <bool BF16>
__device__ __forceinline__ float logit_from_order(uint32_t o) {
    const uint32_t b = (o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu);
    return rule_to_f32<BF16>(b);
}

// Block-wide: keys[0, n_pad) = (logit order << 16 | id) of the logits this thread holds (as
// gate_keys; padding 0).  Ends with a barrier.
template <bool BF16>
__device__ __forceinline__ void spec_keys(const float (&lraw)[kPer], int n_exp, uint32_t* keys) {
    const int tid = threadIdx.x;
    const int n_pad = ((n_exp + 63) / 64) * 64;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        if (e < n_pad) keys[e] = (e < n_exp) ? ((logit_order<BF16>(lraw[i]) << 16) | (uint32_t)e) : 0u;
    }
    __syncthreads();
}

// Block-wide, after spec_keys and the k + 1 rounds: the softmax sum of gate_keys (the same
// arithmetic and order; mx = the largest logit, wave 0's first pick) and, in wave 0, the gates of
// the first k + 1 picks (lane r holds pick `top`).  Returns true, block-uniform, when two of them
// that decide the ranking clash: pick r's gate below pick r + 1's for some r < k, or equal to it
// from a different logit with pick r's id the lower (r < k - 1), or equal at all (r = k - 1).  lane
// r < k of wave 0 gets the rule's key in `exact`.  lv / sum are kept for fallback_keys.
// Contains one barrier, plus one more to broadcast the answer (flag: an int of LDS).
template <bool BF16>
__device__ __forceinline__ bool spec_check(const float (&lraw)[kPer], int n_exp, int k, uint32_t top, double mx,
                                           double* reds, int* flag, double (&lv)[kPer], double& sum,
                                           uint32_t& exact) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    sum = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        lv[i] = (e < n_exp) ? exp((double)lraw[i] - mx) : 0.0;
        sum += lv[i];
    }
    sum = lanes::wave_sum_f64(sum);
    if (lane == 0) reds[wv] = sum;
    __syncthreads();
    sum = (reds[0] + reds[1]) + (reds[2] + reds[3]);
    if (wv == 0) {
        const bool valid = lane <= k && top != 0u;
        const uint32_t g = valid ? (uint32_t)rule_from_f64<BF16>(exp((double)logit_from_order<BF16>(top >> 16) - mx) / sum)
                                 : 0u;
        const uint32_t g_next = (uint32_t)__shfl_down((int)g, 1, 64);
        const uint32_t top_next = (uint32_t)__shfl_down((int)top, 1, 64);
        const bool next_valid = __shfl_down((int)valid, 1, 64) != 0;
        // inside the first k, equal gates keep the logit ranking when the logits are equal (both
        // rankings then order by id) or when the higher logit also has the higher id; at the
        // boundary any equal gate is a clash, since experts ranked below pick k (lower logits,
        // possibly higher ids) may share that gate
        const bool same_logit = (top >> 16) == (top_next >> 16);
        const bool id_down = (top & 0xFFFFu) > (top_next & 0xFFFFu);
        const bool clash = lane < k && next_valid &&
                           (g < g_next || (g == g_next && (lane == k - 1 || (!same_logit && !id_down))));
        exact = (g << 16) | (top & 0xFFFFu);
        const bool any_clash = __any(clash);              // the whole wave votes, then lane 0 writes
        if (lane == 0) *flag = any_clash ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

// Block-wide fallback after spec_check found equal gates: gate_keys' keys from the kept lv / sum.
// Ends with a barrier.
template <bool BF16>
__device__ __forceinline__ void fallback_keys(const double (&lv)[kPer], double sum, int n_exp, uint32_t* keys) {
    const int tid = threadIdx.x;
    const int n_pad = ((n_exp + 63) / 64) * 64;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = tid + kThreads * i;
        if (e < n_pad) keys[e] = (e < n_exp) ? (((uint32_t)rule_from_f64<BF16>(lv[i] / sum) << 16) | (uint32_t)e) : 0u;
    }
    __syncthreads();
}

// One wave, from the k largest keys (lane r holds the r-th largest, wave_topn): the id and score
// bits that go to output position k - 1 - r (ascending gate order) for lanes r < k; position -1
// for the other lanes.  The scores are g / s with s the left-to-right sum over ascending order,
// each partial rounded to the rule's format: fp16 (11 bits) or bf16 (8 bits); an f32 sum or
// quotient of two such values, rounded again, equals the single rounding (24 >= 2 p + 2).
template <bool BF16>
__device__ __forceinline__ int topk_score_bits(uint32_t mine, int k, int lane, uint32_t& id, uint16_t& score) {
    const float g = rule_to_f32<BF16>(mine >> 16);
    float s = 0.0f;
    for (int j = 0; j < k; ++j) {
        float gj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), k - 1 - j));
        s = rule_to_f32<BF16>(rule_from_f32<BF16>(s + gj));
    }
    id = mine & 0xFFFFu;
    score = rule_from_f32<BF16>(g / s);                // correctly rounded f32 division, then rounded
    return lane < k ? k - 1 - lane : -1;
}

__device__ __forceinline__ int topk_scores(uint32_t mine, int k, int lane, uint32_t& id, __half& score) {
    uint16_t b;
    const int pos = topk_score_bits<false>(mine, k, lane, id, b);
    score = __ushort_as_half(b);
    return pos;
}

// One wave: the selection from the keys.  Lane r < k returns the id and score that go to output
// position k - 1 - r (ascending gate order); other lanes return position -1.
__device__ __forceinline__ int select_topk(const uint32_t* keys, int n_pad, int k, int lane, uint32_t& id,
                                           __half& score) {
    // Top-k by rounds of wave maxima, one wave over all keys: a round is a short dependent chain,
    // and splitting the keys over waves adds a barrier and a second selection over the
    // candidates, which costs more than it saves.
    return topk_scores(wave_topn(keys, 0, n_pad, k, lane), k, lane, id, score);
}

}  // namespace route
