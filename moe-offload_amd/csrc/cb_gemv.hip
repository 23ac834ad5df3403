// 2-bit codebook gather-GEMV for batch-1 decode of non-gated experts on gfx950:
//     y = residual + sum_j s_j * D_j( relu(U_j x)^2 )
// U_j [inter][hidden], D_j [hidden][inter] in the codebook format of moe_common.h (CbLayout).
//
// Reference semantics: the Nemotron-style experts of the reference run inside llama.cpp's Metal
// backend (llamacpp-bolt/llama-moe-cache.patch; mul_mm_id over IQ2_XXS weights): weights are
// dequantised to floats and multiplied with float activations.  Weight j of an 8-weight group:
//     w = d * (2 s + 1) / 8 * grid[idx][j] * (-1 if bit j of sign7 | parity(sign7) << 7)
//
// Data path.  One 8-byte load per lane is one 32-weight sub-block (4 grid indices + aux word).
// The grid (256 entries x 8 byte magnitudes; {1, 3, 5} in the workload) and the 128 sign patterns
// are tables in LDS built by every block: a group costs one 16-byte grid read (the 8 magnitudes as
// fp16 or bf16), one 16-byte sign-mask read (the sign bit of each half), 4 XORs and 4 dot2.  The
// activation slice a lane needs is fixed across the rows it visits and stays in registers.
// Accumulation is fp32; the sub-block scale d (2 s + 1) / 8 is applied once per 32 weights.
//
// Kernels
//   k_cb_up<T>:   32 lanes per weight row (T sub-blocks each), 8 rows per wave, 32 per block,
//                 grid (inter / 32, k).  h = relu(u)^2 is written as bf16 [k][inter] (fp32
//                 range: a square can exceed fp16).
//   k_cb_down<T>: 16 lanes per row, 8 output rows per block x all k experts (4 waves split the
//                 experts: whole experts in rounds of 4, then the remaining experts' 4-row halves
//                 dealt round robin, so no wave carries a whole expert more than another; the next
//                 task's codes and h slice loaded while the current one is multiplied); the block
//                 reduces over its waves in a fixed order and writes y = residual + sum_j s_j y_j
//                 (fp32) or the per-expert rows.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "lane_reduce.h"
#include "moe_common.h"
#include "norm_f64.h"

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));

constexpr int kUpRowsPerBlock = 32;
constexpr int kDownRows = 8;
static_assert((kDownRows & (kDownRows - 1)) == 0, "the epilogue row of a thread is tid & (kDownRows - 1)");

// fp16 / bf16 bit pattern of a grid magnitude (any byte value is exact in both: bf16 keeps 8
// significant bits).
__device__ __forceinline__ uint32_t mag_bits(uint32_t v, bool bf16) {
    if (bf16) return __float_as_uint((float)v) >> 16;
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v);
}

// gtab[e] = the 8 magnitudes of grid entry e as halves (fp16 or bf16), in weight order, built by
// thread e from its grid entry g (loaded early by the caller: 256 threads, one entry each);
// stab[s7] = the sign bit (bit 15 of a half) of each of the 8 weights for sign7 = s7.
__device__ __forceinline__ void build_tables(uint2 g, uint4* gtab, uint4* stab, int tid, bool bf16) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t src = k < 2 ? g.x : g.y;
        const uint32_t lo = (src >> (16 * (k & 1))) & 0xFF, hi = (src >> (16 * (k & 1) + 8)) & 0xFF;
        w[k] = mag_bits(lo, bf16) | (mag_bits(hi, bf16) << 16);
    }
    gtab[tid] = make_uint4(w[0], w[1], w[2], w[3]);
    if (tid < 128) {
        const uint32_t s8 = (uint32_t)tid | ((uint32_t)(__popc(tid) & 1) << 7);
        uint32_t m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = (((s8 >> (2 * k)) & 1u) << 15) | (((s8 >> (2 * k + 1)) & 1u) << 31);
        stab[tid] = make_uint4(m[0], m[1], m[2], m[3]);
    }
}

// The table entries of one sub-block's 4 groups (8 LDS reads, issued together).
struct SubTab {
    uint4 m[4], sg[4];
};

__device__ __forceinline__ SubTab fetch_tab(uint2 q, const uint4* gtab, const uint4* stab) {
    SubTab r;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        r.m[g] = gtab[(q.x >> (8 * g)) & 0xFF];
        r.sg[g] = stab[(q.y >> (7 * g)) & 0x7F];
    }
    return r;
}

// Dot of one sub-block (4 groups of 8) with 32 activations xa[0..15] (pairs, natural order):
// unscaled sum over the sub-block of grid magnitude * sign * x.
template <bool BF16>
__device__ __forceinline__ float sub_dot(const SubTab& tb, const uint32_t* xa) {
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 m = tb.m[g], sg = tb.sg[g];
        const uint32_t w[4] = {m.x ^ sg.x, m.y ^ sg.y, m.z ^ sg.z, m.w ^ sg.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (BF16)
                s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, w[k]), __builtin_bit_cast(b2_t, xa[4 * g + k]),
                                                    s, false);
            else
                s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[k]), __builtin_bit_cast(h2_t, xa[4 * g + k]), s,
                                           false);
        }
    }
    return s;
}

__device__ __forceinline__ float sub_scale(uint2 q, float d) {
    return d * (float)(2u * (q.y >> 28) + 1u) * 0.125f;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));   // inf / nan
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// NORM: the input is the previous layer's fp32 output h, normalised here (norm64: every block
// computes x = RMSNorm(h) into LDS while its weight loads fly; block (0, 0) also writes x to
// x_out for the down projection's residual), instead of an fp16 x read from memory.
template <int T, bool NORM>
__global__ __launch_bounds__(256) void k_cb_up(const __half* __restrict__ x, const float* __restrict__ h_in,
                                               const __half* __restrict__ norm_w, float eps, __half* __restrict__ x_out,
                                               const uint8_t* __restrict__ pool, size_t stride,
                                               const uint32_t* __restrict__ slots, int n_slots, CbLayout L,
                                               const uint8_t* __restrict__ grid, uint16_t* __restrict__ h_out) {
    __shared__ uint4 gtab[256];
    __shared__ uint4 stab[128];
    __shared__ __align__(16) uint16_t xs[NORM ? norm64::kMaxHidden : 8];
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint2 gentry = reinterpret_cast<const uint2*>(grid)[tid];     // blockDim == 256
    norm64::NormIn nin;
    if constexpr (NORM) {
        norm64::load(nin, h_in, norm_w, L.hidden);
        __builtin_amdgcn_sched_barrier(0);                // the norm's loads ahead of the weights'
    }

    const int j = blockIdx.y;
    const uint32_t slot = slots[j];
    const bool ok = slot < (uint32_t)n_slots;             // an invalid slot reads nothing, yields 0
    const int nsub = L.hidden / 32, nsb = L.hidden / 256, inter = L.inter;
    const int li = lane & 31, rsel = lane >> 5;

    // All loads are unconditional, from clamped in-range addresses, and masked where the value
    // is used: a load under a branch makes the compiler wait for it at the join, serialising
    // the round trips.
    const uint8_t* blob = pool + (size_t)(ok ? slot : 0) * stride;
    const uint2* qs = reinterpret_cast<const uint2*>(blob + L.up_qs);
    const uint16_t* dd = reinterpret_cast<const uint16_t*>(blob + L.up_d);
    const int row_base = blockIdx.x * kUpRowsPerBlock + wv * 8;

    uint2 q[4][T];
    uint16_t dr[4][T];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int row = row_base + 2 * it + rsel;
        const int rc = row < inter ? row : inter - 1;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int sb = li + 32 * t;
            const int sc = sb < nsub ? sb : nsub - 1;
            q[it][t] = qs[(size_t)rc * nsub + sc];
            dr[it][t] = dd[(size_t)rc * nsb + sc / 8];
        }
    }

    // activation slice: sub-blocks li + 32 t, 16 pairs each (a clamped sub-block past the end
    // is masked by its scale below); from memory, or from the block's normalised copy in LDS
    uint32_t xa[T][16];
    auto take_x = [&](const __half* src) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int sb = li + 32 * t;
            const int sc = sb < nsub ? sb : nsub - 1;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 u = reinterpret_cast<const uint4*>(src + (size_t)sc * 32)[v];
                xa[t][4 * v] = u.x;
                xa[t][4 * v + 1] = u.y;
                xa[t][4 * v + 2] = u.z;
                xa[t][4 * v + 3] = u.w;
            }
        }
    };
    if constexpr (!NORM) take_x(x);
    build_tables(gentry, gtab, stab, tid, false);
    if constexpr (NORM)
        norm64::finish(nin, norm_w != nullptr, eps, L.hidden, xs,
                       blockIdx.x == 0 && blockIdx.y == 0 ? x_out : nullptr, red);
    __syncthreads();                                      // tables (and the normalised x) built
    if constexpr (NORM) take_x(reinterpret_cast<const __half*>(xs));
    // a lane whose sub-block, row or expert is out of range contributes nothing (scale 0)
    float dv[4][T];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int row = row_base + 2 * it + rsel;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const bool v = ok && row < inter && li + 32 * t < nsub;
            dv[it][t] = v ? __half2float(__ushort_as_half(dr[it][t])) : 0.f;
        }
    }

    // the next sub-block's table entries are fetched while the current one is multiplied
    SubTab tb[2];
    tb[0] = fetch_tab(q[0][0], gtab, stab);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int i = it * T + t;
            if (i + 1 < 4 * T) tb[(i + 1) & 1] = fetch_tab(q[(i + 1) / T][(i + 1) % T], gtab, stab);
            acc += sub_scale(q[it][t], dv[it][t]) * sub_dot<false>(tb[i & 1], xa[t]);
        }
        acc = lanes::group_sum<32>(acc);
        const int row = row_base + 2 * it + rsel;
        if (li == 0 && row < inter) {
            const float r = acc > 0.f ? acc : 0.f;
            h_out[(size_t)j * inter + row] = f32_to_bf16_rne(r * r);
        }
    }
}

template <int T>
struct DownLoad {                    // one expert's operands for one lane
    uint2 q[2][T];                   // sub-block codes of the lane's 2 rows
    uint16_t dr[2][T];               // their super-block scales (fp16 bits)
    uint32_t ha[T][16];              // h slice: T sub-blocks x 16 bf16 pairs
    bool ok;
};

template <int T>
__global__ __launch_bounds__(256) void k_cb_down(const uint16_t* __restrict__ h, const uint8_t* __restrict__ pool,
                                                 size_t stride, const uint32_t* __restrict__ slots, int n_slots,
                                                 const __half* __restrict__ scores, int k, CbLayout L,
                                                 const uint8_t* __restrict__ grid, const __half* __restrict__ residual,
                                                 float* __restrict__ y_out, int per_expert) {
    constexpr int kMaxTasks = (MOE_MAX_K + 3) / 4 + 1;
    __shared__ uint4 gtab[256];
    __shared__ uint4 stab[128];
    __shared__ float red[4][kDownRows];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int inter = L.inter, hidden = L.hidden, nsub = inter / 32, nsb = inter / 256;
    const int li = lane & 15, rsel = lane >> 4;
    const int row0 = blockIdx.x * kDownRows;
    const uint2 gentry = reinterpret_cast<const uint2*>(grid)[tid];     // blockDim == 256

    // The wave's tasks, in order: whole experts wv, wv + 4, ... (every expert when rows per expert
    // are written; else only the k / 4 full rounds), then the remaining experts' row halves
    // (4 rows each) dealt round robin, so no wave multiplies more than a half expert beyond the
    // others.  The next task's operands are loaded while the current one is multiplied.
    const int nfull = per_expert ? 0 : k / 4;
    const int nwhole = per_expert ? (k > wv ? (k - wv + 3) / 4 : 0) : nfull;
    const int nhalf_all = per_expert ? 0 : 2 * (k - 4 * nfull);
    const int ntask = nwhole + (nhalf_all > wv ? (nhalf_all - wv + 3) / 4 : 0);
    auto task = [&](int tk, int& e, int& hsel) {           // hsel -1: both row halves
        if (tk < nwhole) {
            e = wv + 4 * tk;
            hsel = -1;
        } else {
            const int idx = wv + 4 * (tk - nwhole);
            e = 4 * nfull + (idx >> 1);
            hsel = idx & 1;
        }
        e = e < k ? e : k - 1;                             // a task past the wave's last reloads it
    };
    // Loads are unconditional from clamped addresses (see k_cb_up); a half task loads its rows
    // into both row slots.
    auto load = [&](int tk, DownLoad<T>& b) {
        int e, hsel;
        task(tk, e, hsel);
        const uint32_t slot = slots[e];
        b.ok = slot < (uint32_t)n_slots;
        const uint8_t* blob = pool + (size_t)(b.ok ? slot : 0) * stride;
        const uint2* qs = reinterpret_cast<const uint2*>(blob + L.down_qs);
        const uint16_t* dd = reinterpret_cast<const uint16_t*>(blob + L.down_d);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int row = row0 + 4 * (hsel < 0 ? it : hsel) + rsel;
            const int rc = row < hidden ? row : hidden - 1;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int sb = li + 16 * t;
                const int sc = sb < nsub ? sb : nsub - 1;
                b.q[it][t] = qs[(size_t)rc * nsub + sc];
                b.dr[it][t] = dd[(size_t)rc * nsb + sc / 8];
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int sc = li + 16 * t < nsub ? li + 16 * t : nsub - 1;
            const uint4* hp = reinterpret_cast<const uint4*>(h + (size_t)e * inter + (size_t)sc * 32);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 u = hp[v];
                b.ha[t][4 * v] = u.x;
                b.ha[t][4 * v + 1] = u.y;
                b.ha[t][4 * v + 2] = u.z;
                b.ha[t][4 * v + 3] = u.w;
            }
        }
    };
    // every task's score, read unconditionally (any k halves stand in for absent scores)
    const __half* sp = scores ? scores : reinterpret_cast<const __half*>(grid);
    float sjv[kMaxTasks];
#pragma unroll
    for (int tk = 0; tk < kMaxTasks; ++tk) {
        int e, hsel;
        task(tk, e, hsel);
        const float sv = __half2float(sp[e]);
        sjv[tk] = scores ? sv : 1.0f;
    }

    // the residual row of the epilogue, loaded now so that no round trip follows the reduction
    // (without a residual, y_out's first bytes, unused)
    const int erow = row0 + (tid & (kDownRows - 1)) < hidden ? row0 + (tid & (kDownRows - 1)) : hidden - 1;
    const __half r_prev = (residual ? residual : reinterpret_cast<const __half*>(y_out))[erow];

    DownLoad<T> buf[2];
    load(0, buf[0]);
    build_tables(gentry, gtab, stab, tid, true);
    __syncthreads();

    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int tk = 0; tk < kMaxTasks; ++tk) {
        if (tk >= ntask) break;                            // wave-uniform
        if (tk + 1 < kMaxTasks) load(tk + 1, buf[(tk + 1) & 1]);
        const DownLoad<T>& b = buf[tk & 1];
        int e, hsel;
        task(tk, e, hsel);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            if (hsel >= 0 && it == 1) break;               // a half task has one row slot
            const int rit = hsel < 0 ? it : hsel;
            const int row = row0 + 4 * rit + rsel;
            float part = 0.f;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const bool v = b.ok && row < hidden && li + 16 * t < nsub;
                const float d = v ? __half2float(__ushort_as_half(b.dr[it][t])) : 0.f;
                part += sub_scale(b.q[it][t], d) * sub_dot<true>(fetch_tab(b.q[it][t], gtab, stab), b.ha[t]);
            }
            part = lanes::group_sum<16>(part);
            if (per_expert) {
                if (li == 0 && row < hidden) y_out[(size_t)e * hidden + row] = part;
            } else {
                const float c = sjv[tk] * part;
                acc[0] += rit == 0 ? c : 0.f;
                acc[1] += rit == 1 ? c : 0.f;
            }
        }
    }
    if (per_expert) return;
#pragma unroll
    for (int it = 0; it < 2; ++it)
        if (li == 0) red[wv][4 * it + rsel] = acc[it];
    __syncthreads();
    if (tid < kDownRows) {
        const int row = row0 + tid;
        if (row < hidden) {
            float y = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
            if (residual) y += __half2float(r_prev);
            y_out[row] = y;
        }
    }
}

bool check_cb(const char* who, int k, int hidden, int inter, const void* pool, int n_slots, size_t stride,
              const void* slots, const void* grid, const void* a, const void* b) {
    if (k <= 0 || k > MOE_MAX_K) { moe_set_error("%s: k=%d out of range 1..%d", who, k, MOE_MAX_K); return false; }
    if (hidden <= 0 || inter <= 0 || hidden % 256 || inter % 256 || hidden > 4096 || inter > 2048) {
        moe_set_error("%s: hidden=%d inter=%d must be multiples of 256 (hidden <= 4096, inter <= 2048)", who, hidden,
                      inter);
        return false;
    }
    if (n_slots <= 0 || !pool || !slots || !grid || !a || !b) { moe_set_error("%s: empty pool or null pointer", who); return false; }
    const CbLayout L = cb_layout(hidden, inter);
    if (stride < L.bytes) { moe_set_error("%s: expert stride %zu < blob bytes %zu", who, stride, L.bytes); return false; }
    return true;
}

template <int T>
int up_t(const __half* x, const float* h_in, const __half* norm_w, float eps, __half* x_out, const uint8_t* pool,
         size_t stride, const uint32_t* slots, int n_slots, int k, const CbLayout& L, const uint8_t* grid,
         uint16_t* h_out, hipStream_t s) {
    dim3 g((L.inter + kUpRowsPerBlock - 1) / kUpRowsPerBlock, k);
    if (h_in)
        MOE_LAUNCH(TK_CB_UP, (k_cb_up<T, true>), g, dim3(256), 0, s, x, h_in, norm_w, eps, x_out, pool, stride, slots,
                   n_slots, L, grid, h_out);
    else
        MOE_LAUNCH(TK_CB_UP, (k_cb_up<T, false>), g, dim3(256), 0, s, x, h_in, norm_w, eps, x_out, pool, stride, slots,
                   n_slots, L, grid, h_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int T>
int down_t(const uint16_t* h, const uint8_t* pool, size_t stride, const uint32_t* slots, int n_slots,
           const __half* scores, int k, const CbLayout& L, const uint8_t* grid, const __half* residual, float* y_out,
           int per_expert, hipStream_t s) {
    dim3 g((L.hidden + kDownRows - 1) / kDownRows);
    MOE_LAUNCH(TK_CB_DOWN, (k_cb_down<T>), g, dim3(256), 0, s, h, pool, stride, slots, n_slots, scores, k, L,
               grid, residual, y_out, per_expert);
    HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

namespace {

int up_any(const __half* x, const float* h_in, const __half* norm_w, float eps, __half* x_out, const uint8_t* pool,
           size_t stride, int n_slots, const uint32_t* slots, int k, int hidden, int inter, const uint8_t* grid,
           uint16_t* h_out, hipStream_t s) {
    const CbLayout L = cb_layout(hidden, inter);
    switch ((hidden / 32 + 31) / 32) {
        case 1: return up_t<1>(x, h_in, norm_w, eps, x_out, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        case 2: return up_t<2>(x, h_in, norm_w, eps, x_out, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        case 3: return up_t<3>(x, h_in, norm_w, eps, x_out, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        default: return up_t<4>(x, h_in, norm_w, eps, x_out, pool, stride, slots, n_slots, k, L, grid, h_out, s);
    }
}

}  // namespace

int launch_cb_up(const __half* x, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots, int k,
                 int hidden, int inter, const uint8_t* grid, uint16_t* h_out, hipStream_t s) {
    if (!check_cb("cb_up", k, hidden, inter, pool, n_slots, stride, slots, grid, x, h_out)) return -1;
    return up_any(x, nullptr, nullptr, 0.f, nullptr, pool, stride, n_slots, slots, k, hidden, inter, grid, h_out, s);
}

int launch_cb_up_norm(const float* h_in, const __half* norm_w, float eps, __half* x_out, const uint8_t* pool,
                      size_t stride, int n_slots, const uint32_t* slots, int k, int hidden, int inter,
                      const uint8_t* grid, uint16_t* h_out, hipStream_t s) {
    if (!check_cb("cb_up_norm", k, hidden, inter, pool, n_slots, stride, slots, grid, h_in, h_out)) return -1;
    if (!x_out) { moe_set_error("cb_up_norm: x_out is null"); return -1; }
    return up_any(nullptr, h_in, norm_w, eps, x_out, pool, stride, n_slots, slots, k, hidden, inter, grid, h_out, s);
}

int launch_cb_down(const uint16_t* h, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots,
                   const __half* scores, int k, int hidden, int inter, const uint8_t* grid, const __half* residual,
                   float* y_out, int per_expert, hipStream_t s) {
    if (!check_cb("cb_down", k, hidden, inter, pool, n_slots, stride, slots, grid, h, y_out)) return -1;
    if (per_expert != 0 && per_expert != 1) { moe_set_error("cb_down: mode %d (0 sum, 1 per expert)", per_expert); return -1; }
    const CbLayout L = cb_layout(hidden, inter);
    switch ((inter / 32 + 15) / 16) {
        case 1: return down_t<1>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        case 2: return down_t<2>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        case 3: return down_t<3>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        default: return down_t<4>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
    }
}
