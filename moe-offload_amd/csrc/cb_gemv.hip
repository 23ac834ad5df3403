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
//                 experts); h is staged in LDS; the block reduces over experts in a fixed order
//                 and writes y = residual + sum_j s_j y_j (fp32) or the per-expert rows.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "moe_common.h"

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));

constexpr int kUpRowsPerBlock = 32;
constexpr int kDownRows = 8;

// fp16 / bf16 bit pattern of a grid magnitude (any byte value is exact in both: bf16 keeps 8
// significant bits).
__device__ __forceinline__ uint32_t mag_bits(uint32_t v, bool bf16) {
    if (bf16) return __float_as_uint((float)v) >> 16;
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v);
}

// gtab[e] = the 8 magnitudes of grid entry e as halves (fp16 or bf16), in weight order;
// stab[s7] = the sign bit (bit 15 of a half) of each of the 8 weights for sign7 = s7.
__device__ __forceinline__ void build_tables(const uint8_t* __restrict__ grid, uint4* gtab, uint4* stab, int tid,
                                             bool bf16) {
    for (int e = tid; e < 256; e += blockDim.x) {
        const uint2 g = reinterpret_cast<const uint2*>(grid)[e];
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t src = k < 2 ? g.x : g.y;
            const uint32_t lo = (src >> (16 * (k & 1))) & 0xFF, hi = (src >> (16 * (k & 1) + 8)) & 0xFF;
            w[k] = mag_bits(lo, bf16) | (mag_bits(hi, bf16) << 16);
        }
        gtab[e] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (int s = tid; s < 128; s += blockDim.x) {
        const uint32_t s8 = (uint32_t)s | ((uint32_t)(__popc(s) & 1) << 7);
        uint32_t m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = (((s8 >> (2 * k)) & 1u) << 15) | (((s8 >> (2 * k + 1)) & 1u) << 31);
        stab[s] = make_uint4(m[0], m[1], m[2], m[3]);
    }
}

// Dot of one sub-block (4 groups of 8) with 32 activations xa[0..15] (pairs, natural order):
// unscaled sum over the sub-block of grid magnitude * sign * x.
template <bool BF16>
__device__ __forceinline__ float sub_dot(uint2 q, const uint32_t* xa, const uint4* gtab, const uint4* stab) {
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 m = gtab[(q.x >> (8 * g)) & 0xFF];
        const uint4 sg = stab[(q.y >> (7 * g)) & 0x7F];
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

template <int T>
__global__ __launch_bounds__(256) void k_cb_up(const __half* __restrict__ x, const uint8_t* __restrict__ pool,
                                               size_t stride, const uint32_t* __restrict__ slots, int n_slots,
                                               CbLayout L, const uint8_t* __restrict__ grid,
                                               uint16_t* __restrict__ h_out) {
    __shared__ uint4 gtab[256];
    __shared__ uint4 stab[128];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    build_tables(grid, gtab, stab, tid, false);

    const int j = blockIdx.y;
    const uint32_t slot = slots[j];
    const bool ok = slot < (uint32_t)n_slots;             // an invalid slot reads nothing, yields 0
    const int nsub = L.hidden / 32, nsb = L.hidden / 256, inter = L.inter;
    const int li = lane & 31, rsel = lane >> 5;

    // activation slice: sub-blocks li + 32 t, 16 pairs each
    uint32_t xa[T][16];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int sb = li + 32 * t;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 u = sb < nsub ? reinterpret_cast<const uint4*>(x + (size_t)sb * 32)[v] : make_uint4(0, 0, 0, 0);
            xa[t][4 * v] = u.x;
            xa[t][4 * v + 1] = u.y;
            xa[t][4 * v + 2] = u.z;
            xa[t][4 * v + 3] = u.w;
        }
    }

    const uint8_t* blob = pool + (size_t)(ok ? slot : 0) * stride;
    const uint2* qs = reinterpret_cast<const uint2*>(blob + L.up_qs);
    const __half* dd = reinterpret_cast<const __half*>(blob + L.up_d);
    const int row_base = blockIdx.x * kUpRowsPerBlock + wv * 8;

    uint2 q[4][T];
    float dv[4][T];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int row = row_base + 2 * it + rsel;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int sb = li + 32 * t;
            const bool v = ok && row < inter && sb < nsub;
            q[it][t] = v ? qs[(size_t)row * nsub + sb] : make_uint2(0, 0);
            dv[it][t] = v ? __half2float(dd[(size_t)row * nsb + sb / 8]) : 0.f;
        }
    }
    __syncthreads();                                      // tables built

#pragma unroll
    for (int it = 0; it < 4; ++it) {
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < T; ++t) acc += sub_scale(q[it][t], dv[it][t]) * sub_dot<false>(q[it][t], xa[t], gtab, stab);
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
        const int row = row_base + 2 * it + rsel;
        if (li == 0 && row < inter) {
            const float r = acc > 0.f ? acc : 0.f;
            h_out[(size_t)j * inter + row] = f32_to_bf16_rne(r * r);
        }
    }
}

template <int T>
__global__ __launch_bounds__(256) void k_cb_down(const uint16_t* __restrict__ h, const uint8_t* __restrict__ pool,
                                                 size_t stride, const uint32_t* __restrict__ slots, int n_slots,
                                                 const __half* __restrict__ scores, int k, CbLayout L,
                                                 const uint8_t* __restrict__ grid, const __half* __restrict__ residual,
                                                 float* __restrict__ y_out, int per_expert) {
    __shared__ uint4 gtab[256];
    __shared__ uint4 stab[128];
    extern __shared__ uint4 hs[];                         // h [k][inter] bf16
    __shared__ float red[4][kDownRows];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    build_tables(grid, gtab, stab, tid, true);
    const int inter = L.inter, hidden = L.hidden, nsub = inter / 32, nsb = inter / 256;
    const int n16 = k * inter / 8;                        // uint4 units of h
    for (int i = tid; i < n16; i += 256) hs[i] = reinterpret_cast<const uint4*>(h)[i];

    const int li = lane & 15, rsel = lane >> 4;
    const int row0 = blockIdx.x * kDownRows;
    __syncthreads();

    float acc[2] = {0.f, 0.f};
    for (int jj = wv; jj < k; jj += 4) {
        const uint32_t slot = slots[jj];
        const bool ok = slot < (uint32_t)n_slots;         // an invalid slot reads nothing, yields 0
        const uint8_t* blob = pool + (size_t)(ok ? slot : 0) * stride;
        const uint2* qs = reinterpret_cast<const uint2*>(blob + L.down_qs);
        const __half* dd = reinterpret_cast<const __half*>(blob + L.down_d);
        uint2 q[2][T];
        float dv[2][T];
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int row = row0 + 4 * it + rsel;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int sb = li + 16 * t;
                const bool v = ok && row < hidden && sb < nsub;
                q[it][t] = v ? qs[(size_t)row * nsub + sb] : make_uint2(0, 0);
                dv[it][t] = v ? __half2float(dd[(size_t)row * nsb + sb / 8]) : 0.f;
            }
        }
        uint32_t ha[T][16];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int sb = li + 16 * t;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 u = sb < nsub ? hs[((size_t)jj * inter + (size_t)sb * 32) / 8 + v] : make_uint4(0, 0, 0, 0);
                ha[t][4 * v] = u.x;
                ha[t][4 * v + 1] = u.y;
                ha[t][4 * v + 2] = u.z;
                ha[t][4 * v + 3] = u.w;
            }
        }
        const float sj = scores ? __half2float(scores[jj]) : 1.0f;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            float part = 0.f;
#pragma unroll
            for (int t = 0; t < T; ++t) part += sub_scale(q[it][t], dv[it][t]) * sub_dot<true>(q[it][t], ha[t], gtab, stab);
#pragma unroll
            for (int o = 8; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
            const int row = row0 + 4 * it + rsel;
            if (per_expert) {
                if (li == 0 && row < hidden) y_out[(size_t)jj * hidden + row] = part;
            } else {
                acc[it] += sj * part;
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
            if (residual) y += __half2float(residual[row]);
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
int up_t(const __half* x, const uint8_t* pool, size_t stride, const uint32_t* slots, int n_slots, int k,
         const CbLayout& L, const uint8_t* grid, uint16_t* h_out, hipStream_t s) {
    dim3 g((L.inter + kUpRowsPerBlock - 1) / kUpRowsPerBlock, k);
    MOE_LAUNCH(TK_CB_UP, (k_cb_up<T>), g, dim3(256), 0, s, x, pool, stride, slots, n_slots, L, grid, h_out);
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int T>
int down_t(const uint16_t* h, const uint8_t* pool, size_t stride, const uint32_t* slots, int n_slots,
           const __half* scores, int k, const CbLayout& L, const uint8_t* grid, const __half* residual, float* y_out,
           int per_expert, hipStream_t s) {
    const size_t shmem = (size_t)k * L.inter * sizeof(uint16_t);
    dim3 g((L.hidden + kDownRows - 1) / kDownRows);
    MOE_LAUNCH(TK_CB_DOWN, (k_cb_down<T>), g, dim3(256), shmem, s, h, pool, stride, slots, n_slots, scores, k, L,
               grid, residual, y_out, per_expert);
    HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

int launch_cb_up(const __half* x, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots, int k,
                 int hidden, int inter, const uint8_t* grid, uint16_t* h_out, hipStream_t s) {
    if (!check_cb("cb_up", k, hidden, inter, pool, n_slots, stride, slots, grid, x, h_out)) return -1;
    const CbLayout L = cb_layout(hidden, inter);
    switch ((hidden / 32 + 31) / 32) {
        case 1: return up_t<1>(x, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        case 2: return up_t<2>(x, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        case 3: return up_t<3>(x, pool, stride, slots, n_slots, k, L, grid, h_out, s);
        default: return up_t<4>(x, pool, stride, slots, n_slots, k, L, grid, h_out, s);
    }
}

int launch_cb_down(const uint16_t* h, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots,
                   const __half* scores, int k, int hidden, int inter, const uint8_t* grid, const __half* residual,
                   float* y_out, int per_expert, hipStream_t s) {
    if (!check_cb("cb_down", k, hidden, inter, pool, n_slots, stride, slots, grid, h, y_out)) return -1;
    if (per_expert != 0 && per_expert != 1) { moe_set_error("cb_down: mode %d (0 sum, 1 per expert)", per_expert); return -1; }
    if ((size_t)k * inter * sizeof(uint16_t) > 48 * 1024) {
        moe_set_error("cb_down: k * inter = %d exceeds the 48 KiB LDS stage of h", k * inter);
        return -1;
    }
    const CbLayout L = cb_layout(hidden, inter);
    switch ((inter / 32 + 15) / 16) {
        case 1: return down_t<1>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        case 2: return down_t<2>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        case 3: return down_t<3>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
        default: return down_t<4>(h, pool, stride, slots, n_slots, scores, k, L, grid, residual, y_out, per_expert, s);
    }
}
