// Grouped Q2 SwitchGLU for chunked prefill on gfx950 (MFMA).
//
// Reference semantics: mlx-qwen38/loader.py:566-699 (CachedSwitchGLU prefill: the (token, k)
// rows sorted by expert, chunk-local slot = rank of the expert in the chunk),
// prefill_qproj.py:18-40 (gather_qmm over the sorted rows), cpp/src/layers.cpp:364-600.
// For the sorted rows r of segment u (one expert, weights = blob seg_slot[u] of the pool):
//     h_r = silu(G_u x_r) * (U_u x_r)        (k_q2g_proj<.., kGateUp>, fp16 out)
//     y_r = D_u h_r                          (k_q2g_proj<.., kDown>, fp16 out, row row_out[r])
// with W = scale * q + bias per group of 64 inputs (2-bit codes, 16 per u32, LSB first).
//
// Tiling.  The rows of a segment form M tiles of 16 (v_mfma_f32_16x16x32_f16).  A block of 4
// waves owns 16 consecutive output rows per subtile and 4 subtiles per wave (gate/up: 2 x 16
// rows of each projection = 128 intermediate rows per block; down: 4 x 16 = 256 output rows).
// Per 256-wide K chunk j a lane (n = lane & 15, kq = lane >> 4) loads group 4j + kq of weight
// row n: one 16-byte load of 64 codes plus one (scale, bias) word.
//
// Dequantisation.  A 2-bit code in the low bits of a nibble is the fp4 (e2m1) value q/2, so
// w & 0x33333333 (even codes) and (w >> 2) & 0x33333333 (odd codes) are 8 fp4 values each;
// v_cvt_scalef32_pk_f16_fp4 turns a byte into two exact halves and one v_pk_mul_f16 by 2*scale
// gives scale*q rounded once to fp16.  The bias contributes sum_g b[n,g] * sum_{k in g} x[m,k]:
// one more pair of MFMAs per subtile and 8 chunks, with B = the lane's 8 biases and A = the
// per-group row sums of the tile split into fp16 hi + lo.
//
// K order.  Inside an MFMA the K positions are permuted identically for A and B: activations
// are staged in LDS with each 16-element chunk stored as [x0 x2 .. x14 | x1 x3 .. x15], which
// is the order of the even / odd codes of one 32-bit word.
#include <hip/hip_fp16.h>

#include "moe_common.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMT = 16;          // rows per M tile
constexpr int kSub = 4;          // 16-row weight subtiles per wave
constexpr int kMaxChunks = 10;   // K <= 2560
constexpr int kGateUp = 0, kDown = 1;

template <int NCH>
struct Tile {
    static constexpr int KP = NCH * 256 + 8;          // LDS row stride (halves); +8 staggers banks
    static constexpr int NB = (NCH + 7) / 8;          // bias MFMA blocks
    static constexpr size_t XS_BYTES = (size_t)kMT * KP * 2;
    static constexpr size_t SX_HALVES = (size_t)NB * kMT * 4 * 8;
    static constexpr size_t LDS_BYTES = XS_BYTES + 2 * SX_HALVES * 2;
};

// Block index -> work item, keeping consecutive work items on one XCD (blocks are dealt to the
// 8 XCDs round robin), so the blocks of one segment share that XCD's L2 for the activations.
__device__ __forceinline__ int xcd_order(int b, int nb) {
    const int per = nb / 8, rem = nb % 8, x = b % 8, i = b / 8;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

// Stage the M tile (rows row0 .. row0+cnt-1 of the source; mapped through row_map when given)
// into LDS in the permuted K order, with the per-group row sums for the bias MFMA.
template <int NCH>
__device__ __forceinline__ void stage_tile(const __half* __restrict__ src, int K, const int32_t* __restrict__ row_map,
                                           int n_src_rows, int row0, int cnt, _Float16* xs, _Float16* sx_hi,
                                           _Float16* sx_lo) {
    using T = Tile<NCH>;
    constexpr int GROUPS = T::NB * 32;                 // groups covered by the bias fragments
    const int kg = K / 64;
    for (int it = threadIdx.x; it < kMT * GROUPS; it += blockDim.x) {
        const int m = it / GROUPS, g = it % GROUPS;
        int srow = -1;
        if (m < cnt) {
            const int r = row0 + m;
            srow = row_map ? row_map[r] : r;
            if (srow < 0 || srow >= n_src_rows) srow = -1;
        }
        uint32_t w[32];
        if (srow >= 0 && g < kg) {
            const uint4* p = reinterpret_cast<const uint4*>(src + (size_t)srow * K + (size_t)g * 64);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint4 v = p[i];
                w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) w[i] = 0;
        }
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            f16x2 v = __builtin_bit_cast(f16x2, w[i]);
            sum += (float)v.x;
            sum += (float)v.y;
        }
        if (g < NCH * 4) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const uint32_t* r = w + 8 * cc;       // x[16cc .. 16cc+15] as 8 words of 2 halves
                uint4 ev, od;
                ev.x = (r[0] & 0xFFFFu) | (r[1] << 16); od.x = (r[0] >> 16) | (r[1] & 0xFFFF0000u);
                ev.y = (r[2] & 0xFFFFu) | (r[3] << 16); od.y = (r[2] >> 16) | (r[3] & 0xFFFF0000u);
                ev.z = (r[4] & 0xFFFFu) | (r[5] << 16); od.z = (r[4] >> 16) | (r[5] & 0xFFFF0000u);
                ev.w = (r[6] & 0xFFFFu) | (r[7] << 16); od.w = (r[6] >> 16) | (r[7] & 0xFFFF0000u);
                uint4* d = reinterpret_cast<uint4*>(xs + (size_t)m * T::KP + g * 64 + cc * 16);
                d[0] = ev;
                d[1] = od;
            }
        }
        const _Float16 hi = (_Float16)sum;
        const _Float16 lo = (_Float16)(sum - (float)hi);
        const int chunk = g >> 2, kq = g & 3, jb = chunk >> 3, j = chunk & 7;
        const int at = ((jb * kMT + m) * 4 + kq) * 8 + j;
        sx_hi[at] = hi;
        sx_lo[at] = lo;
    }
}

__device__ __forceinline__ f16x8 dequant8(uint32_t bits, f16x2 s2) {
    f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 0);
    f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 1);
    f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 2);
    f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 3);
    a *= s2; b *= s2; c *= s2; d *= s2;
    return (f16x8){a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

template <int NCH, int MODE>
__global__ __launch_bounds__(256) void k_q2g_proj(
    const __half* __restrict__ src, int n_src_rows, const int32_t* __restrict__ row_map,
    const int32_t* __restrict__ row_out, int n_out_rows,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_slot, int n_seg, int n_rows,
    const uint8_t* __restrict__ pool, size_t stride, int n_slots, BlobLayout L, int tiles_per_seg,
    __half* __restrict__ out) {
    using T = Tile<NCH>;
    extern __shared__ __align__(16) unsigned char lds[];
    _Float16* xs = reinterpret_cast<_Float16*>(lds);
    _Float16* sx_hi = reinterpret_cast<_Float16*>(lds + T::XS_BYTES);
    _Float16* sx_lo = sx_hi + T::SX_HALVES;

    const int K = MODE == kGateUp ? L.hidden : L.inter;          // contraction length
    const int N = MODE == kGateUp ? L.inter : L.hidden;          // output rows per projection
    const int kg = K / 64;
    const int work = xcd_order(blockIdx.x, gridDim.x);
    const int seg = work / tiles_per_seg, tile = work % tiles_per_seg;
    if (seg >= n_seg) return;
    int r0 = seg_start[seg], r1 = seg_start[seg + 1];
    r0 = r0 < 0 ? 0 : (r0 > n_rows ? n_rows : r0);
    r1 = r1 < r0 ? r0 : (r1 > n_rows ? n_rows : r1);
    const int slot = seg_slot ? seg_slot[seg] : seg;
    if (r1 == r0 || slot < 0 || slot >= n_slots) return;          // uniform per block

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n = lane & 15, kq = lane >> 4;
    const uint8_t* blob = pool + (size_t)slot * stride;
    const size_t code_row = (size_t)K / 4, sb_row = (size_t)kg;   // bytes / words per weight row

    const uint8_t* codes[kSub];
    const uint32_t* sbp[kSub];
    bool rv[kSub];
    int col[kSub];
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        size_t co, so;
        int row;
        if (MODE == kGateUp) {
            row = tile * 128 + wv * 32 + (s >> 1) * 16 + n;
            co = (s & 1) ? L.up_codes : L.gate_codes;
            so = (s & 1) ? L.up_sb : L.gate_sb;
        } else {
            row = tile * 256 + wv * 64 + s * 16 + n;
            co = L.down_codes;
            so = L.down_sb;
        }
        col[s] = row;
        rv[s] = row < N;
        const int rr = rv[s] ? row : 0;
        codes[s] = blob + co + (size_t)rr * code_row;
        sbp[s] = reinterpret_cast<const uint32_t*>(blob + so) + (size_t)rr * sb_row;
    }

    for (int m0 = r0; m0 < r1; m0 += kMT) {
        const int cnt = (r1 - m0) < kMT ? (r1 - m0) : kMT;
        __syncthreads();                                   // previous tile's LDS reads done
        stage_tile<NCH>(src, K, row_map, n_src_rows, m0, cnt, xs, sx_hi, sx_lo);
        __syncthreads();

        f32x4 acc[kSub];
#pragma unroll
        for (int s = 0; s < kSub; ++s) acc[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
        f16x8 bias[kSub];
#pragma unroll
        for (int s = 0; s < kSub; ++s) bias[s] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};

        uint4 cw[kSub], nw[kSub];
        uint32_t sw[kSub], ns[kSub];
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
            const bool ok = rv[s] && kq < kg;
            cw[s] = ok ? *reinterpret_cast<const uint4*>(codes[s] + kq * 16) : make_uint4(0, 0, 0, 0);
            sw[s] = ok ? sbp[s][kq] : 0u;
        }
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (j + 1 < NCH) {
                const int g = 4 * (j + 1) + kq;
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    const bool ok = rv[s] && g < kg;
                    nw[s] = ok ? *reinterpret_cast<const uint4*>(codes[s] + (size_t)g * 16) : make_uint4(0, 0, 0, 0);
                    ns[s] = ok ? sbp[s][g] : 0u;
                }
            }
            f16x2 s2[kSub];
#pragma unroll
            for (int s = 0; s < kSub; ++s) {
                const f16x2 sb = __builtin_bit_cast(f16x2, sw[s]);
                const _Float16 two_s = sb.x * (_Float16)2.0f;
                s2[s] = (f16x2){two_s, two_s};
                bias[s][j & 7] = sb.y;
            }
            const _Float16* arow = xs + (size_t)n * T::KP + (size_t)(16 * j + 4 * kq) * 16;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f16x8 a_ev = *reinterpret_cast<const f16x8*>(arow + q * 16);
                const f16x8 a_od = *reinterpret_cast<const f16x8*>(arow + q * 16 + 8);
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    const uint32_t w = q == 0 ? cw[s].x : q == 1 ? cw[s].y : q == 2 ? cw[s].z : cw[s].w;
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_ev, dequant8(w & 0x33333333u, s2[s]), acc[s], 0, 0, 0);
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_od, dequant8((w >> 2) & 0x33333333u, s2[s]), acc[s], 0, 0, 0);
                }
            }
            if ((j & 7) == 7 || j == NCH - 1) {
                const int at = (((j >> 3) * kMT + n) * 4 + kq) * 8;
                const f16x8 ah = *reinterpret_cast<const f16x8*>(sx_hi + at);
                const f16x8 al = *reinterpret_cast<const f16x8*>(sx_lo + at);
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bias[s], acc[s], 0, 0, 0);
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bias[s], acc[s], 0, 0, 0);
                    bias[s] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
            if (j + 1 < NCH) {
#pragma unroll
                for (int s = 0; s < kSub; ++s) { cw[s] = nw[s]; sw[s] = ns[s]; }
            }
        }

        // Epilogue: lane holds rows 4*kq + i (i = 0..3) of column n of each subtile.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * kq + i;
            if (m >= cnt) continue;
            const int r = m0 + m;
            if (MODE == kGateUp) {
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    if (!rv[2 * p]) continue;
                    const float g = acc[2 * p][i], u = acc[2 * p + 1][i];
                    out[(size_t)r * N + col[2 * p]] = __float2half_rn(g / (1.0f + __expf(-g)) * u);
                }
            } else {
                const int orow = row_out ? row_out[r] : r;
                if (orow < 0 || orow >= n_out_rows) continue;
#pragma unroll
                for (int s = 0; s < kSub; ++s)
                    if (rv[s]) out[(size_t)orow * N + col[s]] = __float2half_rn(acc[s][i]);
            }
        }
    }
}

template <int NCH, int MODE>
int launch_proj(const __half* src, int n_src_rows, const int32_t* row_map, const int32_t* row_out, int n_out_rows,
                const int32_t* seg_start, const int32_t* seg_slot, int n_seg, int n_rows, const uint8_t* pool,
                size_t stride, int n_slots, const BlobLayout& L, __half* out, hipStream_t s) {
    using T = Tile<NCH>;
    static bool attr_set = false;
    if (!attr_set) {
        HIP_TRY(hipFuncSetAttribute((const void*)k_q2g_proj<NCH, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)T::LDS_BYTES));
        attr_set = true;
    }
    const int N = MODE == kGateUp ? L.inter : L.hidden;
    const int rows_per_block = MODE == kGateUp ? 128 : 256;
    const int tiles = (N + rows_per_block - 1) / rows_per_block;
    const long long nb = (long long)n_seg * tiles;
    if (nb <= 0) return 0;
    if (nb > 0x7FFFFFFFLL) { moe_set_error("grouped q2: grid too large"); return -1; }
    MOE_LAUNCH(MODE == kGateUp ? TK_PF_GATE_UP : TK_PF_DOWN, (k_q2g_proj<NCH, MODE>), dim3((unsigned)nb), dim3(256),
               T::LDS_BYTES, s, src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg, n_rows, pool,
               stride, n_slots, L, tiles, out);
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int MODE>
int dispatch_proj(int K, const __half* src, int n_src_rows, const int32_t* row_map, const int32_t* row_out,
                  int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg, int n_rows,
                  const uint8_t* pool, size_t stride, int n_slots, const BlobLayout& L, __half* out, hipStream_t s) {
    switch ((K + 255) / 256) {
#define PF_CASE(c) \
    case c: return launch_proj<c, MODE>(src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg, \
                                        n_rows, pool, stride, n_slots, L, out, s);
        PF_CASE(1) PF_CASE(2) PF_CASE(3) PF_CASE(4) PF_CASE(5)
        PF_CASE(6) PF_CASE(7) PF_CASE(8) PF_CASE(9) PF_CASE(10)
#undef PF_CASE
        default: moe_set_error("grouped q2: contraction length %d unsupported (<= %d)", K, kMaxChunks * 256); return -1;
    }
}

bool check_grouped(const char* who, int hidden, int inter, int group, int n_seg, int n_rows, const void* pool,
                   size_t stride, int n_slots, const void* a, const void* b, const void* c) {
    if (group != 64) { moe_set_error("%s: group=%d unsupported (kernels take group 64)", who, group); return false; }
    if (hidden <= 0 || inter <= 0 || hidden % 64 || inter % 64 || hidden > kMaxChunks * 256 || inter > kMaxChunks * 256) {
        moe_set_error("%s: hidden=%d inter=%d must be multiples of 64 in 64..%d", who, hidden, inter, kMaxChunks * 256);
        return false;
    }
    if (n_seg < 0 || n_rows < 0) { moe_set_error("%s: negative segment or row count", who); return false; }
    if (n_seg > 0 && (!pool || n_slots <= 0 || !a || !b || !c)) {
        moe_set_error("%s: empty pool or null pointer", who);
        return false;
    }
    BlobLayout L = blob_layout(hidden, inter, group);
    if (n_seg > 0 && stride < L.bytes) {
        moe_set_error("%s: expert stride %zu < blob bytes %zu", who, stride, L.bytes);
        return false;
    }
    return true;
}

__global__ __launch_bounds__(256) void k_pair_combine(const __half* __restrict__ y, const __half* __restrict__ scores,
                                                      const __half* __restrict__ residual, int k, int hidden,
                                                      float* __restrict__ out) {
    const int t = blockIdx.y;
    const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 2;
    if (c >= hidden) return;
    float a0 = 0.f, a1 = 0.f;
    for (int j = 0; j < k; ++j) {
        const float sj = __half2float(scores[(size_t)t * k + j]);
        const __half* row = y + ((size_t)t * k + j) * hidden;
        a0 += sj * __half2float(row[c]);
        if (c + 1 < hidden) a1 += sj * __half2float(row[c + 1]);
    }
    if (residual) {
        a0 += __half2float(residual[(size_t)t * hidden + c]);
        if (c + 1 < hidden) a1 += __half2float(residual[(size_t)t * hidden + c + 1]);
    }
    out[(size_t)t * hidden + c] = a0;
    if (c + 1 < hidden) out[(size_t)t * hidden + c + 1] = a1;
}

}  // namespace

int launch_q2_grouped_gate_up(const __half* x, int n_tokens, const int32_t* row_token, int n_rows,
                              const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const uint8_t* pool,
                              size_t stride, int n_slots, int hidden, int inter, int group, __half* h_out,
                              hipStream_t s) {
    if (!check_grouped("q2_grouped_gate_up", hidden, inter, group, n_seg, n_rows, pool, stride, n_slots, x, seg_start,
                       h_out))
        return -1;
    if (n_seg == 0 || n_rows == 0) return 0;
    BlobLayout L = blob_layout(hidden, inter, group);
    return dispatch_proj<kGateUp>(hidden, x, n_tokens, row_token, nullptr, 0, seg_start, seg_slot, n_seg, n_rows, pool,
                                  stride, n_slots, L, h_out, s);
}

int launch_q2_grouped_down(const __half* h, int n_rows, const int32_t* row_out, int n_out_rows,
                           const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const uint8_t* pool,
                           size_t stride, int n_slots, int hidden, int inter, int group, __half* y_out, hipStream_t s) {
    if (!check_grouped("q2_grouped_down", hidden, inter, group, n_seg, n_rows, pool, stride, n_slots, h, seg_start,
                       y_out))
        return -1;
    if (n_seg == 0 || n_rows == 0) return 0;
    BlobLayout L = blob_layout(hidden, inter, group);
    return dispatch_proj<kDown>(inter, h, n_rows, nullptr, row_out, row_out ? n_out_rows : n_rows, seg_start, seg_slot,
                                n_seg, n_rows, pool, stride, n_slots, L, y_out, s);
}

int launch_pair_combine(const __half* y, const __half* scores, const __half* residual, int n_tokens, int k,
                        int hidden, float* out, hipStream_t s) {
    if (n_tokens < 0 || k <= 0 || hidden <= 0 || n_tokens > 65535) {
        moe_set_error("pair_combine: n_tokens=%d (<= 65535) k=%d hidden=%d", n_tokens, k, hidden);
        return -1;
    }
    if (n_tokens == 0) return 0;
    if (!y || !scores || !out) { moe_set_error("pair_combine: null pointer"); return -1; }
    dim3 grid(((hidden + 1) / 2 + 255) / 256, n_tokens);
    MOE_LAUNCH(TK_COMBINE, k_pair_combine, grid, dim3(256), 0, s, y, scores, residual, k, hidden, out);
    HIP_TRY(hipGetLastError());
    return 0;
}
