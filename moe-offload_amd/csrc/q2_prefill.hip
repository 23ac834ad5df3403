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
// Tiling.  The rows of a segment form M tiles of 16 (v_mfma_f32_16x16x32_f16), taken in
// batches of up to 2 tiles.  A block of 4 waves works on one segment and one slice of weight
// rows; each wave owns 4 subtiles of 16 weight rows (gate/up: 2 x 16 rows of each projection =
// 128 intermediate rows per block; down: 4 x 16 = 256 output rows).  Per 256-wide K chunk j a
// lane (n = lane & 15, kq = lane >> 4) loads group 4j + kq of weight row n (one 16-byte load of
// 64 codes plus the (scale, bias) word), dequantises it once and multiplies it into every tile
// of the batch; the chunk's activations of the batch's rows are staged in LDS (each thread
// stages 2 units of 16 bytes per tile).  The next chunk's weights and activations are loaded
// while the current chunk is multiplied.  The gate/up grid holds every (segment, slice) item
// twice: segments of more than one batch run in the first half, so their blocks, the longest,
// are dispatched before the rest.  At K = 2048 gate/up runs in the whole-K form instead
// (k_q2g_gu_wk: per M tile, each wave's weight subtiles requested over the whole K at once, the
// tile's activations staged once; the same two-pass grid, long segments first).  At K = 512 down
// runs in the whole-K form as well (k_q2g_dn_wk: each wave's 4 subtiles loaded once over the whole
// K and kept in registers while the segment's M tiles pass through LDS; two-pass grid).
//
// Dequantisation.  A 2-bit code in the low bits of a nibble is the fp4 (e2m1) value q/2, so
// w & 0x33333333 (even codes) and (w >> 2) & 0x33333333 (odd codes) are 8 fp4 values each;
// v_cvt_scalef32_pk_f16_fp4 turns a byte into two exact halves, and one v_pk_fma_f16 with
// (2*scale, bias) gives the fp16 weight scale*q + bias rounded once (MLX's dequantised weight).
//
// K order.  Inside an MFMA the K positions are permuted identically for A and B: the even codes
// of a 32-bit word pair with activations [x0 x2 .. x14] of its 16 inputs and the odd codes with
// [x1 x3 .. x15]; the activation halves are regrouped in registers with v_perm_b32.
//
// Weight sources (SBF): 0 = the blob pool, (scale, bias) interleaved as fp16 words; 1 / 2 = the
// reference's 9 tensors (loader.py:332-406: codes, scales, biases in pools of their own), scales and
// biases fp16 / bf16, turned into the same (scale, bias) fp16 words as they are loaded (bf16 ->
// fp16 is exact for the normal range of fp16).
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

// Block index -> work item, keeping consecutive work items on one XCD (blocks are dealt to the
// 8 XCDs round robin), so the blocks of one segment share that XCD's L2 for the activations.
__device__ __forceinline__ int xcd_order(int b, int nb) {
    const int per = nb / 8, rem = nb % 8, x = b % 8, i = b / 8;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

__device__ __forceinline__ f16x8 dequant8(uint32_t bits, f16x2 s2, f16x2 b2) {
    f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 0);
    f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 1);
    f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 2);
    f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(bits, 1.0f, 3);
    a = __builtin_elementwise_fma(a, s2, b2);
    b = __builtin_elementwise_fma(b, s2, b2);
    c = __builtin_elementwise_fma(c, s2, b2);
    d = __builtin_elementwise_fma(d, s2, b2);
    return (f16x8){a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// 16 activations x[0..15] (two 16-byte words, natural order) -> (even, odd) MFMA fragments.
__device__ __forceinline__ void split_even_odd(uint4 lo, uint4 hi, f16x8& ev, f16x8& od) {
    const uint32_t r[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    uint32_t e[4], o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        e[i] = __builtin_amdgcn_perm(r[2 * i + 1], r[2 * i], 0x05040100u);
        o[i] = __builtin_amdgcn_perm(r[2 * i + 1], r[2 * i], 0x07060302u);
    }
    ev = __builtin_bit_cast(f16x8, make_uint4(e[0], e[1], e[2], e[3]));
    od = __builtin_bit_cast(f16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

// Block barrier ordering LDS only (the loop shares nothing else between waves): the fences
// are limited to the local address space, so a wait at the barrier covers LDS accesses and
// not the global loads in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// M tiles multiplied per pass over a segment's weights: 2 for both projections.  Gate/up: the
// registers 4 tiles would hold leave no room for the next chunk's activations in flight (only
// segments of more than 32 rows take a second pass; 128 us per 512-token chunk against 133 with
// 4 tiles and the activations loaded after the multiply).  Down: a short K, every pass is two
// chunks of dependent round trips (62 us at 2 tiles, 70 at 1 and at 4).
template <int MODE>
constexpr int max_mt() { return 2; }

// One (scale, bias) fp16 word from two 16-bit values of the 9-tensor form.
template <int SBF>
__device__ __forceinline__ uint32_t sb_word(uint32_t sc, uint32_t bi) {
    if constexpr (SBF == 2) {
        sc = __half_as_ushort(__float2half_rn(__uint_as_float(sc << 16)));
        bi = __half_as_ushort(__float2half_rn(__uint_as_float(bi << 16)));
    }
    return (sc & 0xFFFFu) | (bi << 16);
}

// Gate/up of one M tile (at most 16 rows r0 .. r0 + rows - 1 of a segment) and one 128-row slice,
// the weight rows streamed whole: each wave owns two (gate, up) pairs of 16-row subtiles and
// requests a pair's whole K at once (lane (n, kq) loads groups GPL*kq .. GPL*kq + GPL - 1 of row
// n: 16 rows x 64 * GPL contiguous bytes per subtile), the second pair's loads issued before the
// first pair is multiplied.  The tile's activation rows are staged in LDS once for the whole K,
// already split into the MFMA's even / odd input fragments: one barrier per tile, after which the
// waves run independently.  A K position of an MFMA pairs lane group kq's group GPL*kq + i with
// the same inputs on the A side; the even/odd code split inside a word is the one of k_q2g_proj.
// Bit for bit this is not k_q2g_proj's sum order (another K order inside the MFMAs).
template <int GPL, int SBF>
__device__ __forceinline__ void gu_whole_k(const __half* __restrict__ src, int n_src_rows,
                                           const int32_t* __restrict__ row_map, int r0, int rows, int slot,
                                           int tile, const Q2Experts& E, int inter, __half* __restrict__ out,
                                           uint4* __restrict__ a_lds) {
    constexpr int K = 256 * GPL;
    constexpr int kg = 4 * GPL;                       // groups per weight row
    constexpr int UPR = K / 8;                        // 16-byte units per activation row
    constexpr int kPairsPerThread = UPR / 32;         // unit pairs a thread stages
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));                       // per call: no address is kept across calls
    const int lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n = lane & 15, kq = lane >> 4;

    // thread t stages unit pairs (2 pv, 2 pv + 1), pv = (t & 15) + 16 c, of row t >> 4; rows past
    // the segment and out-of-range source rows are staged as zeros (a_lds: unit v of row m at
    // m * UPR + (v ^ m), so the 16 lanes reading one unit column hit distinct banks)
    const int sm = t >> 4, sv0 = t & 15;
    int srow = -1;
    if (sm < rows) {
        srow = row_map ? row_map[r0 + sm] : r0 + sm;
        if (srow < 0 || srow >= n_src_rows) srow = -1;
    }
    uint4 xv[2 * kPairsPerThread];
    {
        const uint4* xr = reinterpret_cast<const uint4*>(src + (size_t)(srow < 0 ? 0 : srow) * K);
#pragma unroll
        for (int c = 0; c < kPairsPerThread; ++c) {
            xv[2 * c] = xr[2 * (sv0 + 16 * c)];
            xv[2 * c + 1] = xr[2 * (sv0 + 16 * c) + 1];
        }
    }

    // pair pp: gate and up rows base .. base + 15 (inter is a multiple of 64: a subtile is wholly
    // in range or wholly out; one that is out re-reads the last subtile and is not written)
    const Q2Proj& Pg = E.p[0];
    const Q2Proj& Pu = E.p[1];
    const size_t code_row = (size_t)K / 4;
    auto pair_base = [&](int pp) { return tile * 128 + (wv * 2 + pp) * 16; };
    auto load_pair = [&](int pp, uint4 (&c)[2][GPL], uint32_t (&wd)[2][GPL]) {
        int base = pair_base(pp);
        base = base < inter ? base : inter - 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const Q2Proj& P = h ? Pu : Pg;
            const uint8_t* cr = P.w + (size_t)slot * P.w_stride + (size_t)(base + n) * code_row + (size_t)(GPL * kq) * 16;
#pragma unroll
            for (int i = 0; i < GPL; ++i) c[h][i] = *reinterpret_cast<const uint4*>(cr + (size_t)i * 16);
            if constexpr (SBF == 0) {
                static_assert(GPL % 4 == 0, "whole 16-byte scale/bias pieces");
                const uint32_t* sr = reinterpret_cast<const uint32_t*>(P.s + (size_t)slot * P.s_stride) +
                                     (size_t)(base + n) * kg + GPL * kq;
#pragma unroll
                for (int i = 0; i < GPL / 4; ++i) {
                    const uint4 v = reinterpret_cast<const uint4*>(sr)[i];
                    wd[h][4 * i] = v.x;
                    wd[h][4 * i + 1] = v.y;
                    wd[h][4 * i + 2] = v.z;
                    wd[h][4 * i + 3] = v.w;
                }
            } else {
                static_assert(GPL % 8 == 0, "whole 16-byte scale / bias pieces");
                const uint16_t* scr = reinterpret_cast<const uint16_t*>(P.s + (size_t)slot * P.s_stride) +
                                      (size_t)(base + n) * kg + GPL * kq;
                const uint16_t* bir = reinterpret_cast<const uint16_t*>(P.b + (size_t)slot * P.b_stride) +
                                      (size_t)(base + n) * kg + GPL * kq;
#pragma unroll
                for (int i = 0; i < GPL / 8; ++i) {
                    const uint4 sc = reinterpret_cast<const uint4*>(scr)[i];
                    const uint4 bi = reinterpret_cast<const uint4*>(bir)[i];
                    const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w}, biw[4] = {bi.x, bi.y, bi.z, bi.w};
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) {
                        wd[h][8 * i + 2 * k2] = sb_word<SBF>(scw[k2] & 0xFFFFu, biw[k2] & 0xFFFFu);
                        wd[h][8 * i + 2 * k2 + 1] = sb_word<SBF>(scw[k2] >> 16, biw[k2] >> 16);
                    }
                }
            }
        }
    };
    auto multiply = [&](int pp, const uint4 (&c)[2][GPL], const uint32_t (&wd)[2][GPL]) {
        f32x4 accg = (f32x4){0.f, 0.f, 0.f, 0.f}, accu = (f32x4){0.f, 0.f, 0.f, 0.f};
        const uint4* arow = a_lds + n * UPR;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            f16x2 s2[2], b2[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f16x2 sb = __builtin_bit_cast(f16x2, wd[h][i]);
                const _Float16 two_s = sb.x * (_Float16)2.0f;
                s2[h] = (f16x2){two_s, two_s};
                b2[h] = (f16x2){sb.y, sb.y};
            }
            const int u0 = 8 * (GPL * kq + i);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int v = u0 + 2 * q;
                const f16x8 a_ev = __builtin_bit_cast(f16x8, arow[v ^ n]);
                const f16x8 a_od = __builtin_bit_cast(f16x8, arow[(v + 1) ^ n]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 cv = c[h][i];
                    const uint32_t wq = q == 0 ? cv.x : q == 1 ? cv.y : q == 2 ? cv.z : cv.w;
                    const f16x8 b_ev = dequant8(wq & 0x33333333u, s2[h], b2[h]);
                    const f16x8 b_od = dequant8((wq >> 2) & 0x33333333u, s2[h], b2[h]);
                    f32x4& acc = h ? accu : accg;
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_ev, b_ev, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_od, b_od, acc, 0, 0, 0);
                }
            }
        }
        // lane holds rows 4 kq + i of column n
        const int base = pair_base(pp);
        if (base < inter) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * kq + i;
                if (m < rows) {
                    const float g = accg[i], u = accu[i];
                    out[(size_t)(r0 + m) * inter + base + n] = __float2half_rn(g / (1.0f + __expf(-g)) * u);
                }
            }
        }
    };

    uint4 cw0[2][GPL], cw1[2][GPL];
    uint32_t sw0[2][GPL], sw1[2][GPL];
    load_pair(0, cw0, sw0);                           // after the activations: those retire first
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < kPairsPerThread; ++c) {
        const int v = 2 * (sv0 + 16 * c);
        f16x8 ev, od;
        split_even_odd(xv[2 * c], xv[2 * c + 1], ev, od);
        const uint4 e4 = __builtin_bit_cast(uint4, ev), o4 = __builtin_bit_cast(uint4, od);
        a_lds[sm * UPR + (v ^ sm)] = srow >= 0 ? e4 : make_uint4(0, 0, 0, 0);
        a_lds[sm * UPR + ((v + 1) ^ sm)] = srow >= 0 ? o4 : make_uint4(0, 0, 0, 0);
    }
    lds_barrier();
    load_pair(1, cw1, sw1);
    __builtin_amdgcn_sched_barrier(0);                // pair 1's loads go out before pair 0's multiply
    multiply(0, cw0, sw0);
    // both pairs read the same activation fragments; without this fence the compiler keeps pair
    // 0's 256 fragment registers for pair 1 and spills
    asm volatile("" ::: "memory");
    multiply(1, cw1, sw1);
}

template <int GPL, int SBF>
__global__ __launch_bounds__(256, 2) void k_q2g_gu_wk(
    const __half* __restrict__ src, int n_src_rows, const int32_t* __restrict__ row_map,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_slot, int n_seg, int n_rows,
    Q2Experts E, int n_slots, int inter, int tiles_per_seg, __half* __restrict__ out) {
    __shared__ uint4 a_lds[16 * 32 * GPL];
    // two passes over the (segment, slice) items: segments of more than one M tile first (their
    // blocks run longest); a block takes its segment's tiles one after the other, each tile's
    // weights loaded again (from L2 while they are still there), since both pairs' weights held
    // across tiles would not fit beside a tile's staging
    const int items = n_seg * tiles_per_seg;
    const int pass = (int)blockIdx.x >= items ? 1 : 0;
    const int work = xcd_order((int)blockIdx.x - pass * items, items);
    const int seg = work / tiles_per_seg, tile = work % tiles_per_seg;
    if (seg >= n_seg) return;
    int r0 = seg_start[seg], r1 = seg_start[seg + 1];
    r0 = r0 < 0 ? 0 : (r0 > n_rows ? n_rows : r0);
    r1 = r1 < r0 ? r0 : (r1 > n_rows ? n_rows : r1);
    const int slot = seg_slot ? seg_slot[seg] : seg;
    if (r1 == r0 || slot < 0 || slot >= n_slots) return;
    if ((pass == 0) != (r1 - r0 > kMT)) return;
#pragma unroll 1
    for (int m0 = r0; m0 < r1; m0 += kMT) {          // block-uniform
        if (m0 > r0) __syncthreads();                // every wave is done with the previous tile
        int slot_i = slot;                           // opaque: the weights are loaded again per tile
        asm volatile("" : "+s"(slot_i) : : "memory");
        gu_whole_k<GPL, SBF>(src, n_src_rows, row_map, m0, (r1 - m0) < kMT ? (r1 - m0) : kMT, slot_i, tile, E, inter,
                             out, a_lds);
    }
}

template <int NCH, int MODE, bool SBL, int SBF>
__global__ __launch_bounds__(256, 2) void k_q2g_proj(
    const __half* __restrict__ src, int n_src_rows, const int32_t* __restrict__ row_map,
    const int32_t* __restrict__ row_out, int n_out_rows,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_slot, int n_seg, int n_rows,
    Q2Experts E, int n_slots, int hidden, int inter, int tiles_per_seg, __half* __restrict__ out) {
    constexpr int kMaxMT = max_mt<MODE>();
    constexpr bool kPrefetch = MODE == kGateUp;        // a short K (down) gains nothing from it
    const int K = MODE == kGateUp ? hidden : inter;              // contraction length
    const int N = MODE == kGateUp ? inter : hidden;              // output rows per projection
    const int kg = K / 64;
    // Gate/up runs two passes over the (segment, slice) items: the first takes the segments that
    // need more than one batch of M tiles, whose blocks run longest, so that they are dispatched
    // first; the second takes the rest (each block of a pass that is not its own exits at once).
    int work, pass = 0;
    if constexpr (MODE == kGateUp) {
        const int items = n_seg * tiles_per_seg;
        pass = (int)blockIdx.x >= items ? 1 : 0;
        work = xcd_order((int)blockIdx.x - pass * items, items);
    } else {
        work = xcd_order(blockIdx.x, gridDim.x);
    }
    const int seg = work / tiles_per_seg, tile = work % tiles_per_seg;
    if (seg >= n_seg) return;
    int r0 = seg_start[seg], r1 = seg_start[seg + 1];
    r0 = r0 < 0 ? 0 : (r0 > n_rows ? n_rows : r0);
    r1 = r1 < r0 ? r0 : (r1 > n_rows ? n_rows : r1);
    const int slot = seg_slot ? seg_slot[seg] : seg;
    if (r1 == r0 || slot < 0 || slot >= n_slots) return;
    if constexpr (MODE == kGateUp) {
        if ((pass == 0) != (r1 - r0 > kMT * kMaxMT)) return;
    }

    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kq = lane >> 4;
    const size_t code_row = (size_t)K / 4, sb_row = (size_t)kg;   // bytes / (scale, bias) pairs per weight row

    // Weight row of lane n in subtile s = base_s + n: a wave-uniform base per subtile plus one
    // per-lane offset shared by all subtiles.
    const uint8_t* codes[kSub];
    const uint32_t* sbp[kSub];                 // SBF 0: (scale, bias) words of the subtile's rows
    const uint16_t* scp[kSub];                 // SBF 1 / 2: scales and biases
    const uint16_t* bip[kSub];
    bool rv[kSub];
    int col[kSub];
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        int base, p;
        if (MODE == kGateUp) {
            base = tile * 128 + wv * 32 + (s >> 1) * 16;
            p = (s & 1) ? 1 : 0;
        } else {
            base = tile * 256 + wv * 64 + s * 16;
            p = 2;
        }
        col[s] = base + n;
        // N is a multiple of 64, so a subtile is wholly in range or wholly out; one that is out
        // reads the last in-range subtile (unconditional loads) and is never written
        rv[s] = base < N;
        if (base >= N) base = N - 16;
        const Q2Proj& P = E.p[p];
        codes[s] = P.w + (size_t)slot * P.w_stride + (size_t)base * code_row;
        sbp[s] = reinterpret_cast<const uint32_t*>(P.s + (size_t)slot * P.s_stride) + (size_t)base * sb_row;
        scp[s] = reinterpret_cast<const uint16_t*>(P.s + (size_t)slot * P.s_stride) + (size_t)base * sb_row;
        bip[s] = reinterpret_cast<const uint16_t*>(P.b + (size_t)slot * P.b_stride) + (size_t)base * sb_row;
    }
    const uint32_t lane_code0 = (uint32_t)((size_t)n * code_row + (size_t)kq * 16);
    const uint32_t lane_sb0 = (uint32_t)((size_t)n * sb_row + kq);

    // Scale/bias words.  With SBL (gate/up, K a multiple of 256 and at least 512: rows of 4 k
    // words, so every 16-byte piece below is aligned) each wave loads them four chunks at a time
    // into its own LDS area, one 16-byte piece per lane and subtile: lane (n, q) loads groups
    // 16 jj + 4 q .. + 3 of its row n (a piece past the row's end is moved back to its last 4
    // groups), and chunk j = 4 jj + c reads group 4 j + kq from the piece of lane (n, c).  One
    // such load touches as many cache lines as one of the per-chunk 4-byte loads it replaces,
    // and there are four times fewer of them.  The pieces of block jj + 1 are loaded after chunk
    // 4 jj is multiplied and written to LDS by the staging of chunk 4 jj + 1 (the compiler moves
    // that write up to the loads, so they are waited for once per block); two buffers, so block
    // jj + 1 lands while block jj is read.  Without SBL the words are loaded with the codes.
    constexpr bool kSbLds = SBL;
    static_assert(!SBL || NCH >= 2, "the LDS path needs K >= 512");
    __shared__ uint32_t sb_lds[kSbLds ? 2 : 1][4][kSub][kSbLds ? 256 : 1];
    const uint32_t lane_row_sb = (uint32_t)((size_t)n * sb_row);
    auto sb_piece = [&](int jj, int q) {                       // first group of lane (., q)'s piece
        const int g0 = 16 * jj + 4 * q;
        return g0 + 4 <= kg ? g0 : kg - 4;
    };
    // a block's pieces on their way to LDS, one named register set per subtile (as an array the
    // compiler keeps them in memory: in LDS, or in scratch with a wait right after the loads)
    uint4 sbn0, sbn1, sbn2, sbn3;
    static_assert(kSub == 4, "one named piece per subtile");
    auto sbn = [&](int s) -> uint4& { return s == 0 ? sbn0 : s == 1 ? sbn1 : s == 2 ? sbn2 : sbn3; };
    auto fetch_sb = [&](int jj) {
        const int gs = sb_piece(jj, kq);
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
            if constexpr (SBF == 0) {
                sbn(s) = *reinterpret_cast<const uint4*>(sbp[s] + lane_row_sb + gs);
            } else {                           // 4 scales and 4 biases (8-byte aligned: kg % 4 == 0)
                const uint2 sc = *reinterpret_cast<const uint2*>(scp[s] + lane_row_sb + gs);
                const uint2 bi = *reinterpret_cast<const uint2*>(bip[s] + lane_row_sb + gs);
                sbn(s) = make_uint4(sb_word<SBF>(sc.x & 0xFFFFu, bi.x & 0xFFFFu), sb_word<SBF>(sc.x >> 16, bi.x >> 16),
                                    sb_word<SBF>(sc.y & 0xFFFFu, bi.y & 0xFFFFu), sb_word<SBF>(sc.y >> 16, bi.y >> 16));
            }
        }
    };
    auto put_sb = [&](int jj) {
#pragma unroll
        for (int s = 0; s < kSub; ++s) reinterpret_cast<uint4*>(&sb_lds[jj & 1][wv][s][0])[lane] = sbn(s);
    };

    // The segment's rows are taken in batches of up to kMaxMT M tiles (32 rows); within a batch
    // every K chunk's weights are loaded and dequantised once and multiplied into every tile, so
    // a long segment costs one pass over its weights per batch, not one per tile.
    //
    // Activation chunks are staged in LDS, shared by the 4 waves: per tile 16 rows x 32 units of
    // 16 bytes (256 inputs), unit v of row m stored at m * 32 + (v ^ m) so that the 16 lanes
    // reading one unit column hit distinct banks.  Each thread stages 2 units per tile.
    __shared__ uint4 a_lds[kMaxMT][kMT * 32];
    const int t = threadIdx.x;
    const int sm0 = t >> 5, sm1 = sm0 + 8, sv = t & 31;       // the two units this thread stages

    for (int b0 = r0; b0 < r1; b0 += kMT * kMaxMT) {
        const int rows = (r1 - b0) < kMT * kMaxMT ? (r1 - b0) : kMT * kMaxMT;
        const int mts = (rows + kMT - 1) / kMT;                // tiles in this batch (wave-uniform)
        // The weight loads do not depend on the batch; an opaque copy of the lane offsets keeps
        // the compiler from hoisting (and holding) a short K's whole weight slice across batches.
        uint32_t lane_code = lane_code0, lane_sb = lane_sb0;
        asm volatile("" : "+v"(lane_code), "+v"(lane_sb));
        // source rows of the staged units; a row past the segment or naming an out-of-range
        // source row is staged as zeros
        int sr[kMaxMT][2];
#pragma unroll
        for (int mt = 0; mt < kMaxMT; ++mt) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = mt * kMT + (h ? sm1 : sm0);
                int v = -1;
                if (m < rows) {
                    const int r = b0 + m;
                    v = row_map ? row_map[r] : r;
                    if (v < 0 || v >= n_src_rows) v = -1;
                }
                sr[mt][h] = v;
            }
        }

        f32x4 acc[kMaxMT][kSub];
#pragma unroll
        for (int mt = 0; mt < kMaxMT; ++mt)
#pragma unroll
            for (int s = 0; s < kSub; ++s) acc[mt][s] = (f32x4){0.f, 0.f, 0.f, 0.f};

        uint4 cwa[kSub], cwb[kSub];                            // weights of the current / next chunk
        uint32_t swa[kSub], swb[kSub];
        uint4 xs[kMaxMT][2];                                   // staged activation units in flight
        // Loads are unconditional from clamped in-range addresses and nothing masks them where
        // they land: a load whose value is selected right away is sunk into a branch by the
        // compiler, which then waits for it at the join and serialises a chunk's round trips.
        // Groups past K (a K that is not a multiple of 256) read group kg - 1: their activations
        // are staged as zeros, so those finite weights add nothing.  Rows past the segment and
        // out-of-range source rows are zeroed when staged.
        auto load_w = [&](int j, uint4 (&cw)[kSub], uint32_t (&sw)[kSub]) {
            const bool gv = 4 * j + kq < kg;
            const int gdelta = gv ? 0 : (kg - 1) - (4 * j + kq);      // clamp to group kg - 1
#pragma unroll
            for (int s = 0; s < kSub; ++s) {
                cw[s] = *reinterpret_cast<const uint4*>(codes[s] + lane_code + (size_t)j * 64 + (ptrdiff_t)gdelta * 16);
                if constexpr (!kSbLds) {
                    const uint32_t gi = lane_sb + 4 * j + gdelta;
                    if constexpr (SBF == 0) sw[s] = sbp[s][gi];
                    else sw[s] = sb_word<SBF>(scp[s][gi], bip[s][gi]);
                }
            }
        };
        // After chunk j's multiply (j = 4 jj): the loads of the next block's words (needed from
        // chunk 4 jj + 4 on); staging chunk j + 1 writes them to the buffer of block jj - 1, which
        // the wave's reads have left.
        auto next_sb_block = [&](int j) {
            if constexpr (kSbLds) {
                if ((j & 3) == 0 && 4 * ((j >> 2) + 1) < NCH) fetch_sb((j >> 2) + 1);
            }
        };
        auto stage_sb = [&](int j) {
            if constexpr (kSbLds) {
                if (j == 0) put_sb(0);
                else if ((j & 3) == 1 && 4 * ((j >> 2) + 1) < NCH) put_sb((j >> 2) + 1);
            }
        };
        auto load_x = [&](int j) {
            const int u = 32 * j + sv;                         // 16-byte unit within the row
            const int uc = u * 8 < K ? u : K / 8 - 1;
#pragma unroll
            for (int mt = 0; mt < kMaxMT; ++mt) {
                if (mt >= mts) break;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int v = sr[mt][h] < 0 ? 0 : sr[mt][h];
                    xs[mt][h] = reinterpret_cast<const uint4*>(src + (size_t)v * K)[uc];
                }
            }
        };
        auto stage = [&](int j) {
            const bool uv = (32 * j + sv) * 8 < K;
#pragma unroll
            for (int mt = 0; mt < kMaxMT; ++mt) {
                if (mt >= mts) break;
                a_lds[mt][sm0 * 32 + (sv ^ sm0)] = (sr[mt][0] >= 0 && uv) ? xs[mt][0] : make_uint4(0, 0, 0, 0);
                a_lds[mt][sm1 * 32 + (sv ^ sm1)] = (sr[mt][1] >= 0 && uv) ? xs[mt][1] : make_uint4(0, 0, 0, 0);
            }
        };
        // Per 32-bit word q of the lane's group: the activation fragments of every tile, then per
        // subtile the two dequantised weight fragments, multiplied into every tile.
        auto compute = [&](int j, const uint4 (&cw)[kSub], const uint32_t (&sw)[kSub]) {
            uint32_t swv[kSub];
#pragma unroll
            for (int s = 0; s < kSub; ++s) swv[s] = sw[s];
            if constexpr (kSbLds) {
                const int c = j & 3, jj = j >> 2;
                int e = 16 * jj + 4 * c + kq - sb_piece(jj, c);       // > 3 only for a group past K
                e = e > 3 ? 3 : e;
#pragma unroll
                for (int s = 0; s < kSub; ++s) swv[s] = sb_lds[jj & 1][wv][s][(16 * c + n) * 4 + e];
            }
            f16x2 s2[kSub], b2[kSub];
#pragma unroll
            for (int s = 0; s < kSub; ++s) {
                const f16x2 sb = __builtin_bit_cast(f16x2, swv[s]);
                const _Float16 two_s = sb.x * (_Float16)2.0f;
                s2[s] = (f16x2){two_s, two_s};
                b2[s] = (f16x2){sb.y, sb.y};
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int v = 8 * kq + 2 * q;
                f16x8 a_ev[kMaxMT], a_od[kMaxMT];
#pragma unroll
                for (int mt = 0; mt < kMaxMT; ++mt) {
                    if (mt >= mts) break;
                    const uint4* arow = a_lds[mt] + n * 32;
                    split_even_odd(arow[v ^ n], arow[(v + 1) ^ n], a_ev[mt], a_od[mt]);
                }
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    const uint32_t w = q == 0 ? cw[s].x : q == 1 ? cw[s].y : q == 2 ? cw[s].z : cw[s].w;
                    const f16x8 b_ev = dequant8(w & 0x33333333u, s2[s], b2[s]);
                    const f16x8 b_od = dequant8((w >> 2) & 0x33333333u, s2[s], b2[s]);
#pragma unroll
                    for (int mt = 0; mt < kMaxMT; ++mt) {
                        if (mt >= mts) break;
                        acc[mt][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_ev[mt], b_ev, acc[mt][s], 0, 0, 0);
                        acc[mt][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_od[mt], b_od, acc[mt][s], 0, 0, 0);
                    }
                }
            }
        };
        // Software pipeline, one chunk deep: chunk j + 1's weights and activations are in flight
        // while chunk j is multiplied (the activation registers are free once chunk j is staged).
        // Loads retire in issue order: staging chunk j + 1 waits for its activations, and with
        // them for chunk j + 1's weights, issued before them and needed next anyway.  The last
        // chunk's look-ahead re-reads the last chunk (an L2 hit), so no load is conditional.
        if constexpr (kSbLds) fetch_sb(0);
        if constexpr (kPrefetch) {
            load_x(0);
            load_w(0, cwa, swa);
#pragma unroll 1
            for (int j = 0; j < NCH; ++j) {
                load_w(j + 1 < NCH ? j + 1 : NCH - 1, cwb, swb);
                lds_barrier();                                 // every wave is done with chunk j - 1
                stage(j);
                stage_sb(j);
                lds_barrier();
                load_x(j + 1 < NCH ? j + 1 : NCH - 1);
                compute(j, cwa, swa);
                next_sb_block(j);
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    cwa[s] = cwb[s];
                    swa[s] = swb[s];
                }
            }
        } else {
#pragma unroll 1
            for (int j = 0; j < NCH; ++j) {
                load_x(j);
                load_w(j, cwa, swa);
                lds_barrier();                                 // every wave is done with chunk j - 1
                stage(j);
                stage_sb(j);
                lds_barrier();
                compute(j, cwa, swa);
                next_sb_block(j);
            }
        }

        // Epilogue: lane holds rows 4*kq + i (i = 0..3) of column n of each subtile of each tile.
#pragma unroll
        for (int mt = 0; mt < kMaxMT; ++mt) {
            if (mt >= mts) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mt * kMT + 4 * kq + i;
                if (m >= rows) continue;
                const int r = b0 + m;
                if (MODE == kGateUp) {
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        if (!rv[2 * p]) continue;
                        const float g = acc[mt][2 * p][i], u = acc[mt][2 * p + 1][i];
                        out[(size_t)r * N + col[2 * p]] = __float2half_rn(g / (1.0f + __expf(-g)) * u);
                    }
                } else {
                    const int orow = row_out ? row_out[r] : r;
                    if (orow < 0 || orow >= n_out_rows) continue;
#pragma unroll
                    for (int s = 0; s < kSub; ++s)
                        if (rv[s]) out[(size_t)orow * N + col[s]] = __float2half_rn(acc[mt][s][i]);
                }
            }
        }
        __syncthreads();                                       // a_lds is reused by the next batch
    }
}


// Down in the whole-K form (K = inter = 256 * GPL): a block takes one segment and 256 output rows,
// each wave 4 subtiles of 16 rows whose whole K it requests at once and keeps in registers while
// the segment's 16-row tiles of h pass through LDS (staged for the whole K, split into the MFMA's
// even / odd fragments; one barrier per tile).  Output row r goes to row_out[r] (or r).
template <int GPL, int SBF>
__global__ __launch_bounds__(256, 2) void k_q2g_dn_wk(
    const __half* __restrict__ src, int n_src_rows, const int32_t* __restrict__ row_out, int n_out_rows,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_slot, int n_seg, int n_rows,
    Q2Experts E, int n_slots, int hidden, int tiles_per_seg, __half* __restrict__ out) {
    constexpr int K = 256 * GPL;
    constexpr int kg = 4 * GPL;
    constexpr int UPR = K / 8;                        // 16-byte units per h row
    constexpr int kPairsPerThread = UPR / 32;         // unit pairs a thread stages per tile
    static_assert(kPairsPerThread >= 1, "K >= 256");
    __shared__ uint4 a_lds[16 * UPR];
    const int items = n_seg * tiles_per_seg;
    const int pass = (int)blockIdx.x >= items ? 1 : 0;
    const int work = xcd_order((int)blockIdx.x - pass * items, items);
    const int seg = work / tiles_per_seg, tile = work % tiles_per_seg;
    if (seg >= n_seg) return;
    int r0 = seg_start[seg], r1 = seg_start[seg + 1];
    r0 = r0 < 0 ? 0 : (r0 > n_rows ? n_rows : r0);
    r1 = r1 < r0 ? r0 : (r1 > n_rows ? n_rows : r1);
    const int slot = seg_slot ? seg_slot[seg] : seg;
    if (r1 == r0 || slot < 0 || slot >= n_slots) return;
    if ((pass == 0) != (r1 - r0 > kMT)) return;       // segments of several tiles first

    const int t0 = threadIdx.x, lane0 = t0 & 63, wv = __builtin_amdgcn_readfirstlane(t0 >> 6);
    const int n0 = lane0 & 15, kq0 = lane0 >> 4;
    const Q2Proj& P = E.p[2];
    const size_t code_row = (size_t)K / 4;
    // the wave's 4 subtiles: output rows base_s .. base_s + 15 (hidden is a multiple of 64)
    uint4 cw[4][GPL];
    uint32_t sw[4][GPL];
    bool rv[4];
    int col[4];
#pragma unroll
    for (int sIdx = 0; sIdx < 4; ++sIdx) {
        int base = tile * 256 + wv * 64 + sIdx * 16;
        rv[sIdx] = base < hidden;
        col[sIdx] = base + n0;
        if (base >= hidden) base = hidden - 16;
        const uint8_t* cr = P.w + (size_t)slot * P.w_stride + (size_t)(base + n0) * code_row + (size_t)(GPL * kq0) * 16;
#pragma unroll
        for (int i = 0; i < GPL; ++i) cw[sIdx][i] = *reinterpret_cast<const uint4*>(cr + (size_t)i * 16);
        if constexpr (SBF == 0) {
            const uint32_t* sr = reinterpret_cast<const uint32_t*>(P.s + (size_t)slot * P.s_stride) +
                                 (size_t)(base + n0) * kg + GPL * kq0;
#pragma unroll
            for (int i = 0; i < GPL; ++i) sw[sIdx][i] = sr[i];
        } else {
            const uint16_t* scr = reinterpret_cast<const uint16_t*>(P.s + (size_t)slot * P.s_stride) +
                                  (size_t)(base + n0) * kg + GPL * kq0;
            const uint16_t* bir = reinterpret_cast<const uint16_t*>(P.b + (size_t)slot * P.b_stride) +
                                  (size_t)(base + n0) * kg + GPL * kq0;
#pragma unroll
            for (int i = 0; i < GPL; ++i) sw[sIdx][i] = sb_word<SBF>(scr[i], bir[i]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    const int sm = t0 >> 4, sv0 = t0 & 15;
#pragma unroll 1
    for (int m0 = r0; m0 < r1; m0 += kMT) {          // block-uniform
        const int rows_t = (r1 - m0) < kMT ? (r1 - m0) : kMT;
        int srow = -1;
        if (sm < rows_t) {
            srow = m0 + sm;
            if (srow >= n_src_rows) srow = -1;
        }
        uint4 xv[2 * kPairsPerThread];
        const uint4* xr = reinterpret_cast<const uint4*>(src + (size_t)(srow < 0 ? 0 : srow) * K);
#pragma unroll
        for (int c = 0; c < kPairsPerThread; ++c) {
            xv[2 * c] = xr[2 * (sv0 + 16 * c)];
            xv[2 * c + 1] = xr[2 * (sv0 + 16 * c) + 1];
        }
        if (m0 > r0) lds_barrier();                   // every wave is done with the last tile
#pragma unroll
        for (int c = 0; c < kPairsPerThread; ++c) {
            const int v = 2 * (sv0 + 16 * c);
            f16x8 ev, od;
            split_even_odd(xv[2 * c], xv[2 * c + 1], ev, od);
            const uint4 e4 = __builtin_bit_cast(uint4, ev), o4 = __builtin_bit_cast(uint4, od);
            a_lds[sm * UPR + (v ^ sm)] = srow >= 0 ? e4 : make_uint4(0, 0, 0, 0);
            a_lds[sm * UPR + ((v + 1) ^ sm)] = srow >= 0 ? o4 : make_uint4(0, 0, 0, 0);
        }
        lds_barrier();
        // opaque per tile: the converted weights and the fragment addresses are not kept across
        // tiles
        uint32_t z;
        asm volatile("v_mov_b32 %0, 0" : "=v"(z));
        int tq = (int)threadIdx.x;
        asm volatile("" : "+v"(tq));
        const int n = tq & 15, kq = (tq & 63) >> 4;
        f32x4 acc[4];
#pragma unroll
        for (int sIdx = 0; sIdx < 4; ++sIdx) acc[sIdx] = (f32x4){0.f, 0.f, 0.f, 0.f};
        const uint4* arow = a_lds + n * UPR;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            f16x2 s2[4], b2[4];
#pragma unroll
            for (int sIdx = 0; sIdx < 4; ++sIdx) {
                const f16x2 sb = __builtin_bit_cast(f16x2, sw[sIdx][i] ^ z);
                const _Float16 two_s = sb.x * (_Float16)2.0f;
                s2[sIdx] = (f16x2){two_s, two_s};
                b2[sIdx] = (f16x2){sb.y, sb.y};
            }
            const int u0 = 8 * (GPL * kq + i);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int v = u0 + 2 * q;
                const f16x8 a_ev = __builtin_bit_cast(f16x8, arow[v ^ n]);
                const f16x8 a_od = __builtin_bit_cast(f16x8, arow[(v + 1) ^ n]);
#pragma unroll
                for (int sIdx = 0; sIdx < 4; ++sIdx) {
                    const uint4 cv = cw[sIdx][i];
                    const uint32_t wq = (q == 0 ? cv.x : q == 1 ? cv.y : q == 2 ? cv.z : cv.w) ^ z;
                    const f16x8 b_ev = dequant8(wq & 0x33333333u, s2[sIdx], b2[sIdx]);
                    const f16x8 b_od = dequant8((wq >> 2) & 0x33333333u, s2[sIdx], b2[sIdx]);
                    acc[sIdx] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_ev, b_ev, acc[sIdx], 0, 0, 0);
                    acc[sIdx] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_od, b_od, acc[sIdx], 0, 0, 0);
                }
            }
        }
        // lane holds rows 4 kq + i of column n of each subtile
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * kq + i;
            if (m >= rows_t) continue;
            const int r = m0 + m;
            const int orow = row_out ? row_out[r] : r;
            if (orow < 0 || orow >= n_out_rows) continue;
#pragma unroll
            for (int sIdx = 0; sIdx < 4; ++sIdx)
                if (rv[sIdx]) out[(size_t)orow * hidden + col[sIdx]] = __float2half_rn(acc[sIdx][i]);
        }
    }
}

template <int NCH, int MODE, bool SBL, int SBF>
int launch_proj(const __half* src, int n_src_rows, const int32_t* row_map, const int32_t* row_out, int n_out_rows,
                const int32_t* seg_start, const int32_t* seg_slot, int n_seg, int n_rows, const Q2Experts& E,
                int n_slots, int hidden, int inter, __half* out, hipStream_t s) {
    const int N = MODE == kGateUp ? inter : hidden;
    const int rows_per_block = MODE == kGateUp ? 128 : 256;
    const int tiles = (N + rows_per_block - 1) / rows_per_block;
    // K = 512 exactly (whole 256-wide chunks): down in the whole-K form
    const bool dn_wk = MODE == kDown && NCH == 2 && !SBL && inter == 256 * NCH;
    const long long nb = (MODE == kGateUp || dn_wk ? 2LL : 1LL) * n_seg * tiles;   // two passes
    if (nb <= 0) return 0;
    if (nb > 0x7FFFFFFFLL) { moe_set_error("grouped q2: grid too large"); return -1; }
    if (dn_wk) {
        if constexpr (MODE == kDown && NCH == 2 && !SBL)
            MOE_LAUNCH(TK_PF_DOWN, (k_q2g_dn_wk<NCH, SBF>), dim3((unsigned)nb), dim3(256), 0, s, src, n_src_rows, row_out,
                       n_out_rows, seg_start, seg_slot, n_seg, n_rows, E, n_slots, hidden, tiles, out);
    } else if constexpr (MODE == kGateUp && SBL && NCH == 8) {
        // K = 2048: the whole-K form (128 rows per block, as here)
        MOE_LAUNCH(TK_PF_GATE_UP, (k_q2g_gu_wk<NCH, SBF>), dim3((unsigned)nb), dim3(256), 0, s, src, n_src_rows, row_map,
                   seg_start, seg_slot, n_seg, n_rows, E, n_slots, inter, tiles, out);
    } else {
        MOE_LAUNCH(MODE == kGateUp ? TK_PF_GATE_UP : TK_PF_DOWN, (k_q2g_proj<NCH, MODE, SBL, SBF>), dim3((unsigned)nb),
                   dim3(256), 0, s, src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg, n_rows,
                   E, n_slots, hidden, inter, tiles, out);
    }
    HIP_TRY(hipGetLastError());
    return 0;
}

template <int MODE, int SBF>
int dispatch_proj_f(int K, const __half* src, int n_src_rows, const int32_t* row_map, const int32_t* row_out,
                    int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg, int n_rows,
                    const Q2Experts& E, int n_slots, int hidden, int inter, __half* out, hipStream_t s) {
    // the four-chunk scale/bias blocks pay on gate/up's long K; down (K = inter, often 2 chunks)
    // is faster with the per-chunk loads
    const bool sbl = MODE == kGateUp && K % 256 == 0 && K >= 512;
    switch ((K + 255) / 256) {
#define PF_CASE(c) \
    case c: \
        if (sbl) \
            return launch_proj<c, MODE, (c >= 2 && MODE == kGateUp), SBF>(src, n_src_rows, row_map, row_out, n_out_rows, \
                                                                          seg_start, seg_slot, n_seg, n_rows, E, n_slots, \
                                                                          hidden, inter, out, s); \
        return launch_proj<c, MODE, false, SBF>(src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, \
                                                n_seg, n_rows, E, n_slots, hidden, inter, out, s);
        PF_CASE(1) PF_CASE(2) PF_CASE(3) PF_CASE(4) PF_CASE(5)
        PF_CASE(6) PF_CASE(7) PF_CASE(8) PF_CASE(9) PF_CASE(10)
#undef PF_CASE
        default: moe_set_error("grouped q2: contraction length %d unsupported (<= %d)", K, kMaxChunks * 256); return -1;
    }
}

template <int MODE>
int dispatch_proj(int K, const __half* src, int n_src_rows, const int32_t* row_map, const int32_t* row_out,
                  int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg, int n_rows,
                  const Q2Experts& E, int n_slots, int hidden, int inter, __half* out, hipStream_t s) {
    if (E.p[0].sb_step == 4)
        return dispatch_proj_f<MODE, 0>(K, src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg,
                                        n_rows, E, n_slots, hidden, inter, out, s);
    if (E.bf16)
        return dispatch_proj_f<MODE, 2>(K, src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg,
                                        n_rows, E, n_slots, hidden, inter, out, s);
    return dispatch_proj_f<MODE, 1>(K, src, n_src_rows, row_map, row_out, n_out_rows, seg_start, seg_slot, n_seg,
                                    n_rows, E, n_slots, hidden, inter, out, s);
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

// The same sum for hidden a multiple of 8: each thread 8 consecutive columns, 16-byte loads of
// the fp16 rows and two 16-byte stores (the same operations per element in the same order, so
// bit-identical to k_pair_combine).
__global__ __launch_bounds__(256) void k_pair_combine8(const __half* __restrict__ y, const __half* __restrict__ scores,
                                                       const __half* __restrict__ residual, int k, int hidden,
                                                       float* __restrict__ out) {
    const int t = blockIdx.y;
    const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (c >= hidden) return;
    // every row's load first (k <= MOE_MAX_K), then the sums in row order
    uint4 rv[MOE_MAX_K];
#pragma unroll
    for (int j = 0; j < MOE_MAX_K; ++j)
        if (j < k) rv[j] = *reinterpret_cast<const uint4*>(y + ((size_t)t * k + j) * hidden + c);
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MOE_MAX_K; ++j) {
        if (j < k) {
            const float sj = __half2float(scores[(size_t)t * k + j]);
            const uint4 v = rv[j];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[2 * i] += sj * __half2float(__ushort_as_half((unsigned short)(w[i] & 0xFFFFu)));
                a[2 * i + 1] += sj * __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
            }
        }
    }
    if (residual) {
        const uint4 v = *reinterpret_cast<const uint4*>(residual + (size_t)t * hidden + c);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[2 * i] += __half2float(__ushort_as_half((unsigned short)(w[i] & 0xFFFFu)));
            a[2 * i + 1] += __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
        }
    }
    float4* o = reinterpret_cast<float4*>(out + (size_t)t * hidden + c);
    o[0] = make_float4(a[0], a[1], a[2], a[3]);
    o[1] = make_float4(a[4], a[5], a[6], a[7]);
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
    if (n_tokens <= 0) {                      // the kernel reads source row 0 unconditionally
        moe_set_error("q2_grouped_gate_up: %d rows but no tokens", n_rows);
        return -1;
    }
    const Q2Experts E = q2_experts_from_blob(pool, stride, blob_layout(hidden, inter, group));
    return dispatch_proj<kGateUp>(hidden, x, n_tokens, row_token, nullptr, 0, seg_start, seg_slot, n_seg, n_rows, E,
                                  n_slots, hidden, inter, h_out, s);
}

int launch_q2_grouped_down(const __half* h, int n_rows, const int32_t* row_out, int n_out_rows,
                           const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const uint8_t* pool,
                           size_t stride, int n_slots, int hidden, int inter, int group, __half* y_out, hipStream_t s) {
    if (!check_grouped("q2_grouped_down", hidden, inter, group, n_seg, n_rows, pool, stride, n_slots, h, seg_start,
                       y_out))
        return -1;
    if (n_seg == 0 || n_rows == 0) return 0;
    const Q2Experts E = q2_experts_from_blob(pool, stride, blob_layout(hidden, inter, group));
    return dispatch_proj<kDown>(inter, h, n_rows, nullptr, row_out, row_out ? n_out_rows : n_rows, seg_start, seg_slot,
                                n_seg, n_rows, E, n_slots, hidden, inter, y_out, s);
}

// The same over the reference's 9 tensors (E from their pools; see q2t_shape_ok for the shapes the
// decode kernels take -- the grouped kernels take any multiple of 64 up to 2560).
int launch_q2t_grouped_gate_up(const __half* x, int n_tokens, const int32_t* row_token, int n_rows,
                               const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const Q2Experts& E,
                               int n_slots, int hidden, int inter, int group, __half* h_out, hipStream_t s) {
    if (!check_grouped("q2t_grouped_gate_up", hidden, inter, group, n_seg, n_rows, E.p[0].w, ~size_t(0), n_slots, x,
                       seg_start, h_out))
        return -1;
    if (n_seg == 0 || n_rows == 0) return 0;
    if (n_tokens <= 0) {
        moe_set_error("q2t_grouped_gate_up: %d rows but no tokens", n_rows);
        return -1;
    }
    return dispatch_proj<kGateUp>(hidden, x, n_tokens, row_token, nullptr, 0, seg_start, seg_slot, n_seg, n_rows, E,
                                  n_slots, hidden, inter, h_out, s);
}

int launch_q2t_grouped_down(const __half* h, int n_rows, const int32_t* row_out, int n_out_rows,
                            const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const Q2Experts& E,
                            int n_slots, int hidden, int inter, int group, __half* y_out, hipStream_t s) {
    if (!check_grouped("q2t_grouped_down", hidden, inter, group, n_seg, n_rows, E.p[2].w, ~size_t(0), n_slots, h,
                       seg_start, y_out))
        return -1;
    if (n_seg == 0 || n_rows == 0) return 0;
    return dispatch_proj<kDown>(inter, h, n_rows, nullptr, row_out, row_out ? n_out_rows : n_rows, seg_start, seg_slot,
                                n_seg, n_rows, E, n_slots, hidden, inter, y_out, s);
}

int launch_pair_combine(const __half* y, const __half* scores, const __half* residual, int n_tokens, int k,
                        int hidden, float* out, hipStream_t s) {
    if (n_tokens < 0 || k <= 0 || hidden <= 0 || n_tokens > 65535) {
        moe_set_error("pair_combine: n_tokens=%d (<= 65535) k=%d hidden=%d", n_tokens, k, hidden);
        return -1;
    }
    if (n_tokens == 0) return 0;
    if (!y || !scores || !out) { moe_set_error("pair_combine: null pointer"); return -1; }
    const bool aligned = ((uintptr_t)y | (uintptr_t)out | (uintptr_t)residual) % 16 == 0;
    if (hidden % 8 == 0 && aligned && k <= MOE_MAX_K) {
        dim3 grid((hidden / 8 + 255) / 256, n_tokens);
        MOE_LAUNCH(TK_COMBINE, k_pair_combine8, grid, dim3(256), 0, s, y, scores, residual, k, hidden, out);
    } else {
        dim3 grid(((hidden + 1) / 2 + 255) / 256, n_tokens);
        MOE_LAUNCH(TK_COMBINE, k_pair_combine, grid, dim3(256), 0, s, y, scores, residual, k, hidden, out);
    }
    HIP_TRY(hipGetLastError());
    return 0;
}
