// Device-side slot table and miss staging for gfx950.
//
// k_slot_step / k_slot_prefetch run one table operation in one wave (slot_table_dev.h), so the
// host never has to read the router's ids: the step and prefetch run on the stream right after
// the router (or inside it, see router.hip), and their copy lists drive k_stage, which pulls the
// missing expert blobs from the pinned (host-mapped) expert store into the HBM slot pool.
#include "moe_common.h"
#include "slot_table_dev.h"

namespace {

// The ids / predictions are loaded with the table, in the same round trip.
__global__ __launch_bounds__(64) void k_slot_step(SlotTable* __restrict__ t, const uint32_t* __restrict__ ids,
                                                  int k, uint32_t* __restrict__ slot_inds) {
    __shared__ slot_dev::LdsTable L;
    const int lane = threadIdx.x;
    const slot_dev::TabRegs r = slot_dev::fetch_table(t, lane);
    const uint32_t id = ids[lane < k ? lane : 0];
    slot_dev::dev_slot_step(t, L, r, id, k, slot_inds, lane);
}

__global__ __launch_bounds__(64) void k_slot_prefetch(SlotTable* __restrict__ t, const int32_t* __restrict__ preds,
                                                      int m, int max_fetch) {
    __shared__ slot_dev::LdsTable L;
    __shared__ int32_t p[MOE_MAX_PREFETCH];
    const int lane = threadIdx.x;
    const slot_dev::TabRegs r = slot_dev::fetch_table(t, lane);
    const int32_t v = m > 0 ? preds[lane < m ? lane : 0] : 0;     // m = 0 may come with no list
    if (lane < m) p[lane] = v;
    slot_dev::wave_sync();
    slot_dev::dev_slot_prefetch(t, L, r, p, m, max_fetch, lane);
}

// Copy the blobs listed in the table's copy list: store[eid] -> pool[slot].  blockIdx.y picks
// the copy, blockIdx.x strides over its 16-byte units, four in flight per thread; the store is
// pinned host memory read over PCIe (a kernel copy sustains the link rate with blob-sized
// pieces, where one DMA request per blob does not).
__global__ __launch_bounds__(256) void k_stage(const SlotTable* __restrict__ t, int list,
                                               const uint8_t* __restrict__ store, size_t store_stride,
                                               uint8_t* __restrict__ pool, size_t pool_stride, size_t bytes) {
    const int c = blockIdx.y;
    const int n = list ? t->pf_n_copy : t->n_copy;
    if (c >= min(n, MOE_MAX_PREFETCH)) return;
    const int eid = list ? t->pf_copy_eid[c] : t->copy_eid[c];
    const int slot = list ? t->pf_copy_slot[c] : t->copy_slot[c];
    if (eid < 0 || eid >= MOE_NUM_EXPERTS || slot < 0 || slot >= t->capacity) return;
    const uint4* src = reinterpret_cast<const uint4*>(store + (size_t)eid * store_stride);
    uint4* dst = reinterpret_cast<uint4*>(pool + (size_t)slot * pool_stride);
    const unsigned units = (unsigned)(bytes / 16);
    const unsigned step = gridDim.x * blockDim.x;
    // Four independent 16-byte loads in flight per thread, held in named registers (an array
    // here gets moved to LDS by the compiler, which serialises the loads behind LDS writes).
    for (unsigned u = blockIdx.x * blockDim.x + threadIdx.x; u < units; u += 4 * step) {
        const bool m1 = u + step < units, m2 = u + 2 * step < units, m3 = u + 3 * step < units;
        uint4 a = src[u], b = {}, c = {}, d = {};
        if (m1) b = src[u + step];
        if (m2) c = src[u + 2 * step];
        if (m3) d = src[u + 3 * step];
        dst[u] = a;
        if (m1) dst[u + step] = b;
        if (m2) dst[u + 2 * step] = c;
        if (m3) dst[u + 3 * step] = d;
    }
}

// k_stage for a layer whose experts are several tensors (the reference's 9 per layer): one launch
// per list, each listed expert's tensors copied as one run of 16-byte units (unit u of the
// concatenation lies in the tensor whose first unit is the last one <= u), so an expert gets the
// same `ctas` blocks and the link the same requests as a one-blob expert, instead of one launch per
// tensor.
__device__ __forceinline__ void stage_unit(const StageSet& S, unsigned u, int eid, int slot, const uint4*& src,
                                           uint4*& dst) {
    int i = 0;
#pragma unroll
    for (int j = 1; j < MOE_NUM_TENSORS; ++j)
        if (j < S.n && S.first[j] <= u) i = j;
    const unsigned v = u - S.first[i];
    src = reinterpret_cast<const uint4*>(S.src[i] + (size_t)eid * S.src_stride[i]) + v;
    dst = reinterpret_cast<uint4*>(S.dst[i] + (size_t)slot * S.dst_stride[i]) + v;
}

__global__ __launch_bounds__(256) void k_stage_set(const SlotTable* __restrict__ t, int list, StageSet S) {
    const int c = blockIdx.y;
    const int n = list ? t->pf_n_copy : t->n_copy;
    if (c >= min(n, MOE_MAX_PREFETCH)) return;
    const int eid = list ? t->pf_copy_eid[c] : t->copy_eid[c];
    const int slot = list ? t->pf_copy_slot[c] : t->copy_slot[c];
    if (eid < 0 || eid >= MOE_NUM_EXPERTS || slot < 0 || slot >= t->capacity) return;
    const unsigned units = S.total;
    const unsigned step = gridDim.x * blockDim.x;
    for (unsigned u = blockIdx.x * blockDim.x + threadIdx.x; u < units; u += 4 * step) {
        const bool m1 = u + step < units, m2 = u + 2 * step < units, m3 = u + 3 * step < units;
        const uint4 *s0, *s1 = nullptr, *s2 = nullptr, *s3 = nullptr;
        uint4 *d0, *d1 = nullptr, *d2 = nullptr, *d3 = nullptr;
        stage_unit(S, u, eid, slot, s0, d0);
        if (m1) stage_unit(S, u + step, eid, slot, s1, d1);
        if (m2) stage_unit(S, u + 2 * step, eid, slot, s2, d2);
        if (m3) stage_unit(S, u + 3 * step, eid, slot, s3, d3);
        uint4 a = *s0, b = {}, cc = {}, d = {};
        if (m1) b = *s1;
        if (m2) cc = *s2;
        if (m3) d = *s3;
        *d0 = a;
        if (m1) *d1 = b;
        if (m2) *d2 = cc;
        if (m3) *d3 = d;
    }
}

// Host-listed copies (a synchronous load of a prefill chunk's experts): copy c of the launch
// moves expert P.eid[c] to slot P.slot[c] over every tensor of S, blockIdx.x striding over the
// expert's 16-byte units as in k_stage_set.
constexpr int kStagePairsMax = 128;
struct StagePairs {
    int32_t eid[kStagePairsMax];
    int32_t slot[kStagePairsMax];
    int n;
};

__global__ __launch_bounds__(256) void k_stage_pairs(StagePairs P, StageSet S) {
    const int c = blockIdx.y;
    if (c >= P.n) return;
    const int eid = P.eid[c], slot = P.slot[c];
    const unsigned units = S.total;
    const unsigned step = gridDim.x * blockDim.x;
    for (unsigned u = blockIdx.x * blockDim.x + threadIdx.x; u < units; u += 4 * step) {
        const bool m1 = u + step < units, m2 = u + 2 * step < units, m3 = u + 3 * step < units;
        const uint4 *s0, *s1 = nullptr, *s2 = nullptr, *s3 = nullptr;
        uint4 *d0, *d1 = nullptr, *d2 = nullptr, *d3 = nullptr;
        stage_unit(S, u, eid, slot, s0, d0);
        if (m1) stage_unit(S, u + step, eid, slot, s1, d1);
        if (m2) stage_unit(S, u + 2 * step, eid, slot, s2, d2);
        if (m3) stage_unit(S, u + 3 * step, eid, slot, s3, d3);
        uint4 a = *s0, b = {}, cc = {}, d = {};
        if (m1) b = *s1;
        if (m2) cc = *s2;
        if (m3) d = *s3;
        *d0 = a;
        if (m1) *d1 = b;
        if (m2) *d2 = cc;
        if (m3) *d3 = d;
    }
}

// Plain device copy of a known byte count: the reference reading for scaling memory counters
// (FETCH_SIZE / WRITE_SIZE per dispatch) to bytes.
__global__ __launch_bounds__(256) void k_copy_calib(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Streams `n16` 16-byte units and reduces them: the fastest a single launch reading that many
// bytes from HBM can be (no dependent loads, no outputs), for comparing kernels of the same size.
__global__ __launch_bounds__(256) void k_stream_calib(const uint4* __restrict__ src, size_t n16, float* __restrict__ out) {
    float acc = 0.f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = src[i];
        acc += __uint_as_float(v.x & 0x3f800000u) + __uint_as_float(v.w & 0x3f800000u);
    }
    if (acc == -1.0f) out[0] = acc;                  // never true for the inputs used; keeps the loads
}

struct U32x16 { uint32_t v[16]; };

__global__ void k_store_u32(uint32_t* dst, U32x16 vals, int n) {
    int i = threadIdx.x;
    if (i < n) dst[i] = vals.v[i];
}

// One thread per id of the step (router order i): its slot and score go to the hit half
// [0, MOE_MAX_K) or the miss half [MOE_MAX_K, 2 MOE_MAX_K) at its rank there.
__global__ void k_split_lists(SplitLists a, const __half* __restrict__ scores, uint32_t* __restrict__ slots_out,
                              __half* __restrict__ scores_out) {
    const int i = threadIdx.x;
    if (i >= a.k) return;
    const int d = a.inv[i];
    const bool hit = d < a.n_hit;
    const int dst = hit ? d : MOE_MAX_K + (d - a.n_hit);
    slots_out[dst] = hit ? a.hit[d] : a.miss[d - a.n_hit];
    scores_out[dst] = scores[i];
}

// Accounting control of the device-driven tables, one thread per table: 0 off (no token open),
// 1 on, 2 open the next token (its counters start at zero), 3 restart the token numbering.  The
// host keeps the same state for its own tables (capi.hip), so both number tokens alike.
__global__ void k_acct_ctl(TableSet ts, int mode) {
    const int i = threadIdx.x;
    if (i >= ts.n) return;
    SlotTable* t = ts.t[i];
    if (mode == 0) { t->acct_on = 0; t->acct_token = -1; }
    else if (mode == 1) t->acct_on = 1;
    else if (mode == 2) {
        t->acct_token = t->acct_seq++;
        for (int c = 0; c < 10; ++c) t->acct[c] = 0;
    } else { t->acct_seq = 0; t->acct_token = -1; }
}

// The open token's counters summed over the tables (lane c: counter c).
__global__ void k_acct_sum(TableSet ts, uint64_t* __restrict__ out10) {
    const int c = threadIdx.x;
    if (c >= 10) return;
    uint64_t v = 0;
    for (int i = 0; i < ts.n; ++i) v += ts.t[i]->acct[c];
    out10[c] = v;
}

}  // namespace

int launch_acct_ctl(const TableSet& ts, int mode, hipStream_t s) {
    if (ts.n <= 0 || ts.n > MOE_MAX_LAYERS || mode < 0 || mode > 3) {
        moe_set_error("acct_ctl: %d tables, mode %d", ts.n, mode);
        return -1;
    }
    hipLaunchKernelGGL(k_acct_ctl, dim3(1), dim3(64), 0, s, ts, mode);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_acct_sum(const TableSet& ts, uint64_t* out10, hipStream_t s) {
    if (ts.n <= 0 || ts.n > MOE_MAX_LAYERS || !out10) { moe_set_error("acct_sum: %d tables", ts.n); return -1; }
    hipLaunchKernelGGL(k_acct_sum, dim3(1), dim3(64), 0, s, ts, out10);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_slot_step(SlotTable* t, const uint32_t* ids, int k, uint32_t* slot_inds, hipStream_t s) {
    if (k <= 0 || k > MOE_MAX_K) { moe_set_error("slot_step: k=%d out of range", k); return -1; }
    MOE_LAUNCH(TK_SLOT, k_slot_step, dim3(1), dim3(64), 0, s, t, ids, k, slot_inds);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_slot_prefetch(SlotTable* t, const int32_t* preds, int m, int max_fetch, hipStream_t s) {
    if (m < 0 || m > MOE_MAX_PREFETCH) { moe_set_error("slot_prefetch: m=%d out of range", m); return -1; }
    MOE_LAUNCH(TK_SLOT, k_slot_prefetch, dim3(1), dim3(64), 0, s, t, preds, m, max_fetch);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_stage(const SlotTable* t, int list, const uint8_t* store, size_t store_stride, uint8_t* pool,
                 size_t pool_stride, size_t bytes, int ctas, hipStream_t s) {
    if (bytes % 16 || store_stride % 16 || pool_stride % 16 || bytes > pool_stride || bytes > store_stride) {
        moe_set_error("stage: bytes=%zu strides=%zu/%zu must be multiples of 16 with bytes <= stride",
                      bytes, store_stride, pool_stride);
        return -1;
    }
    if (bytes / 16 > 0xFFFFFFFFull) { moe_set_error("stage: blob of %zu bytes too large", bytes); return -1; }
    // ctas = blocks per copy; the grid covers the largest possible copy list, empty rows exit.
    // 2 blocks x 256 threads x 4 x 16 B in flight per copy already saturate PCIe; more only
    // crowds other kernels' memory requests.
    if (ctas <= 0) ctas = 2;
    MOE_LAUNCH(TK_STAGE, k_stage, dim3(ctas, MOE_MAX_PREFETCH), dim3(256), 0, s, t, list, store, store_stride,
               pool, pool_stride, bytes);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_stage_pairs(const int32_t* eids, const int32_t* slots, int n, const StageSet& S, hipStream_t s) {
    if (S.n <= 0 || S.n > MOE_NUM_TENSORS) { moe_set_error("stage_pairs: %d tensors", S.n); return -1; }
    for (int i0 = 0; i0 < n; i0 += kStagePairsMax) {
        StagePairs P;
        P.n = n - i0 < kStagePairsMax ? n - i0 : kStagePairsMax;
        for (int i = 0; i < P.n; ++i) {
            P.eid[i] = eids[i0 + i];
            P.slot[i] = slots[i0 + i];
        }
        // ~128 blocks over the launch's copies, 16 KB in flight each (a prefill chunk's ~100
        // copies: 9.6 ms per chunk through a 102-slot layer against 9.8 with ~32 or ~512 blocks)
        const int ctas = P.n >= 128 ? 1 : (128 + P.n - 1) / P.n;
        MOE_LAUNCH(TK_STAGE, k_stage_pairs, dim3(ctas, P.n), dim3(256), 0, s, P, S);
        HIP_TRY(hipGetLastError());
    }
    return 0;
}

int launch_stage_set(const SlotTable* t, int list, const StageSet& S, int ctas, hipStream_t s) {
    if (S.n <= 0 || S.n > MOE_NUM_TENSORS) { moe_set_error("stage_set: %d tensors", S.n); return -1; }
    if (ctas <= 0) ctas = 2;
    MOE_LAUNCH(TK_STAGE, k_stage_set, dim3(ctas, MOE_MAX_PREFETCH), dim3(256), 0, s, t, list, S);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_copy_calib(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (!dst || !src || bytes == 0 || bytes % 16) { moe_set_error("copy_calib: bytes must be a positive multiple of 16"); return -1; }
    hipLaunchKernelGGL(k_copy_calib, dim3(1024), dim3(256), 0, s, (const uint4*)src, (uint4*)dst, bytes / 16);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_stream_calib(const void* src, size_t bytes, int grid, float* out, hipStream_t s) {
    if (!src || !out || bytes == 0 || bytes % 16 || grid <= 0) {
        moe_set_error("stream_calib: bytes must be a positive multiple of 16, grid > 0");
        return -1;
    }
    MOE_LAUNCH(TK_STREAM_CALIB, k_stream_calib, dim3(grid), dim3(256), 0, s, (const uint4*)src, bytes / 16, out);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_store_u32(uint32_t* dst, const uint32_t* vals, int n, hipStream_t s) {
    if (n <= 0 || n > 16) { moe_set_error("store_u32: n=%d out of range", n); return -1; }
    U32x16 v = {};
    for (int i = 0; i < n; ++i) v.v[i] = vals[i];
    hipLaunchKernelGGL(k_store_u32, dim3(1), dim3(64), 0, s, dst, v, n);
    HIP_TRY(hipGetLastError());
    return 0;
}

int launch_split_lists(const SplitLists& a, const __half* scores, uint32_t* slots_out, __half* scores_out,
                       hipStream_t s) {
    if (a.k <= 0 || a.k > MOE_MAX_K || a.n_hit < 0 || a.n_miss < 0 || a.n_hit + a.n_miss != a.k) {
        moe_set_error("split_lists: inconsistent split (k=%d hits=%d misses=%d)", a.k, a.n_hit, a.n_miss);
        return -1;
    }
    for (int i = 0; i < a.k; ++i)
        if (a.inv[i] < 0 || a.inv[i] >= a.k) { moe_set_error("split_lists: order entry %d out of range", a.inv[i]); return -1; }
    if (!scores || !slots_out || !scores_out) { moe_set_error("split_lists: null pointer"); return -1; }
    hipLaunchKernelGGL(k_split_lists, dim3(1), dim3(64), 0, s, a, scores, slots_out, scores_out);
    HIP_TRY(hipGetLastError());
    return 0;
}
