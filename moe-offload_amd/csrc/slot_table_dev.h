// Device-side slot-table operations (one wave each), shared by the standalone table kernels
// and the router's last block.
//
// The decisions are those of mlx-qwen38/expert_io.c: decode step 583-685, prefetch 527-581,
// victim choice 404-426 (free stack first, else the oldest resident slot whose expert is not
// protected, else the oldest resident slot).  The table is held in recency-stamp form
// (SlotTable): the oldest resident slot is the one with the smallest stamp, and refreshing a
// slot gives it the next clock value.  Each operation takes the table as fetch_table read it
// (one round trip for all of it), decides on a copy in LDS (~4.5 KB), and writes it back.
//
// With bit 0 of t->sched set, the scheduler variant of mlx-qwen38/cpp/third_party/expert_io.c:
// 1094-1394 applies: the step's victim choice also protects the experts the last prefetch
// fetched (1141-1146), the prefetch skips repeated predictions (1311-1322) and does nothing at
// all when max_fetch <= 0 (1288-1290).  With bit 1 set, a step with 0 < misses < k records its
// hit/miss split lists in t->split (1062-1092).
//
// With t->acct_on set, the operations count the open token's accounting (expert_io.c:98-111,
// the same counters as the host table's Acct): hits, misses, prefetch loads / hits / waste,
// reloads within 16 and 64 tokens of the expert's eviction, and the bytes staged, into t->acct.
//
// All synchronisation is wave-level: a wave's LDS accesses complete in program order, so a
// compiler fence at wavefront scope is all that separates one step from the next.  That lets
// two operations on different tables run at once in two waves of one block.
#pragma once
#include "moe_common.h"

namespace slot_dev {

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

struct LdsTable {
    uint64_t stats[18];        // the table's counters, written back once at the end
    alignas(16) int16_t slot_of[MOE_NUM_EXPERTS];
    alignas(16) int16_t eid_of[MOE_NUM_EXPERTS];
    alignas(16) uint32_t stamp[MOE_NUM_EXPERTS];
    uint32_t protect[16];      // bitmap over expert ids
    uint32_t resident[16];
    uint32_t pred[16];
    uint32_t fetched[16];
    uint32_t spare[16];        // step: its own ids (never the fallback victim)
    uint32_t snap_r[16];       // step: the residency snapshot of the last prefetch
    int32_t list_e[MOE_MAX_PREFETCH];
    int32_t list_s[MOE_MAX_PREFETCH];
    int32_t n_list;
};

// Index of each counter in SlotTable::acct (the order of c_end_decode_token's 10 words).
enum { AC_DEV_LRU_HIT = 0, AC_DEV_MISS, AC_DEV_PF_LOADS, AC_DEV_PF_HITS, AC_DEV_PF_WASTED, AC_DEV_DEM_RE16,
       AC_DEV_DEM_RE64, AC_DEV_PF_RE16, AC_DEV_PF_RE64, AC_DEV_BYTES };

__device__ __forceinline__ bool bit(const uint32_t* bm, int e) { return (bm[e >> 5] >> (e & 31)) & 1u; }

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        uint64_t w = __shfl_xor(v, o, 64);
        v = w < v ? w : v;
    }
    return v;
}

// Everything an operation reads from its table, in one wave's registers: the three arrays
// (entries 8 lane .. 8 lane + 7, one 128-bit load per array and lane), the header, the counters
// and the snapshot bitmaps.  fetch_table issues every load before any is used, so the whole
// table arrives in one round trip; a caller with other work to do (the router's last block)
// fetches early and lets the loads fly meanwhile.  Only the free stack is read later, by the
// allocations that pop it (while the pool is still filling).
struct TabRegs {
    uint4 so, eo, s0, s1;
    int4 hdr;                  // capacity, n_free, clock, snap_valid
    int32_t sched;
    int32_t acct_on, acct_token;
    uint64_t ebytes, stage_bytes;
    uint64_t stat;             // stats[lane] for lane < 18
    uint32_t sr, sp, sf;       // snapshot bitmap words [lane & 15]
};

__device__ __forceinline__ TabRegs fetch_table(const SlotTable* t, int lane) {
    static_assert(MOE_NUM_EXPERTS == 64 * 8, "one 8-entry vector per lane");
    static_assert(offsetof(SlotTable, capacity) == 0 && offsetof(SlotTable, n_free) == 4 &&
                      offsetof(SlotTable, clock) == 8 && offsetof(SlotTable, snap_valid) == 12,
                  "header read as one int4");
    TabRegs r;
    r.hdr = *reinterpret_cast<const int4*>(t);
    r.so = reinterpret_cast<const uint4*>(t->slot_of)[lane];
    r.eo = reinterpret_cast<const uint4*>(t->eid_of)[lane];
    r.s0 = reinterpret_cast<const uint4*>(t->stamp)[2 * lane];
    r.s1 = reinterpret_cast<const uint4*>(t->stamp)[2 * lane + 1];
    r.sched = t->sched;
    r.acct_on = t->acct_on;
    r.acct_token = t->acct_token;
    r.ebytes = t->expert_bytes;
    r.stage_bytes = t->stage_bytes;
    r.stat = t->stats[lane < 18 ? lane : 0];
    r.sr = reinterpret_cast<const uint32_t*>(t->snap_resident)[lane & 15];
    r.sp = reinterpret_cast<const uint32_t*>(t->snap_pred)[lane & 15];
    r.sf = reinterpret_cast<const uint32_t*>(t->snap_fetched)[lane & 15];
    return r;
}

// Write the fetched table into LDS.  Entries at or past the capacity hold -1 / 0 in every table
// (reset, state import and store_table keep them so); they are masked here anyway.
__device__ inline void commit_table(const TabRegs& r, LdsTable& L, int lane) {
    const int cap = r.hdr.x;
    uint4 eo = r.eo, s0 = r.s0, s1 = r.s1;
    const int i0 = 8 * lane;
    if (i0 + 8 > cap) {                        // mask the entries past the capacity
        uint32_t e[4] = {eo.x, eo.y, eo.z, eo.w};
        uint32_t st[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (i0 + j < cap) continue;
            e[j >> 1] |= 0xFFFFu << (16 * (j & 1));
            st[j] = 0u;
        }
        eo = make_uint4(e[0], e[1], e[2], e[3]);
        s0 = make_uint4(st[0], st[1], st[2], st[3]);
        s1 = make_uint4(st[4], st[5], st[6], st[7]);
    }
    reinterpret_cast<uint4*>(L.slot_of)[lane] = r.so;
    reinterpret_cast<uint4*>(L.eid_of)[lane] = eo;
    reinterpret_cast<uint4*>(L.stamp)[2 * lane] = s0;
    reinterpret_cast<uint4*>(L.stamp)[2 * lane + 1] = s1;
    if (lane < 16) {
        L.protect[lane] = 0;
        L.resident[lane] = 0;
        L.pred[lane] = 0;
        L.fetched[lane] = 0;
        L.spare[lane] = 0;
        L.snap_r[lane] = r.sr;
    }
    if (lane == 0) L.n_list = 0;
    if (lane < 18) L.stats[lane] = r.stat;
    wave_sync();
}

// Entries past the capacity are -1 / 0 in LDS as well (commit_table masks them and no operation
// touches them), so the whole arrays are written back.
__device__ inline void store_table(SlotTable* t, const LdsTable& L, int lane) {
    reinterpret_cast<uint4*>(t->slot_of)[lane] = reinterpret_cast<const uint4*>(L.slot_of)[lane];
    reinterpret_cast<uint4*>(t->eid_of)[lane] = reinterpret_cast<const uint4*>(L.eid_of)[lane];
    reinterpret_cast<uint4*>(t->stamp)[2 * lane] = reinterpret_cast<const uint4*>(L.stamp)[2 * lane];
    reinterpret_cast<uint4*>(t->stamp)[2 * lane + 1] = reinterpret_cast<const uint4*>(L.stamp)[2 * lane + 1];
}

// Relabel stamps by rank when the clock nears wrap-around (order unchanged).
__device__ inline void renorm(int cap, LdsTable& L, int lane, uint32_t& clock) {
    if (clock < STAMP_RENORM_AT) return;
    uint32_t newst[MOE_NUM_EXPERTS / 64];
    for (int i = 0; i < MOE_NUM_EXPERTS / 64; ++i) {
        int s = lane + 64 * i;
        newst[i] = 0;
        if (s < cap && L.stamp[s]) {
            uint32_t mine = L.stamp[s], rank = 1;
            for (int q = 0; q < cap; ++q) rank += (L.stamp[q] && L.stamp[q] < mine);
            newst[i] = rank;
        }
    }
    wave_sync();
    uint32_t n = 0;
    for (int i = 0; i < MOE_NUM_EXPERTS / 64; ++i) {
        int s = lane + 64 * i;
        if (s < cap) { L.stamp[s] = newst[i]; n += newst[i] != 0; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o, 64);
    clock = n;
    wave_sync();
}

// One victim for a slot allocation (uniform across the wave). Returns the slot.  When every
// resident expert is protected, the oldest one not in `spare` (may be null) goes before the
// oldest outright (the host table's rule, slot_table_host.h).  evlog (null when not counting)
// gets the open token's number at the evicted expert.
__device__ inline int take_slot(const SlotTable* t, int cap, LdsTable& L, int lane, int& n_free,
                                const uint32_t* protect, const uint32_t* spare, int32_t* evlog, int token) {
    if (n_free > 0) {
        --n_free;
        return t->free_stack[n_free];
    }
    uint64_t best = ~0ull, oldest = ~0ull, spared = ~0ull;
    for (int s = lane; s < cap; s += 64) {
        uint32_t st = L.stamp[s];
        if (!st) continue;
        uint64_t key = ((uint64_t)st << 32) | (uint32_t)s;
        oldest = key < oldest ? key : oldest;
        int e = L.eid_of[s];
        if (e >= 0 && !bit(protect, e)) best = key < best ? key : best;
        if (spare && e >= 0 && !bit(spare, e)) spared = key < spared ? key : spared;
    }
    best = wave_min_u64(best);
    oldest = wave_min_u64(oldest);
    spared = wave_min_u64(spared);
    uint64_t pick = (best != ~0ull) ? best : (spared != ~0ull ? spared : oldest);
    int s = (int)(pick & 0xFFFFFFFFu);
    wave_sync();
    if (lane == 0 && pick != ~0ull) {
        int e = L.eid_of[s];
        if (e >= 0) {
            L.slot_of[e] = -1;
            if (evlog) evlog[e] = token;
        }
        L.eid_of[s] = -1;
        L.stamp[s] = 0;
    }
    wave_sync();
    return pick == ~0ull ? -1 : s;
}

// Bind expert e to slot s at the MRU end (an already-resident expert is only refreshed).
__device__ inline void bind(LdsTable& L, int lane, int e, int s, uint32_t& clock) {
    if (lane == 0) {
        int cur = L.slot_of[e];
        if (cur >= 0) {
            L.stamp[cur] = ++clock;
        } else {
            L.slot_of[e] = (int16_t)s;
            L.eid_of[s] = (int16_t)e;
            L.stamp[s] = ++clock;
        }
    }
    clock = __shfl(clock, 0, 64);
    wave_sync();
}

__device__ inline void count_runs(LdsTable& L, const int32_t* e, int n) {
    if (n <= 0) return;
    int32_t v[MOE_MAX_PREFETCH];
    for (int i = 0; i < n; ++i) v[i] = e[i];
    for (int i = 1; i < n; ++i) {
        int32_t x = v[i];
        int j = i;
        while (j > 0 && v[j - 1] > x) { v[j] = v[j - 1]; --j; }
        v[j] = x;
    }
    int runs = 1;
    for (int i = 1; i < n; ++i) runs += (v[i] != v[i - 1] + 1);
    L.stats[ST_UNCOAL] += (uint64_t)n * MOE_NUM_TENSORS;
    L.stats[ST_COAL] += (uint64_t)runs * MOE_NUM_TENSORS;
}

// Reload counting of expert_io.c:98-111 for the experts that lanes with `mine` set are about to
// load: one whose last eviction was at most 16 / 64 tokens ago counts as a reload; its mark is
// cleared.  Called only with a token open.  Returns the two counts (uniform).
__device__ inline int2 note_reloads(int32_t* __restrict__ evicted_at, bool mine, int e, int token) {
    bool r16 = false, r64 = false;
    if (mine) {
        const int32_t ev = evicted_at[e];
        if (ev >= 0 && token >= ev) {
            r16 = token - ev <= 16;
            r64 = token - ev <= 64;
        }
        evicted_at[e] = -1;
    }
    return make_int2(__popcll(__ballot(r16)), __popcll(__ballot(r64)));
}

// Decode step of expert_io.c:583-685 for k ids (one wave).  r holds the table as fetch_table
// read it; lane i < k holds the i-th id in id_lane.
__device__ inline void dev_slot_step(SlotTable* __restrict__ t, LdsTable& L, const TabRegs& r, uint32_t id_lane,
                                     int k, uint32_t* __restrict__ slot_inds, int lane) {
    commit_table(r, L, lane);
    const int cap = r.hdr.x;
    int n_free = r.hdr.y;
    uint32_t clock = (uint32_t)r.hdr.z;
    renorm(cap, L, lane, clock);

    int e = -1;
    bool bad = false;
    if (lane < k) {
        bad = id_lane >= MOE_NUM_EXPERTS;
        e = bad ? -1 : (int)id_lane;
    }
    if (__any(bad)) {                      // reject: leave the table untouched
        if (lane == 0) { t->status = 1; t->n_copy = 0; }
        return;
    }
    if (lane < k) L.list_s[lane] = e;
    wave_sync();
    bool dup = false;
    for (int q = 0; q < lane && lane < k; ++q) dup |= (L.list_s[q] == e);
    if (__any(dup)) {                      // repeated id: reject, table untouched
        if (lane == 0) { t->status = 2; t->n_copy = 0; }
        return;
    }
    if (e >= 0) {
        atomicOr(&L.protect[e >> 5], 1u << (e & 31));
        atomicOr(&L.spare[e >> 5], 1u << (e & 31));
    }
    wave_sync();

    const bool snap = r.hdr.w != 0;
    if (lane == 0) L.stats[ST_DEC_REQ] += (uint64_t)k;
    if (snap && lane < 16) {
        // per 32-bit word of the bitmaps (the counters are sums of popcounts); lane < 16 holds
        // word `lane` of each snapshot bitmap
        uint32_t want = L.protect[lane], before_missing = want & ~r.sr;
        uint32_t c0 = __popc(want & r.sp), c1 = __popc(want), c2 = __popc(r.sp);
        uint32_t c3 = __popc(before_missing & r.sf), c4 = __popc(before_missing), c5 = __popc(r.sf);
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) {
            c0 += __shfl_xor(c0, o, 16); c1 += __shfl_xor(c1, o, 16); c2 += __shfl_xor(c2, o, 16);
            c3 += __shfl_xor(c3, o, 16); c4 += __shfl_xor(c4, o, 16); c5 += __shfl_xor(c5, o, 16);
        }
        if (lane == 0) {
            L.stats[ST_PRED_HITS] += c0; L.stats[ST_PRED_ACTUAL] += c1; L.stats[ST_PRED_TOTAL] += c2;
            L.stats[ST_MISS_PREF_HITS] += c3; L.stats[ST_MISS_ACTUAL] += c4; L.stats[ST_MISS_FETCHED] += c5;
        }
    }

    // classify in id order
    const bool resident = (e >= 0) && L.slot_of[e] >= 0;
    const bool miss = (e >= 0) && !resident;
    bool lru_hit = false;
    if (resident) lru_hit = !snap || bit(L.snap_r, e);
    const uint64_t miss_mask = __ballot(miss);
    const int n_miss = __popcll(miss_mask);
    const int n_lru = __popcll(__ballot(lru_hit));
    const int n_pref = __popcll(__ballot(resident && !lru_hit));
    if (lane == 0) {
        L.stats[ST_DEC_LRU_HIT] += n_lru;
        L.stats[ST_DEC_PREF_HIT] += n_pref;
        L.stats[ST_DEC_MISS] += n_miss;
        t->snap_valid = 0;
    }
    if (miss) {
        int rank = __popcll(miss_mask & ((1ull << lane) - 1));
        L.list_e[rank] = e;
    }
    wave_sync();
    if ((r.sched & 1) && snap && lane < 16)  // in-flight prefetched experts are protected too
        L.protect[lane] |= r.sf;
    wave_sync();

    // accounting: the misses' reloads are counted before the victims are marked (the two sets
    // are disjoint: a victim is resident, a miss is not)
    const bool counting = r.acct_on != 0;
    const int token = r.acct_token;
    int32_t* evlog = (counting && token >= 0) ? t->evicted_at : nullptr;
    if (counting) {
        const int2 re = evlog ? note_reloads(t->evicted_at, miss, e, token) : make_int2(0, 0);
        uint32_t fetched = 0;
        if (snap) {
            fetched = lane < 16 ? __popc(r.sf) : 0u;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) fetched += __shfl_xor(fetched, o, 64);
        }
        if (lane == 0) {
            uint64_t* a = t->acct;
            a[AC_DEV_LRU_HIT] += (uint64_t)n_lru;
            a[AC_DEV_MISS] += (uint64_t)n_miss;
            if (snap) {
                a[AC_DEV_PF_HITS] += (uint64_t)n_pref;
                if (fetched >= (uint32_t)n_pref) a[AC_DEV_PF_WASTED] += fetched - (uint32_t)n_pref;
            }
            a[AC_DEV_DEM_RE16] += (uint64_t)re.x;
            a[AC_DEV_DEM_RE64] += (uint64_t)re.y;
            a[AC_DEV_BYTES] += (uint64_t)n_miss * r.stage_bytes;
        }
    }

    for (int r = 0; r < n_miss; ++r) {
        int me = L.list_e[r];
        int s = take_slot(t, cap, L, lane, n_free, L.protect, L.spare, evlog, token);
        bind(L, lane, me, s, clock);
        if (lane == 0) L.list_s[r] = s;
    }
    wave_sync();
    if (lane < n_miss) {
        t->copy_eid[lane] = L.list_e[lane];
        t->copy_slot[lane] = L.list_s[lane];
    }
    wave_sync();

    // refresh every id in order; for a repeated id only its last occurrence counts
    int my_slot = -1;
    if (e >= 0) {                          // ids are distinct: refresh in id order
        my_slot = L.slot_of[e];
        if (my_slot >= 0) L.stamp[my_slot] = clock + 1 + lane;
        slot_inds[lane] = (uint32_t)my_slot;
    }
    clock += (uint32_t)k;
    wave_sync();

    if ((r.sched & 2) && n_miss > 0 && n_miss < k) {   // the split lists, ids in order
        const uint64_t below = (1ull << lane) - 1;
        const uint64_t hit_mask = __ballot(resident);
        const int n_hit = k - n_miss;
        SplitLists& S = t->split;
        if (resident) {
            const int h = __popcll(hit_mask & below);
            S.hit[h] = (uint32_t)my_slot;
            S.inv[lane] = h;
        } else if (miss) {
            const int m = __popcll(miss_mask & below);
            S.miss[m] = (uint32_t)my_slot;
            S.inv[lane] = n_hit + m;
        }
        if (lane == 0) { S.n_hit = n_hit; S.n_miss = n_miss; S.k = k; }
    }

    store_table(t, L, lane);
    if (lane == 0) {
        t->n_copy = n_miss;
        t->clock = clock;
        t->n_free = n_free;
        t->status = 0;
        L.stats[ST_DEC_BYTES] += (uint64_t)n_miss * r.ebytes;
        count_runs(L, L.list_e, n_miss);
    }
    wave_sync();
    if (lane < 18) t->stats[lane] = L.stats[lane];
}

// Prefetch of expert_io.c:527-581 for m predictions (one wave).  r holds the table as
// fetch_table read it; preds is in LDS.
__device__ inline void dev_slot_prefetch(SlotTable* __restrict__ t, LdsTable& L, const TabRegs& r, const int32_t* preds,
                                         int m, int max_fetch, int lane) {
    const bool sched = (r.sched & 1) != 0;
    if (sched && max_fetch <= 0) {            // the scheduler variant prefetches nothing
        if (lane == 0) { t->pf_n_copy = 0; t->status = 0; }
        return;
    }
    commit_table(r, L, lane);
    const int cap = r.hdr.x;
    int n_free = r.hdr.y;
    uint32_t clock = (uint32_t)r.hdr.z;
    renorm(cap, L, lane, clock);

    // residency snapshot
    for (int e = lane; e < MOE_NUM_EXPERTS; e += 64)
        if (L.slot_of[e] >= 0) atomicOr(&L.resident[e >> 5], 1u << (e & 31));
    wave_sync();
    if (lane == 0) {
        int cap = (max_fetch > 0 && max_fetch < 32) ? max_fetch : 32;
        int np = 0;
        for (int i = 0; i < m; ++i) {
            int e = preds[i];
            if (e < 0 || e >= MOE_NUM_EXPERTS) continue;
            L.pred[e >> 5] |= 1u << (e & 31);
            L.protect[e >> 5] |= 1u << (e & 31);
            if (L.slot_of[e] < 0 && np < cap && !(sched && bit(L.fetched, e))) {
                L.list_e[np++] = e;
                L.fetched[e >> 5] |= 1u << (e & 31);
            }
        }
        L.n_list = np;
    }
    wave_sync();
    const int np = L.n_list;
    if (lane < 16) {
        reinterpret_cast<uint32_t*>(t->snap_resident)[lane] = L.resident[lane];
        reinterpret_cast<uint32_t*>(t->snap_pred)[lane] = L.pred[lane];
        reinterpret_cast<uint32_t*>(t->snap_fetched)[lane] = L.fetched[lane];
    }
    int32_t order_e[MOE_MAX_PREFETCH];
    for (int i = 0; i < np; ++i) order_e[i] = L.list_e[np - 1 - i];   // reverse rank order
    const bool counting = r.acct_on != 0;
    const int token = r.acct_token;
    int32_t* evlog = (counting && token >= 0) ? t->evicted_at : nullptr;
    if (counting) {                           // reloads first: the picks are not resident
        const int2 re = evlog ? note_reloads(t->evicted_at, lane < np, lane < np ? L.list_e[lane] : 0, token)
                              : make_int2(0, 0);
        if (lane == 0) {
            uint64_t* a = t->acct;
            a[AC_DEV_PF_LOADS] += (uint64_t)np;
            a[AC_DEV_PF_RE16] += (uint64_t)re.x;
            a[AC_DEV_PF_RE64] += (uint64_t)re.y;
            a[AC_DEV_BYTES] += (uint64_t)np * r.stage_bytes;
        }
    }
    wave_sync();
    for (int i = 0; i < np; ++i) {
        int s = take_slot(t, cap, L, lane, n_free, L.protect, nullptr, evlog, token);
        bind(L, lane, order_e[i], s, clock);
        if (lane == 0) { L.list_e[i] = order_e[i]; L.list_s[i] = s; }
    }
    wave_sync();
    store_table(t, L, lane);
    if (lane < np) {
        t->pf_copy_eid[lane] = L.list_e[lane];
        t->pf_copy_slot[lane] = L.list_s[lane];
    }
    if (lane == 0) {
        t->snap_valid = 1;
        t->pf_n_copy = np;
        t->clock = clock;
        t->n_free = n_free;
        t->status = 0;
        L.stats[ST_PREF_BYTES] += (uint64_t)np * r.ebytes;
        count_runs(L, L.list_e, np);
    }
    wave_sync();
    if (lane < 18) t->stats[lane] = L.stats[lane];
}

}  // namespace slot_dev
