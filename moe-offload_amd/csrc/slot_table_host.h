// Host-side operations on a SlotTable (the host-driven path and every table query).
//
// Behaviour restated from mlx-qwen38/expert_io.c (file:line there):
//   reset 450-468, victim choice 404-426, insert/refresh 387-402, decode step 583-685,
//   prefetch 527-581, state export/import 726-789, coalescing counters 187-276.
// Scheduler variant and per-token accounting of mlx-qwen38/cpp/third_party/expert_io.c:
//   the step's victim choice may also protect the experts the layer's last prefetch fetched
//   and reports which ids were resident (1141-1146, 1257-1276); the prefetch may skip a
//   repeated prediction (1311-1322); evictions are stamped with the token number and re-loads within
//   16 / 64 tokens counted (493-525, 656-666, 756-768).
// The table is kept in recency-stamp form (see SlotTable).
#pragma once
#include <string.h>

#include "moe_common.h"

namespace slot_host {

static inline bool bm_get(const uint64_t* bm, int e) { return (bm[e >> 6] >> (e & 63)) & 1ULL; }
static inline void bm_put(uint64_t* bm, int e) { bm[e >> 6] |= 1ULL << (e & 63); }

// Per-token accounting (c_end_decode_token's 10 counters).  Null when accounting is off.
enum { AC_LRU_HIT = 0, AC_MISS, AC_PF_LOADS, AC_PF_HITS, AC_PF_WASTED, AC_DEM_RE16, AC_DEM_RE64, AC_PF_RE16,
       AC_PF_RE64, AC_BYTES };
struct Acct {
    int32_t cur_token;      // token number of the open token, -1 when none is open
    int32_t* evicted_at;    // per expert: token number of its last eviction, -1 = none
    uint64_t* tok;          // the 10 counters
};

static inline void note_reload(Acct* a, int e, int re16, int re64) {
    if (!a || a->cur_token < 0) return;
    int32_t ev = a->evicted_at[e];
    if (ev >= 0 && a->cur_token >= ev) {
        int32_t d = a->cur_token - ev;
        if (d <= 16) a->tok[re16]++;
        if (d <= 64) a->tok[re64]++;
    }
    a->evicted_at[e] = -1;
}

static inline void renorm_if_needed(SlotTable* t) {
    if (t->clock < STAMP_RENORM_AT) return;
    // Relabel resident stamps by rank; order is unchanged.
    int order[MOE_NUM_EXPERTS], n = 0;
    for (int s = 0; s < t->capacity; ++s)
        if (t->stamp[s]) order[n++] = s;
    for (int i = 1; i < n; ++i) {
        int v = order[i], j = i;
        while (j > 0 && t->stamp[order[j - 1]] > t->stamp[v]) { order[j] = order[j - 1]; --j; }
        order[j] = v;
    }
    for (int i = 0; i < n; ++i) t->stamp[order[i]] = (uint32_t)(i + 1);
    t->clock = (uint32_t)n;
}

static inline void touch(SlotTable* t, int s) {
    renorm_if_needed(t);
    t->stamp[s] = ++t->clock;
}

static inline void reset_cache(SlotTable* t) {
    for (int i = 0; i < MOE_NUM_EXPERTS; ++i) {
        t->slot_of[i] = -1;
        t->eid_of[i] = -1;
        t->stamp[i] = 0;
    }
    t->n_free = t->capacity;
    for (int i = 0; i < t->capacity; ++i) t->free_stack[i] = (int16_t)(t->capacity - 1 - i);
    t->clock = 0;
    t->snap_valid = 0;
    t->n_copy = 0;
    t->pf_n_copy = 0;
    t->status = 0;
    t->io_fault = 0;
    for (int i = 0; i < MOE_NUM_EXPERTS; ++i) t->evicted_at[i] = -1;
}

static inline void reset_stats(SlotTable* t) { memset(t->stats, 0, sizeof(t->stats)); }

static inline void init(SlotTable* t, int capacity, uint64_t expert_bytes) {
    memset(t, 0, sizeof(*t));
    t->capacity = capacity;
    t->expert_bytes = expert_bytes;
    t->acct_token = -1;
    reset_cache(t);
}

// Victim: pop the free stack, else the oldest resident slot whose expert is not protected,
// else (every resident expert protected) the oldest one not in `spare` (the step's own ids;
// may be null), else the oldest resident slot.  The reference's last resort is the oldest
// slot outright; the two differ only when that slot holds one of the step's ids, which the
// published step never reaches (k <= capacity) and where the scheduler step of the reference
// goes on to index slot -1 (undefined behaviour there).
static inline int take_slot(SlotTable* t, const uint64_t* protect, Acct* a = nullptr,
                            const uint64_t* spare = nullptr) {
    if (t->n_free > 0) return t->free_stack[--t->n_free];
    int best = -1, oldest = -1, spared = -1;
    for (int s = 0; s < t->capacity; ++s) {
        uint32_t st = t->stamp[s];
        if (!st) continue;
        if (oldest < 0 || st < t->stamp[oldest]) oldest = s;
        if (!bm_get(protect, t->eid_of[s]) && (best < 0 || st < t->stamp[best])) best = s;
        if (spare && !bm_get(spare, t->eid_of[s]) && (spared < 0 || st < t->stamp[spared])) spared = s;
    }
    if (best < 0) best = spared;
    if (best < 0) best = oldest;
    if (best < 0) return -1;                 // empty table with no free slot (capacity 0)
    int e = t->eid_of[best];
    if (e >= 0) {
        t->slot_of[e] = -1;
        if (a && a->cur_token >= 0) a->evicted_at[e] = a->cur_token;
    }
    t->eid_of[best] = -1;
    t->stamp[best] = 0;
    return best;
}

static inline void bind(SlotTable* t, int e, int s) {
    if (t->slot_of[e] >= 0) { touch(t, t->slot_of[e]); return; }
    t->slot_of[e] = (int16_t)s;
    t->eid_of[s] = (int16_t)e;
    touch(t, s);
}

static inline void count_runs(SlotTable* t, const int32_t* eids, int n) {
    if (n <= 0) return;
    int32_t v[MOE_NUM_EXPERTS];
    memcpy(v, eids, (size_t)n * sizeof(int32_t));
    for (int i = 1; i < n; ++i) {
        int32_t x = v[i];
        int j = i;
        while (j > 0 && v[j - 1] > x) { v[j] = v[j - 1]; --j; }
        v[j] = x;
    }
    int runs = 1;
    for (int i = 1; i < n; ++i) runs += (v[i] != v[i - 1] + 1);
    t->stats[ST_UNCOAL] += (uint64_t)n * MOE_NUM_TENSORS;
    t->stats[ST_COAL] += (uint64_t)runs * MOE_NUM_TENSORS;
}

// Decode step.  Writes every id's slot to out_slots and the copies needed to t->copy_*.
// extra_protect (may be null) joins the step's ids in the victim protection; is_hit (may be
// null) gets whether each id was resident when classified.
static inline int step(SlotTable* t, const uint32_t* eids, int k, uint32_t* out_slots,
                       const uint64_t* extra_protect = nullptr, uint8_t* is_hit = nullptr, Acct* a = nullptr) {
    uint64_t want[8] = {0}, protect[8];
    int32_t miss[MOE_MAX_K];
    int n_miss = 0;
    t->stats[ST_DEC_REQ] += (uint64_t)k;
    for (int i = 0; i < k; ++i) bm_put(want, (int)eids[i]);
    for (int w = 0; w < 8; ++w) protect[w] = want[w] | (extra_protect ? extra_protect[w] : 0ULL);
    uint64_t fetched = 0, lru_h = 0, pref_h = 0;
    const bool had_snap = t->snap_valid != 0;
    if (had_snap) {
        for (int w = 0; w < 8; ++w) {
            uint64_t before_missing = want[w] & ~t->snap_resident[w];
            t->stats[ST_PRED_HITS] += (uint64_t)__builtin_popcountll(want[w] & t->snap_pred[w]);
            t->stats[ST_PRED_ACTUAL] += (uint64_t)__builtin_popcountll(want[w]);
            t->stats[ST_PRED_TOTAL] += (uint64_t)__builtin_popcountll(t->snap_pred[w]);
            t->stats[ST_MISS_PREF_HITS] += (uint64_t)__builtin_popcountll(before_missing & t->snap_fetched[w]);
            t->stats[ST_MISS_ACTUAL] += (uint64_t)__builtin_popcountll(before_missing);
            t->stats[ST_MISS_FETCHED] += (uint64_t)__builtin_popcountll(t->snap_fetched[w]);
            fetched += (uint64_t)__builtin_popcountll(t->snap_fetched[w]);
        }
    }
    for (int i = 0; i < k; ++i) {
        int e = (int)eids[i];
        const bool res = t->slot_of[e] >= 0;
        if (is_hit) is_hit[i] = res;
        if (res) {
            if (!had_snap || bm_get(t->snap_resident, e)) { t->stats[ST_DEC_LRU_HIT]++; lru_h++; }
            else { t->stats[ST_DEC_PREF_HIT]++; pref_h++; }
        } else {
            t->stats[ST_DEC_MISS]++;
            miss[n_miss++] = e;
        }
    }
    if (a) {
        a->tok[AC_LRU_HIT] += lru_h;
        a->tok[AC_MISS] += (uint64_t)n_miss;
        if (had_snap) {
            a->tok[AC_PF_HITS] += pref_h;
            if (fetched >= pref_h) a->tok[AC_PF_WASTED] += fetched - pref_h;
        }
    }
    t->snap_valid = 0;
    t->n_copy = 0;
    for (int i = 0; i < n_miss; ++i) {
        int s = take_slot(t, protect, a, want);
        note_reload(a, miss[i], AC_DEM_RE16, AC_DEM_RE64);
        bind(t, miss[i], s);
        t->copy_eid[t->n_copy] = miss[i];
        t->copy_slot[t->n_copy] = s;
        t->n_copy++;
    }
    t->stats[ST_DEC_BYTES] += (uint64_t)n_miss * t->expert_bytes;
    for (int i = 0; i < k; ++i) {
        int s = t->slot_of[eids[i]];
        touch(t, s);
        out_slots[i] = (uint32_t)s;
    }
    count_runs(t, miss, n_miss);
    return n_miss;
}

// Prefetch.  dedupe: a prediction already taken in this call is not taken again (the
// scheduler variant); the published entry point takes it twice.
static inline int prefetch(SlotTable* t, const int32_t* preds, int n, int max_fetch, bool dedupe = false,
                           Acct* a = nullptr) {
    memset(t->snap_resident, 0, sizeof(t->snap_resident));
    memset(t->snap_pred, 0, sizeof(t->snap_pred));
    memset(t->snap_fetched, 0, sizeof(t->snap_fetched));
    for (int e = 0; e < MOE_NUM_EXPERTS; ++e)
        if (t->slot_of[e] >= 0) bm_put(t->snap_resident, e);
    t->snap_valid = 1;
    t->pf_n_copy = 0;
    int cap = (max_fetch > 0 && max_fetch < 32) ? max_fetch : 32;
    uint64_t protect[8] = {0};
    int32_t pick[MOE_MAX_PREFETCH];
    int np = 0;
    for (int i = 0; i < n; ++i) {
        int e = preds[i];
        if (e < 0 || e >= MOE_NUM_EXPERTS) continue;
        bm_put(t->snap_pred, e);
        bm_put(protect, e);
        if (t->slot_of[e] < 0 && np < cap && !(dedupe && bm_get(t->snap_fetched, e))) {
            pick[np++] = e;
            bm_put(t->snap_fetched, e);
        }
    }
    for (int i = 0; i < np; ++i) {
        int e = pick[np - 1 - i];
        int s = take_slot(t, protect, a);
        note_reload(a, e, AC_PF_RE16, AC_PF_RE64);
        bind(t, e, s);
        t->pf_copy_eid[i] = e;
        t->pf_copy_slot[i] = s;
    }
    t->pf_n_copy = np;
    if (a) a->tok[AC_PF_LOADS] += (uint64_t)np;
    t->stats[ST_PREF_BYTES] += (uint64_t)np * t->expert_bytes;
    count_runs(t, t->pf_copy_eid, np);
    return np;
}

static inline int get_state(const SlotTable* t, int32_t* eids, int32_t* slots) {
    int order[MOE_NUM_EXPERTS], n = 0;
    for (int s = 0; s < t->capacity; ++s)
        if (t->stamp[s]) order[n++] = s;
    for (int i = 1; i < n; ++i) {
        int v = order[i], j = i;
        while (j > 0 && t->stamp[order[j - 1]] > t->stamp[v]) { order[j] = order[j - 1]; --j; }
        order[j] = v;
    }
    for (int i = 0; i < n; ++i) {
        eids[i] = t->eid_of[order[i]];
        slots[i] = order[i];
    }
    return n;
}

static inline void set_state(SlotTable* t, const int32_t* eids, const int32_t* slots, int n,
                             uint64_t add_req, uint64_t add_hits, uint64_t add_miss) {
    t->stats[ST_PRE_REQ] += add_req;
    t->stats[ST_PRE_HIT] += add_hits;
    t->stats[ST_PRE_MISS] += add_miss;
    for (int i = 0; i < MOE_NUM_EXPERTS; ++i) {
        t->slot_of[i] = -1;
        t->eid_of[i] = -1;
        t->stamp[i] = 0;
    }
    t->clock = 0;
    t->snap_valid = 0;
    uint8_t used[MOE_NUM_EXPERTS] = {0};
    for (int i = 0; i < n; ++i) {
        used[slots[i]] = 1;
        bind(t, eids[i], slots[i]);
    }
    t->n_free = 0;
    for (int s = t->capacity - 1; s >= 0; --s)
        if (!used[s]) t->free_stack[t->n_free++] = (int16_t)s;
}

}  // namespace slot_host
