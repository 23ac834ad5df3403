/*
 * lru.c -- plain-C restatement of the per-layer expert slot LRU of the reference's
 * `mlx-qwen38/expert_io.c` (TEST INFRASTRUCTURE ONLY: what the tests compare the HIP
 * library's host and device LRU tables with; never linked into the product).
 *
 * Restated behaviour (file:line of `mlx-qwen38/expert_io.c`):
 *   reset             450-468  all maps -1, free stack [cap-1 .. 0] so pops yield 0,1,2,..
 *   list helpers      358-402  doubly linked list over slots, head = LRU, tail = MRU;
 *                              inserting an already-resident eid only refreshes it
 *   victim choice     404-426  free stack first, else first slot from the LRU end whose eid
 *                              is not protected, else the LRU head
 *   decode step       583-685  classify in id order (lru hit / prefetch hit / miss, via the
 *                              residency snapshot a prefetch leaves), predictor counters by
 *                              popcount, allocate misses protecting the step's ids, refresh
 *                              every id to MRU in id order and report its slot
 *   prefetch          527-581  snapshot residency, cap = max_fetch in (0,32) else 32, take
 *                              non-resident predictions in rank order, insert them in reverse
 *                              rank order protecting all predictions
 *   state get/set     726-789  LRU->MRU export; import rebuilds the free stack descending
 *   counters          791-852  18 per-layer u64, 6 decode totals over layers 1..n-1
 *   coalescing        187-276  (counters only) sort misses by eid, count contiguous runs
 * Expert bytes are a per-layer parameter here; the reference hard-codes 1,536,000.
 *
 * Superset entry points of `mlx-qwen38/cpp/third_party/expert_io.c` (same decisions as above,
 * plus the scheduler variant and per-token accounting):
 *   sched step        1094-1394  one call per layer: decode step of `l` (skipped for l <= 0)
 *                                whose victim choice also protects the experts the last
 *                                prefetch of `l` fetched; optional split of the step's slots
 *                                into hit / miss lists with the inverse order; then a prefetch
 *                                of `next` (only when 0 < next, preds given, cap > 0 and not
 *                                NO_PREFETCH) that skips repeated predictions
 *   split lists       1062-1092  kept per layer until the next split (stale otherwise)
 *   token accounting  1002-1038  10 per-token counters; evictions stamped with the token
 *                                number (493-525), re-reads within 16 / 64 tokens counted
 *                                when an evicted expert is loaded again (656-666, 756-768)
 *   reset             551-574    layer 1's reset also restarts the token numbering
 * "Bytes read" (out10[9]) is the staged byte count per expert set with
 * o_layer_set_staged_bytes (0 for accounting-only layers, as the reference reports for
 * zero-length reads).
 *
 * Pinned by: golden traces written by the reference's own expert_io.c compiled from source
 * (tests/golden/make_lru_traces.py), the independent OrderedDict restatement in lru.py, and
 * invariants / brute force in tests/test_oracle_lru.py.
 */
#include <stdint.h>
#include <string.h>

#define O_MAX_LAYERS 64
#define O_NUM_EXPERTS 512
#define O_NUM_TENSORS 9

typedef struct {
    int capacity;
    uint64_t expert_bytes;
    int16_t slot_of[O_NUM_EXPERTS];   /* eid -> slot or -1 */
    int16_t eid_of[O_NUM_EXPERTS];    /* slot -> eid or -1 */
    int16_t older[O_NUM_EXPERTS];     /* towards the LRU end */
    int16_t newer[O_NUM_EXPERTS];     /* towards the MRU end */
    int16_t lru_end, mru_end;
    int16_t free_stack[O_NUM_EXPERTS];
    int n_free;
    int snap_valid;
    uint64_t snap_resident[8], snap_pred[8], snap_fetched[8];
    uint64_t st[18];
    int32_t evicted_at[O_NUM_EXPERTS];   /* token number of the last eviction, -1 = none */
    uint64_t staged_bytes;               /* bytes one staged expert reads (accounting) */
} OLayer;

static OLayer g_o[O_MAX_LAYERS];

/* scheduler split lists (per layer, kept until the next split) */
static uint32_t g_hit_slots[O_MAX_LAYERS][16], g_miss_slots[O_MAX_LAYERS][16];
static int32_t g_inv[O_MAX_LAYERS][16];
static int g_n_hit[O_MAX_LAYERS], g_n_miss[O_MAX_LAYERS], g_split_k[O_MAX_LAYERS];

/* per-token accounting */
enum { A_LRU_HIT, A_MISS, A_PF_LOADS, A_PF_HITS, A_PF_WASTED, A_DEM_RE16, A_DEM_RE64, A_PF_RE16, A_PF_RE64,
       A_BYTES };
static int g_acct_on = 0;
static int32_t g_token_seq = 0, g_cur_token = -1;
static uint64_t g_tok[10];

static void note_eviction(OLayer *L, int e) {
    if (g_acct_on && g_cur_token >= 0) L->evicted_at[e] = g_cur_token;
}

/* An expert is being loaded again: count it as a re-read when it was evicted recently. */
static void note_reload(OLayer *L, int e, int re16, int re64) {
    if (!(g_acct_on && g_cur_token >= 0)) return;
    int32_t ev = L->evicted_at[e];
    if (ev >= 0 && g_cur_token >= ev) {
        int32_t d = g_cur_token - ev;
        if (d <= 16) g_tok[re16]++;
        if (d <= 64) g_tok[re64]++;
    }
    L->evicted_at[e] = -1;
}

static int bm_has(const uint64_t *bm, int e) { return (int)((bm[e >> 6] >> (e & 63)) & 1ULL); }
static void bm_set(uint64_t *bm, int e) { bm[e >> 6] |= 1ULL << (e & 63); }

static void unlink_slot(OLayer *L, int s) {
    int o = L->older[s], n = L->newer[s];
    if (o >= 0) L->newer[o] = (int16_t)n; else L->lru_end = (int16_t)n;
    if (n >= 0) L->older[n] = (int16_t)o; else L->mru_end = (int16_t)o;
    L->older[s] = L->newer[s] = -1;
}

static void push_mru(OLayer *L, int s) {
    L->older[s] = L->mru_end;
    L->newer[s] = -1;
    if (L->mru_end >= 0) L->newer[L->mru_end] = (int16_t)s; else L->lru_end = (int16_t)s;
    L->mru_end = (int16_t)s;
}

static void refresh(OLayer *L, int s) {
    if (L->mru_end != s) { unlink_slot(L, s); push_mru(L, s); }
}

static void bind(OLayer *L, int e, int s) {
    if (L->slot_of[e] >= 0) { refresh(L, L->slot_of[e]); return; }
    L->slot_of[e] = (int16_t)s;
    L->eid_of[s] = (int16_t)e;
    push_mru(L, s);
}

/* `spare` (may be NULL): when every resident expert is protected, the fallback victim is the
 * oldest one not in `spare` (the step's own ids) rather than the LRU end.  The reference takes
 * the LRU end; that differs only when the LRU end is one of the step's ids, which the
 * published step never reaches (k <= capacity) and where the scheduler step's later list
 * operations index slot -1 (undefined behaviour in the reference). */
static int take_slot(OLayer *L, const uint64_t *protect, const uint64_t *spare) {
    if (L->n_free > 0) return L->free_stack[--L->n_free];
    int s = L->lru_end;
    for (; s >= 0; s = L->newer[s]) {
        int e = L->eid_of[s];
        if (e >= 0 && !bm_has(protect, e)) break;
    }
    if (s < 0 && spare) {
        for (s = L->lru_end; s >= 0; s = L->newer[s]) {
            int e = L->eid_of[s];
            if (e >= 0 && !bm_has(spare, e)) break;
        }
    }
    if (s < 0) s = L->lru_end;            /* every resident expert is protected */
    int e = L->eid_of[s];
    unlink_slot(L, s);
    if (e >= 0) { L->slot_of[e] = -1; note_eviction(L, e); }
    L->eid_of[s] = -1;
    return s;
}

static void count_runs(OLayer *L, const int32_t *eids, int n) {
    if (n <= 0) return;
    int32_t v[O_NUM_EXPERTS];
    memcpy(v, eids, (size_t)n * sizeof(int32_t));
    for (int i = 1; i < n; ++i) {            /* small n: insertion sort */
        int32_t x = v[i]; int j = i;
        while (j > 0 && v[j - 1] > x) { v[j] = v[j - 1]; --j; }
        v[j] = x;
    }
    int runs = 1;
    for (int i = 1; i < n; ++i) runs += (v[i] != v[i - 1] + 1);
    L->st[16] += (uint64_t)n * O_NUM_TENSORS;
    L->st[17] += (uint64_t)runs * O_NUM_TENSORS;
}

void o_layer_reset_cache(int l) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    OLayer *L = &g_o[l];
    for (int i = 0; i < O_NUM_EXPERTS; ++i) L->slot_of[i] = L->eid_of[i] = L->older[i] = L->newer[i] = -1;
    L->lru_end = L->mru_end = -1;
    L->n_free = L->capacity;
    for (int i = 0; i < L->capacity; ++i) L->free_stack[i] = (int16_t)(L->capacity - 1 - i);
    L->snap_valid = 0;
    for (int i = 0; i < O_NUM_EXPERTS; ++i) L->evicted_at[i] = -1;
    if (l == 1) { g_token_seq = 0; g_cur_token = -1; }
}

void o_layer_set_staged_bytes(int l, uint64_t b) {
    if (l >= 0 && l < O_MAX_LAYERS) g_o[l].staged_bytes = b;
}

void o_layer_reset_stats(int l) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    memset(g_o[l].st, 0, sizeof(g_o[l].st));
}

void o_layer_init(int l, int capacity, uint64_t expert_bytes) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    memset(&g_o[l], 0, sizeof(OLayer));
    g_o[l].capacity = capacity;
    g_o[l].expert_bytes = expert_bytes;
    o_layer_reset_cache(l);
}

/* Decode step shared by the published entry point and the scheduler variant.  `extra` (may be
 * NULL) is OR-ed into the victim protection; is_hit[i] (may be NULL) records whether id i was
 * resident when classified. */
static int step_core(OLayer *L, const uint32_t *eids, int k, uint32_t *out_slots, int32_t *miss_eids,
                     int32_t *miss_slots, const uint64_t *extra, uint8_t *is_hit) {
    uint64_t want[8] = {0}, protect[8];
    int n_miss = 0;
    L->st[0] += (uint64_t)k;
    for (int i = 0; i < k; ++i) bm_set(want, (int)eids[i]);
    for (int w = 0; w < 8; ++w) protect[w] = want[w] | (extra ? extra[w] : 0);
    uint64_t fetched_total = 0, lru_h = 0, pref_h = 0;
    const int had_snap = L->snap_valid;
    if (L->snap_valid) {
        for (int w = 0; w < 8; ++w) {
            uint64_t missing_before = want[w] & ~L->snap_resident[w];
            L->st[10] += (uint64_t)__builtin_popcountll(want[w] & L->snap_pred[w]);
            L->st[11] += (uint64_t)__builtin_popcountll(want[w]);
            L->st[12] += (uint64_t)__builtin_popcountll(L->snap_pred[w]);
            L->st[13] += (uint64_t)__builtin_popcountll(missing_before & L->snap_fetched[w]);
            L->st[14] += (uint64_t)__builtin_popcountll(missing_before);
            L->st[15] += (uint64_t)__builtin_popcountll(L->snap_fetched[w]);
            fetched_total += (uint64_t)__builtin_popcountll(L->snap_fetched[w]);
        }
    }
    for (int i = 0; i < k; ++i) {
        int e = (int)eids[i];
        if (is_hit) is_hit[i] = L->slot_of[e] >= 0;
        if (L->slot_of[e] >= 0) {
            if (!L->snap_valid || bm_has(L->snap_resident, e)) { L->st[1]++; lru_h++; }
            else { L->st[2]++; pref_h++; }
        } else {
            L->st[3]++;
            miss_eids[n_miss++] = e;
        }
    }
    if (g_acct_on) {
        g_tok[A_LRU_HIT] += lru_h;
        g_tok[A_MISS] += (uint64_t)n_miss;
        if (had_snap) {
            g_tok[A_PF_HITS] += pref_h;
            if (fetched_total >= pref_h) g_tok[A_PF_WASTED] += fetched_total - pref_h;
        }
        g_tok[A_BYTES] += (uint64_t)n_miss * L->staged_bytes;
    }
    L->snap_valid = 0;
    for (int i = 0; i < n_miss; ++i) {
        int s = take_slot(L, protect, want);
        note_reload(L, miss_eids[i], A_DEM_RE16, A_DEM_RE64);
        bind(L, miss_eids[i], s);
        miss_slots[i] = s;
    }
    L->st[4] += (uint64_t)n_miss * L->expert_bytes;
    for (int i = 0; i < k; ++i) {
        int s = L->slot_of[eids[i]];
        refresh(L, s);
        out_slots[i] = (uint32_t)s;
    }
    count_runs(L, miss_eids, n_miss);
    return n_miss;
}

/* Returns the number of misses; out_slots[k] gets every id's slot, miss_eids/miss_slots
 * (<= 16 each) the demand copies in allocation order. */
int o_layer_step_decode(int l, const uint32_t *eids, int k, uint32_t *out_slots,
                        int32_t *miss_eids, int32_t *miss_slots) {
    if (l < 0 || l >= O_MAX_LAYERS) return 0;
    return step_core(&g_o[l], eids, k, out_slots, miss_eids, miss_slots, NULL, NULL);
}

/* Prefetch shared by both entry points; `dedupe` skips a prediction already taken. */
static int prefetch_core(OLayer *L, const int32_t *preds, int n, int max_fetch, int dedupe,
                         int32_t *fetch_eids, int32_t *fetch_slots) {
    memset(L->snap_resident, 0, sizeof(L->snap_resident));
    memset(L->snap_pred, 0, sizeof(L->snap_pred));
    memset(L->snap_fetched, 0, sizeof(L->snap_fetched));
    for (int e = 0; e < O_NUM_EXPERTS; ++e)
        if (L->slot_of[e] >= 0) bm_set(L->snap_resident, e);
    L->snap_valid = 1;
    int cap = (max_fetch > 0 && max_fetch < 32) ? max_fetch : 32;
    uint64_t protect[8] = {0};
    int32_t pick[32];
    int np = 0;
    for (int i = 0; i < n; ++i) {
        int e = preds[i];
        if (e < 0 || e >= O_NUM_EXPERTS) continue;
        bm_set(L->snap_pred, e);
        bm_set(protect, e);
        if (L->slot_of[e] < 0 && np < cap && !(dedupe && bm_has(L->snap_fetched, e))) {
            pick[np++] = e;
            bm_set(L->snap_fetched, e);
        }
    }
    for (int i = 0; i < np; ++i) {
        int e = pick[np - 1 - i];
        int s = take_slot(L, protect, NULL);
        note_reload(L, e, A_PF_RE16, A_PF_RE64);
        bind(L, e, s);
        fetch_eids[i] = e;
        fetch_slots[i] = s;
    }
    if (g_acct_on) {
        g_tok[A_PF_LOADS] += (uint64_t)np;
        g_tok[A_BYTES] += (uint64_t)np * L->staged_bytes;
    }
    L->st[5] += (uint64_t)np * L->expert_bytes;
    count_runs(L, fetch_eids, np);
    return np;
}

/* Returns the number of experts fetched; fetch_eids/fetch_slots (<= 32) in insertion order. */
int o_layer_start_prefetch(int l, const int32_t *preds, int n, int max_fetch,
                           int32_t *fetch_eids, int32_t *fetch_slots) {
    if (l < 0 || l >= O_MAX_LAYERS) return 0;
    return prefetch_core(&g_o[l], preds, n, max_fetch, 0, fetch_eids, fetch_slots);
}

/* Scheduler entry point.  Returns the step's miss count (0 when the step is skipped);
 * *n_fetch gets the prefetch's count (0 when skipped). */
int o_layer_decode_step_sched(int l, const int32_t *eids, int k, const int32_t *pred, int n_pred, int next,
                              int prefetch_cap, int flags, uint32_t *out_slots, int32_t *miss_eids,
                              int32_t *miss_slots, int32_t *fetch_eids, int32_t *fetch_slots, int *n_fetch) {
    int n_miss = 0;
    *n_fetch = 0;
    if (l > 0 && l < O_MAX_LAYERS && eids && k > 0) {
        if (k > 16) k = 16;
        OLayer *L = &g_o[l];
        uint64_t extra[8] = {0};
        if (L->snap_valid) memcpy(extra, L->snap_fetched, sizeof(extra));
        uint32_t ids[16];
        uint8_t hit[16];
        for (int i = 0; i < k; ++i) ids[i] = (uint32_t)eids[i];
        n_miss = step_core(L, ids, k, out_slots, miss_eids, miss_slots, extra, hit);
        if ((flags & 4) && n_miss > 0 && n_miss < k) {
            int h = 0, m = 0, n_hit = k - n_miss;
            for (int i = 0; i < k; ++i) {
                if (hit[i]) { g_hit_slots[l][h] = out_slots[i]; g_inv[l][i] = h++; }
                else { g_miss_slots[l][m] = out_slots[i]; g_inv[l][i] = n_hit + m++; }
            }
            g_n_hit[l] = n_hit;
            g_n_miss[l] = n_miss;
            g_split_k[l] = k;
        }
    }
    if (!(flags & 2) && next > 0 && next < O_MAX_LAYERS && pred && n_pred > 0 && prefetch_cap > 0)
        *n_fetch = prefetch_core(&g_o[next], pred, n_pred, prefetch_cap, 1, fetch_eids, fetch_slots);
    return n_miss;
}

/* Counts (n_hit, n_miss, k) of the stored split; lists copied when the pointers are non-null. */
void o_layer_get_split_inds(int l, uint32_t *hit, uint32_t *miss, int32_t *inv, int *counts3) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    if (hit && g_n_hit[l] > 0) memcpy(hit, g_hit_slots[l], (size_t)g_n_hit[l] * sizeof(uint32_t));
    if (miss && g_n_miss[l] > 0) memcpy(miss, g_miss_slots[l], (size_t)g_n_miss[l] * sizeof(uint32_t));
    if (inv && g_split_k[l] > 0) memcpy(inv, g_inv[l], (size_t)g_split_k[l] * sizeof(int32_t));
    if (counts3) { counts3[0] = g_n_hit[l]; counts3[1] = g_n_miss[l]; counts3[2] = g_split_k[l]; }
}

void o_set_io_accounting(int on) {
    g_acct_on = on ? 1 : 0;
    if (!g_acct_on) g_cur_token = -1;
}

void o_begin_decode_token(void) {
    g_cur_token = g_token_seq++;
    memset(g_tok, 0, sizeof(g_tok));
}

void o_end_decode_token(uint64_t *out10) { memcpy(out10, g_tok, sizeof(g_tok)); }

void o_layer_load_sync(int l, const int32_t *eids, const int32_t *slots, int n, int is_prefill) {
    (void)slots;
    if (l < 0 || l >= O_MAX_LAYERS || n <= 0) return;
    OLayer *L = &g_o[l];
    if (is_prefill) L->st[9] += (uint64_t)n * L->expert_bytes;
    if (g_acct_on) g_tok[A_BYTES] += (uint64_t)n * L->staged_bytes;
    count_runs(L, eids, n);
}

void o_layer_get_lru_state(int l, int32_t *eids, int32_t *slots, int *count) {
    if (l < 0 || l >= O_MAX_LAYERS) { *count = 0; return; }
    OLayer *L = &g_o[l];
    int c = 0;
    for (int s = L->lru_end; s >= 0; s = L->newer[s]) { eids[c] = L->eid_of[s]; slots[c] = s; ++c; }
    *count = c;
}

void o_layer_set_lru_state(int l, const int32_t *eids, const int32_t *slots, int n,
                           uint64_t add_req, uint64_t add_hits, uint64_t add_miss) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    OLayer *L = &g_o[l];
    L->st[6] += add_req; L->st[7] += add_hits; L->st[8] += add_miss;
    for (int i = 0; i < O_NUM_EXPERTS; ++i) L->slot_of[i] = L->eid_of[i] = L->older[i] = L->newer[i] = -1;
    L->lru_end = L->mru_end = -1;
    L->snap_valid = 0;
    uint8_t used[O_NUM_EXPERTS] = {0};
    for (int i = 0; i < n; ++i) {
        used[slots[i]] = 1;
        if (eids[i] >= 0 && eids[i] < O_NUM_EXPERTS) L->evicted_at[eids[i]] = -1;
        bind(L, eids[i], slots[i]);
    }
    L->n_free = 0;
    for (int s = L->capacity - 1; s >= 0; --s) if (!used[s]) L->free_stack[L->n_free++] = (int16_t)s;
}

void o_layer_get_stats(int l, uint64_t *out) {
    if (l < 0 || l >= O_MAX_LAYERS) return;
    memcpy(out, g_o[l].st, sizeof(g_o[l].st));
}

void o_get_decode_totals(int num_layers, uint64_t *out6) {
    uint64_t t[6] = {0};
    if (num_layers > O_MAX_LAYERS) num_layers = O_MAX_LAYERS;
    for (int l = 1; l < num_layers; ++l) {
        const uint64_t *st = g_o[l].st;
        t[0] += st[1]; t[1] += st[2]; t[2] += st[3]; t[3] += st[0]; t[4] += st[4]; t[5] += st[5];
    }
    memcpy(out6, t, sizeof(t));
}
