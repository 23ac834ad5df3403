// C entry points over the reference's P1IoScheduler (mlx-qwen38/cpp/src/io_sched.{h,cpp}), built
// together with the reference's own io_sched.cpp into _ref/libp1_ref.so by oracle/Makefile.  Test
// infrastructure only: the golden-trace generator (tests/golden/make_p1_traces.py) drives it.
//
// threads <= 0 gives the scheduler without reader threads: init(1) then shutdown() stops its one
// worker, after which queued reads run only inside the waits that execute them themselves
// (io_sched.cpp:787-815,827-848,414-423) -- the deterministic form the traces record.
#include <cstdint>
#include <random>

#include "io_sched.h"

using qwen38::P1IoScheduler;
using qwen38::P1LayerStats;

namespace {
P1IoScheduler* S(void* p) { return static_cast<P1IoScheduler*>(p); }

void put_stats(const P1LayerStats& s, uint64_t* out) {
    const uint64_t v[16] = {s.decode_requests, s.lru_hits, s.urgent_reads, s.prefetch_issued,
                            s.prefetch_cancelled, s.prefetch_promoted, s.prefetch_used, s.prefetch_wasted,
                            s.pin_waits, s.bytes, s.io_wait_ns, s.forced_invalidations, s.prefill_requests,
                            s.prefill_lru_hits, s.prefill_demand_misses, s.prefill_demand_bytes};
    for (int i = 0; i < 16; ++i) out[i] = v[i];
}
}  // namespace

extern "C" {

void* r_p1_new(int threads) {
    auto* s = new P1IoScheduler();
    s->init(threads > 0 ? threads : 1);
    if (threads <= 0) s->shutdown();
    return s;
}
void r_p1_free(void* p) { delete S(p); }
void r_p1_set_unpin_cb(void* p) {
    P1IoScheduler* s = S(p);
    s->set_wait_reader_callback([s](int l) { s->unpin_layer_slots(l); });
}
void r_p1_layer_init(void* p, int l, int fd, int cap, int nt, const uint64_t* offs, const uint64_t* rb,
                     const uint64_t* ptrs, uint64_t slot_inds) {
    S(p)->layer_init(l, fd, cap, nt, offs, rb, ptrs, slot_inds);
}
void r_p1_resize(void* p, int l, int cap, const uint64_t* ptrs, uint64_t slot_inds, const int32_t* e,
                 const int32_t* s, int n) {
    S(p)->resize_layer(l, cap, ptrs, slot_inds, e, s, n);
}
void r_p1_reset_cache(void* p, int l) { S(p)->reset_cache(l); }
void r_p1_reset_stats(void* p, int l) { S(p)->reset_stats(l); }
void r_p1_start_prefetch(void* p, int l, const int32_t* preds, int n, int maxf) {
    S(p)->start_prefetch(l, preds, n, maxf);
}
int r_p1_step_decode(void* p, int l, const uint32_t* e, int k, uint32_t* out) { return S(p)->step_decode(l, e, k, out); }
void r_p1_wait_urgent(void* p, int l) { S(p)->wait_layer_urgent(l); }
void r_p1_wait_layer_all(void* p, int l) { S(p)->wait_layer_all(l); }
void r_p1_wait_all(void* p) { S(p)->wait_all(); }
void r_p1_unpin_layer(void* p, int l) { S(p)->unpin_layer_slots(l); }
void r_p1_pin(void* p, int l, const uint32_t* s, int n) { S(p)->pin_slots(l, s, n); }
void r_p1_unpin(void* p, int l, const uint32_t* s, int n) { S(p)->unpin_slots(l, s, n); }
int r_p1_pin_count(void* p, int l, int s) { return S(p)->get_slot_pin_count(l, s); }
void* r_mt64_new(uint64_t seed) { return new std::mt19937_64(seed); }
void r_mt64_free(void* g) { delete static_cast<std::mt19937_64*>(g); }
uint64_t r_mt64_next(void* g) { return (*static_cast<std::mt19937_64*>(g))(); }
double r_mt64_uniform(void* g) {
    std::uniform_real_distribution<double> d(0.0, 1.0);
    return d(*static_cast<std::mt19937_64*>(g));
}
int r_p1_force_invalidate(void* p, int l, double rate, void* g) {
    return S(p)->force_invalidate(l, rate, *static_cast<std::mt19937_64*>(g));
}
void r_p1_load_sync(void* p, int l, const int32_t* e, const int32_t* s, int n, int prefill) {
    S(p)->load_sync(l, e, s, n, prefill != 0);
}
void r_p1_get_lru(void* p, int l, int32_t* e, int32_t* s, int* n) { S(p)->get_lru_state(l, e, s, n); }
void r_p1_set_lru(void* p, int l, const int32_t* e, const int32_t* s, int n, uint64_t a, uint64_t b, uint64_t c) {
    S(p)->set_lru_state(l, e, s, n, a, b, c);
}
void r_p1_stats(void* p, int l, uint64_t* out) { put_stats(S(p)->get_layer_stats(l), out); }
void r_p1_total(void* p, int n, uint64_t* out) { put_stats(S(p)->get_total_stats(n), out); }

}  // extern "C"
