// C++ face of the P1 I/O scheduler: the class of mlx-qwen38/cpp/src/io_sched.h:46-245
// (`qwen38::P1IoScheduler`, `qwen38::P1LayerStats`) with the same method names, arguments and
// meaning, over the moe_p1_* C-ABI of libmoe_offload.so.  A runner that used the reference class
// switches by including this header and naming `moe::` instead of `qwen38::`.
//
// Additions: set_compute_stream / mark_read (the stream that orders slot-id writes to device
// memory, and the event that ends a layer's GPU reader; without a reader callback an allocation
// that meets pinned slots waits for that event and unpins the layer itself).
#pragma once
#include <cstdint>
#include <functional>
#include <random>

#include "moe_offload.h"

namespace moe {

constexpr int kP1MaxLayers = 64;
constexpr int kP1NumExperts = 512;
constexpr int kP1MaxTensors = 9;
constexpr uint64_t kP1DefaultExpertBytes = 1536000ULL;

// io_sched.h:23-44, same fields in the same order.
struct P1LayerStats {
    uint64_t decode_requests = 0;
    uint64_t lru_hits = 0;
    uint64_t urgent_reads = 0;
    uint64_t prefetch_issued = 0;
    uint64_t prefetch_cancelled = 0;
    uint64_t prefetch_promoted = 0;
    uint64_t prefetch_used = 0;
    uint64_t prefetch_wasted = 0;
    uint64_t pin_waits = 0;
    uint64_t bytes = 0;
    uint64_t io_wait_ns = 0;
    uint64_t forced_invalidations = 0;
    uint64_t prefill_requests = 0;
    uint64_t prefill_lru_hits = 0;
    uint64_t prefill_demand_misses = 0;
    uint64_t prefill_demand_bytes = 0;

    double io_wait_ms() const { return static_cast<double>(io_wait_ns) / 1e6; }

    static P1LayerStats from(const uint64_t* v) {
        P1LayerStats s;
        uint64_t* f[16] = {&s.decode_requests, &s.lru_hits, &s.urgent_reads, &s.prefetch_issued,
                           &s.prefetch_cancelled, &s.prefetch_promoted, &s.prefetch_used, &s.prefetch_wasted,
                           &s.pin_waits, &s.bytes, &s.io_wait_ns, &s.forced_invalidations, &s.prefill_requests,
                           &s.prefill_lru_hits, &s.prefill_demand_misses, &s.prefill_demand_bytes};
        for (int i = 0; i < 16; ++i) *f[i] = v[i];
        return s;
    }
};

class P1IoScheduler {
public:
    P1IoScheduler() : h_(moe_p1_create()) {}
    ~P1IoScheduler() { moe_p1_destroy(h_); }
    P1IoScheduler(const P1IoScheduler&) = delete;
    P1IoScheduler& operator=(const P1IoScheduler&) = delete;

    void init(int num_threads = 6) { moe_p1_init(h_, num_threads); }
    void shutdown() { moe_p1_shutdown(h_); }

    void set_wait_reader_callback(std::function<void(int)> cb) {
        cb_ = std::move(cb);
        if (cb_) moe_p1_set_wait_reader_callback(h_, &P1IoScheduler::reader_thunk, this);
        else moe_p1_set_wait_reader_callback(h_, nullptr, nullptr);
    }
    void set_compute_stream(void* stream) { moe_p1_set_compute_stream(h_, stream); }
    int mark_read(int layer_idx, void* stream) { return moe_p1_mark_read(h_, layer_idx, stream); }

    void layer_init(int layer_idx, int fd, int capacity, int num_tensors, const uint64_t* base_offsets,
                    const uint64_t* row_bytes, const uint64_t* base_ptrs, uint64_t slot_inds_ptr) {
        moe_p1_layer_init(h_, layer_idx, fd, capacity, num_tensors, base_offsets, row_bytes, base_ptrs, slot_inds_ptr);
    }
    void resize_layer(int layer_idx, int new_capacity, const uint64_t* new_base_ptrs, uint64_t slot_inds_ptr,
                      const int32_t* ordered_eids, const int32_t* ordered_slots, int count) {
        moe_p1_resize_layer(h_, layer_idx, new_capacity, new_base_ptrs, slot_inds_ptr, ordered_eids, ordered_slots,
                            count);
    }
    void reset_cache(int layer_idx) { moe_p1_reset_cache(h_, layer_idx); }
    void reset_stats(int layer_idx) { moe_p1_reset_stats(h_, layer_idx); }
    void start_prefetch(int layer_idx, const int32_t* pred_eids, int pred_count, int max_fetch) {
        moe_p1_start_prefetch(h_, layer_idx, pred_eids, pred_count, max_fetch);
    }
    int step_decode(int layer_idx, const uint32_t* eids, int k, uint32_t* out_slots = nullptr) {
        return moe_p1_step_decode(h_, layer_idx, eids, k, out_slots);
    }
    void wait_layer_urgent(int layer_idx) { moe_p1_wait_layer_urgent(h_, layer_idx); }
    void wait_layer_all(int layer_idx) { moe_p1_wait_layer_all(h_, layer_idx); }
    void wait_all() { moe_p1_wait_all(h_); }
    void unpin_layer_slots(int layer_idx) { moe_p1_unpin_layer_slots(h_, layer_idx); }
    void pin_slots(int layer_idx, const uint32_t* slots, int count) { moe_p1_pin_slots(h_, layer_idx, slots, count); }
    void unpin_slots(int layer_idx, const uint32_t* slots, int count) {
        moe_p1_unpin_slots(h_, layer_idx, slots, count);
    }
    int get_slot_pin_count(int layer_idx, int slot) { return moe_p1_get_slot_pin_count(h_, layer_idx, slot); }
    int force_invalidate(int layer_idx, double rate, std::mt19937_64& rng) {
        return moe_p1_force_invalidate(h_, layer_idx, rate, &P1IoScheduler::draw_thunk, &rng);
    }
    void load_sync(int layer_idx, const int32_t* eids, const int32_t* slots, int count, bool is_prefill) {
        moe_p1_load_sync(h_, layer_idx, eids, slots, count, is_prefill ? 1 : 0);
    }
    void get_lru_state(int layer_idx, int32_t* out_eids, int32_t* out_slots, int* out_count) {
        moe_p1_get_lru_state(h_, layer_idx, out_eids, out_slots, out_count);
    }
    void set_lru_state(int layer_idx, const int32_t* ordered_eids, const int32_t* ordered_slots, int count,
                       uint64_t add_prefill_requests, uint64_t add_prefill_hits, uint64_t add_prefill_misses) {
        moe_p1_set_lru_state(h_, layer_idx, ordered_eids, ordered_slots, count, add_prefill_requests, add_prefill_hits,
                             add_prefill_misses);
    }
    P1LayerStats get_layer_stats(int layer_idx) const {
        uint64_t v[16];
        moe_p1_get_layer_stats(h_, layer_idx, v);
        return P1LayerStats::from(v);
    }
    P1LayerStats get_total_stats(int num_layers = 48) const {
        uint64_t v[16];
        moe_p1_get_total_stats(h_, num_layers, v);
        return P1LayerStats::from(v);
    }
    int num_threads() const { return moe_p1_num_threads(h_); }

private:
    static void reader_thunk(int layer_idx, void* self) {
        auto* s = static_cast<P1IoScheduler*>(self);
        if (s->cb_) s->cb_(layer_idx);
    }
    static double draw_thunk(void* rng) {
        std::uniform_real_distribution<double> d(0.0, 1.0);
        return d(*static_cast<std::mt19937_64*>(rng));
    }

    moe_p1* h_;
    std::function<void(int)> cb_;
};

}  // namespace moe
