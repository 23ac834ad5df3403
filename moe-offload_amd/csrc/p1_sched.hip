// P1 I/O scheduler of the on-disk tier (host code), the C++ runner's `--io p1` path
// (mlx-qwen38/cpp/src/io_sched.h:46-245, io_sched.cpp).
//
// What it decides is the reference's, call for call: which slot a miss or a prefetch gets (the
// least recently used one that is neither protected by the call's experts, nor pinned by a GPU
// reader, nor still being read), when a queued prefetch is cancelled (its slot given back to the
// expert it displaced) or promoted to the urgent queue, which reads are coalesced (consecutive
// experts of one tensor, at most 16), in what order the readers take them (urgent before prefetch,
// weight tensors before scale/bias tensors), and every counter.  tests/test_p1_sched.py replays
// traces written by the reference's own io_sched.cpp compiled from source.
//
// How it is kept differs:
//  * recency is a per-slot stamp (head insertions count down, tail insertions count up) instead of
//    a linked list; the victim is the smallest stamp among eligible slots;
//  * slot pools may be HBM: a read then lands in a pinned staging buffer of the reader and goes to
//    the slot rows by DMA on the reader's own stream, and the read counts as done once the copy
//    has completed, so a GPU kernel launched after wait_layer_urgent sees the bytes.  Host-memory
//    pools (the reference's unified memory) are read into directly;
//  * slot ids go to device memory by a copy ordered on the compute stream;
//  * 0 reader threads is a real mode (the reference clamps to 1): reads then run inside the waits,
//    which drain the prefetch queue as well when the urgent one is empty;
//  * the reader wait: without a callback, an allocation that meets pinned slots waits for the
//    layer's GPU reader (the event of moe_p1_mark_read) and unpins the layer's slots itself;
//  * failures are reported (c_last_error) instead of ignored.
#include <errno.h>
#include <string.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

#include "moe_common.h"
#include "moe_offload.h"

namespace {

constexpr int kLayers = 64;
constexpr int kExperts = 512;
constexpr int kTensors = 9;
constexpr int kMaxRun = 16;
constexpr uint64_t kDefaultExpertBytes = 1536000;   // io_sched.h:21
constexpr uint64_t kLargeRow = 100000;               // weight tensors are read before scales/biases
constexpr int64_t kOut = INT64_MIN;                  // stamp of a slot that is not on the list

enum Stat {
    S_DECODE_REQ, S_LRU_HITS, S_URGENT, S_PF_ISSUED, S_PF_CANCELLED, S_PF_PROMOTED, S_PF_USED, S_PF_WASTED,
    S_PIN_WAITS, S_BYTES, S_IO_WAIT_NS, S_FORCED, S_PRE_REQ, S_PRE_HITS, S_PRE_MISSES, S_PRE_BYTES, S_COUNT
};

struct ReadOp {
    int layer = 0;
    int32_t eid = -1;
    int16_t slot = -1, prev_eid = -1;
    bool prefetch = false, promoted = false, cancelled = false, resolved = false, done = false;
    int started = 0, completed = 0, total = 0;
};
using OpRef = std::shared_ptr<ReadOp>;

// One read: n consecutive experts of one tensor, each to its slot row.
struct Task {
    int layer = 0, tensor = 0, n = 0;
    bool prefill = false;
    OpRef ops[kMaxRun];
};

// Pinned staging buffer + stream for reads into HBM pools.
struct Stage {
    uint8_t* buf = nullptr;
    size_t cap = 0;
    hipStream_t stream = nullptr;
    int dev = -1;
};

struct Layer {
    bool init = false;
    int fd = -1, cap = 0, nt = kTensors;
    uint64_t off[kTensors] = {}, rb[kTensors] = {};
    uint8_t* dst[kTensors] = {};
    bool dst_device = false;
    int dev = 0;
    uint32_t* slot_inds = nullptr;
    bool slot_inds_device = false;
    uint64_t expert_bytes = kDefaultExpertBytes;
    int16_t slot_of[kExperts], eid_of[kExperts];
    int64_t stamp[kExperts];
    int64_t hi = 0, lo = 1;
    std::vector<int16_t> free_stack;
    int pins[kExperts] = {};
    std::vector<int16_t> gpu_pinned;
    OpRef active[kExperts];
    bool has_snap = false;
    uint64_t snap[kExperts / 64] = {};
    std::vector<OpRef> last_pf, pending;
    uint64_t st[S_COUNT] = {};
    std::atomic<uint64_t> bytes{0};
    hipEvent_t read_ev = nullptr;                     // the layer's GPU reader (moe_p1_mark_read)
    bool read_rec = false;
};

bool device_ptr(const void* p, int* dev) {
    if (!p) return false;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (a.type != hipMemoryTypeDevice) return false;
    if (dev) *dev = a.device;
    return true;
}

// Read len bytes at off fully into buf (short reads continued); bytes read, -1 on error.
int64_t read_full(int fd, uint8_t* buf, uint64_t len, uint64_t off) {
    uint64_t got = 0;
    while (got < len) {
        const ssize_t r = pread(fd, buf + got, len - got, (off_t)(off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return r < 0 ? -1 : (int64_t)got;
        got += (uint64_t)r;
    }
    return (int64_t)got;
}

}  // namespace

struct moe_p1 {
    std::mutex mu;
    std::condition_variable work_cv, done_cv;
    std::deque<Task> urgent, prefetchq;
    Layer L[kLayers];
    std::vector<std::thread> workers;
    int nthreads = 6;
    bool ready = false, stopping = false;
    moe_p1_reader_fn reader_fn = nullptr;
    void* reader_user = nullptr;
    hipStream_t compute = nullptr;
    std::mutex stage_mu;
    std::vector<Stage*> stages_free;
    std::vector<Stage*> stages_all;

    moe_p1() {
        for (int l = 0; l < kLayers; ++l) clear_table(L[l], true);
    }
    ~moe_p1() {
        shutdown();
        std::lock_guard<std::mutex> g(stage_mu);
        for (Stage* s : stages_all) {
            if (s->stream) (void)hipStreamDestroy(s->stream);
            if (s->buf) (void)hipHostFree(s->buf);
            delete s;
        }
        for (Layer& x : L)
            if (x.read_ev) (void)hipEventDestroy(x.read_ev);
    }

    // ---- recency list as stamps ----------------------------------------------------------------
    static void clear_table(Layer& x, bool pins) {
        for (int i = 0; i < kExperts; ++i) {
            x.slot_of[i] = -1;
            x.eid_of[i] = -1;
            x.stamp[i] = kOut;
            x.active[i].reset();
            if (pins) x.pins[i] = 0;
        }
        if (pins) x.gpu_pinned.clear();
        x.hi = 0;
        x.lo = 1;
    }
    static void unlink(Layer& x, int s) { x.stamp[s] = kOut; }
    static void to_tail(Layer& x, int s) { x.stamp[s] = ++x.hi; }
    static void to_head(Layer& x, int32_t e, int s) {
        x.slot_of[e] = (int16_t)s;
        x.eid_of[s] = (int16_t)e;
        x.stamp[s] = --x.lo;
    }
    static void insert(Layer& x, int32_t e, int s) {
        if (x.slot_of[e] >= 0) {                       // already resident: refreshed only
            to_tail(x, x.slot_of[e]);
            return;
        }
        x.slot_of[e] = (int16_t)s;
        x.eid_of[s] = (int16_t)e;
        to_tail(x, s);
    }
    static int16_t evict(Layer& x, int s) {
        const int16_t e = x.eid_of[s];
        unlink(x, s);
        if (e >= 0) x.slot_of[e] = -1;
        x.eid_of[s] = -1;
        x.active[s].reset();
        return e;
    }
    // Slots on the list, least recently used first.
    static std::vector<int16_t> ordered(const Layer& x) {
        std::vector<int16_t> v;
        for (int s = 0; s < kExperts; ++s)
            if (x.stamp[s] != kOut) v.push_back((int16_t)s);
        std::sort(v.begin(), v.end(), [&](int16_t a, int16_t b) { return x.stamp[a] < x.stamp[b]; });
        return v;
    }
    static bool busy(const Layer& x, int s) { return x.active[s] && !x.active[s]->done; }
    static void rebuild(Layer& x, const int32_t* eids, const int32_t* slots, int n) {
        bool used[kExperts] = {};
        for (int i = 0; i < n; ++i) {
            const int32_t e = eids[i], s = slots[i];
            if (s >= 0 && s < x.cap && e >= 0 && e < kExperts) {
                used[s] = true;
                insert(x, e, s);
            }
        }
        x.free_stack.clear();
        for (int s = x.cap - 1; s >= 0; --s)
            if (!used[s]) x.free_stack.push_back((int16_t)s);
    }

    // ---- readers ---------------------------------------------------------------------------------
    void init(int n) {
        std::unique_lock<std::mutex> lk(mu);
        if (ready) return;
        nthreads = std::min(std::max(n, 0), 32);
        stopping = false;
        urgent.clear();
        prefetchq.clear();
        for (int i = 0; i < nthreads; ++i) workers.emplace_back([this] { worker(); });
        ready = true;
    }
    void shutdown() {
        std::vector<std::thread> ts;
        {
            std::lock_guard<std::mutex> g(mu);
            if (!ready) return;
            stopping = true;
            work_cv.notify_all();
            done_cv.notify_all();
            ts.swap(workers);
            ready = false;
        }
        for (auto& t : ts) t.join();
    }

    // The next read: urgent first (a read whose experts were all cancelled is dropped), then
    // prefetch (a cancelled or promoted prefetch is dropped).
    bool pop(Task& t, bool urgent_only = false) {
        while (!urgent.empty()) {
            t = std::move(urgent.front());
            urgent.pop_front();
            bool live = false;
            for (int i = 0; i < t.n; ++i)
                if (t.ops[i] && !t.ops[i]->cancelled) {
                    t.ops[i]->started++;
                    live = true;
                }
            if (live) return true;
        }
        if (urgent_only) return false;
        while (!prefetchq.empty()) {
            t = std::move(prefetchq.front());
            prefetchq.pop_front();
            const OpRef& op = t.ops[0];
            if (!op || op->cancelled || op->promoted) continue;
            op->started++;
            return true;
        }
        return false;
    }

    Stage* get_stage(int dev, size_t need) {
        Stage* s = nullptr;
        {
            std::lock_guard<std::mutex> g(stage_mu);
            for (size_t i = 0; i < stages_free.size(); ++i)
                if (stages_free[i]->dev == dev) {
                    s = stages_free[i];
                    stages_free.erase(stages_free.begin() + i);
                    break;
                }
        }
        if (hipSetDevice(dev) != hipSuccess) return nullptr;
        if (!s) {
            s = new Stage();
            s->dev = dev;
            if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) {
                delete s;
                return nullptr;
            }
            std::lock_guard<std::mutex> g(stage_mu);
            stages_all.push_back(s);
        }
        if (s->cap < need) {
            if (s->buf) (void)hipHostFree(s->buf);
            s->buf = nullptr;
            s->cap = 0;
            if (hipHostMalloc((void**)&s->buf, need, hipHostMallocDefault) != hipSuccess) {
                put_stage(s);
                return nullptr;
            }
            s->cap = need;
        }
        return s;
    }
    void put_stage(Stage* s) {
        std::lock_guard<std::mutex> g(stage_mu);
        stages_free.push_back(s);
    }

    // Execute one read (without the lock): file -> slot rows; then mark its experts' progress.
    void run(Task& t) {
        Layer& x = L[t.layer];
        const uint64_t rb = x.rb[t.tensor];
        const uint64_t off = x.off[t.tensor] + (uint64_t)t.ops[0]->eid * rb, len = (uint64_t)t.n * rb;
        int64_t got = -1;
        if (!x.dst_device) {
            struct iovec iov[kMaxRun];
            for (int i = 0; i < t.n; ++i) {
                iov[i].iov_base = x.dst[t.tensor] + (uint64_t)t.ops[i]->slot * rb;
                iov[i].iov_len = rb;
            }
            got = 0;
            int first = 0;
            uint64_t skip = 0;
            while (first < t.n) {                    // preadv, continued after a short read
                struct iovec cur[kMaxRun];
                int m = 0;
                for (int i = first; i < t.n; ++i, ++m) cur[m] = iov[i];
                cur[0].iov_base = (uint8_t*)cur[0].iov_base + skip;
                cur[0].iov_len -= skip;
                const ssize_t r = preadv(x.fd, cur, m, (off_t)(off + (uint64_t)got));
                if (r < 0 && errno == EINTR) continue;
                if (r <= 0) break;
                got += r;
                uint64_t adv = (uint64_t)r + skip;
                while (first < t.n && adv >= rb) {
                    adv -= rb;
                    ++first;
                }
                skip = adv;
            }
        } else {
            int cur_dev = 0;
            (void)hipGetDevice(&cur_dev);
            Stage* s = get_stage(x.dev, len);
            if (s) {
                got = read_full(x.fd, s->buf, len, off);
                if (got == (int64_t)len) {
                    bool ok = true;
                    for (int i = 0; i < t.n && ok; ++i)
                        ok = hipMemcpyAsync(x.dst[t.tensor] + (uint64_t)t.ops[i]->slot * rb, s->buf + (uint64_t)i * rb,
                                            rb, hipMemcpyHostToDevice, s->stream) == hipSuccess;
                    ok = ok && hipStreamSynchronize(s->stream) == hipSuccess;
                    if (!ok) {
                        moe_set_error("p1: copy to the slot pool of layer %d failed", t.layer);
                        got = -1;
                    }
                }
                put_stage(s);
            } else {
                moe_set_error("p1: no staging buffer of %llu bytes", (unsigned long long)len);
            }
            (void)hipSetDevice(cur_dev);                // the calling thread's device is left as it was
        }
        if (got != (int64_t)len)
            moe_set_error("p1: read of layer %d tensor %d at %llu: %lld of %llu bytes", t.layer, t.tensor,
                          (unsigned long long)off, (long long)got, (unsigned long long)len);
        if (!t.prefill && got > 0) x.bytes.fetch_add((uint64_t)got, std::memory_order_relaxed);
        std::lock_guard<std::mutex> g(mu);
        bool any = false;
        for (int i = 0; i < t.n; ++i) {
            ReadOp& op = *t.ops[i];
            if (++op.completed >= op.total) {
                op.done = true;
                any = true;
            }
        }
        if (any) done_cv.notify_all();
    }

    void worker() {
        for (;;) {
            Task t;
            {
                std::unique_lock<std::mutex> lk(mu);
                bool have = false;
                while (!stopping && !(have = pop(t))) work_cv.wait(lk);
                if (!have) return;
            }
            run(t);
        }
    }

    // Run one queued read on this thread (the lock is released meanwhile), or wait for one to end.
    // Without reader threads (0 asked for, or not started) any queue is drained here; false:
    // nothing is queued and no reader thread runs, so nothing can change by waiting.
    bool help_or_wait(std::unique_lock<std::mutex>& lk, bool urgent_only) {
        Task t;
        if (pop(t, urgent_only) || (workers.empty() && pop(t))) {
            lk.unlock();
            run(t);
            lk.lock();
            return true;
        }
        if (workers.empty()) return false;
        done_cv.wait_for(lk, std::chrono::milliseconds(50));
        return true;
    }

    // ---- queueing ----------------------------------------------------------------------------
    template <class F>
    void for_tensors(const Layer& x, F f) {          // weight tensors first, then the small ones
        for (int pass = 0; pass < 2; ++pass)
            for (int t = 0; t < x.nt; ++t)
                if ((x.rb[t] > kLargeRow) == (pass == 0)) f(t);
    }
    void queue_prefetch(int layer, Layer& x, const OpRef& op) {
        for_tensors(x, [&](int t) {
            Task k;
            k.layer = layer;
            k.tensor = t;
            k.n = 1;
            k.ops[0] = op;
            prefetchq.push_back(std::move(k));
        });
    }
    void queue_urgent(int layer, Layer& x, std::vector<OpRef> ops, bool prefill) {
        if (ops.empty()) return;
        std::sort(ops.begin(), ops.end(), [](const OpRef& a, const OpRef& b) { return a->eid < b->eid; });
        std::vector<std::pair<size_t, size_t>> runs;
        size_t start = 0;
        for (size_t i = 1; i <= ops.size(); ++i)
            if (i == ops.size() || ops[i]->eid != ops[i - 1]->eid + 1 || i - start >= (size_t)kMaxRun) {
                runs.emplace_back(start, i - start);
                start = i;
            }
        for_tensors(x, [&](int t) {
            for (const auto& r : runs) {
                Task k;
                k.layer = layer;
                k.tensor = t;
                k.n = (int)r.second;
                k.prefill = prefill;
                for (size_t i = 0; i < r.second; ++i) k.ops[i] = ops[r.first + i];
                urgent.push_back(std::move(k));
            }
        });
    }

    // ---- slot allocation ---------------------------------------------------------------------
    // A free slot, else the least recently used slot that is not protected, pinned or being
    // read.  Pinned candidates wait for the layer's GPU reader; in-flight reads are helped along.
    // -1 (with an error) when nothing can free a slot.
    int alloc(int layer, std::unique_lock<std::mutex>& lk, const uint64_t* protect, int16_t* prev) {
        Layer& x = L[layer];
        *prev = -1;
        if (!x.free_stack.empty()) {
            const int s = x.free_stack.back();
            x.free_stack.pop_back();
            return s;
        }
        bool counted = false;
        for (;;) {
            int best = -1, any_free = -1;
            bool saw_pin = false, saw_io = false, saw_pin_all = false, saw_io_all = false;
            for (int s = 0; s < kExperts; ++s) {
                if (x.stamp[s] == kOut) continue;
                const int e = x.eid_of[s];
                const bool prot = e >= 0 && ((protect[e >> 6] >> (e & 63)) & 1);
                const bool pinned = x.pins[s] > 0, io = busy(x, s);
                saw_pin_all |= pinned;
                saw_io_all |= io;
                if (!pinned && !io && (any_free < 0 || x.stamp[s] < x.stamp[any_free])) any_free = s;
                if (prot) continue;
                saw_pin |= pinned;
                saw_io |= io;
                if (!pinned && !io && (best < 0 || x.stamp[s] < x.stamp[best])) best = s;
            }
            if (best >= 0) {
                *prev = evict(x, best);
                return best;
            }
            if (!saw_pin && !saw_io) {
                saw_pin = saw_pin_all;
                saw_io = saw_io_all;
            }
            if (saw_pin) {
                if (!counted) {
                    x.st[S_PIN_WAITS]++;
                    counted = true;
                }
                int before[kExperts];
                memcpy(before, x.pins, sizeof(before));
                lk.unlock();
                wait_reader(layer);
                lk.lock();
                if (!memcmp(before, x.pins, sizeof(before))) {
                    if (workers.empty() && reader_fn == nullptr) {
                        moe_set_error("p1: layer %d: every candidate slot is pinned and nothing unpins it", layer);
                        return -1;
                    }
                    done_cv.wait_for(lk, std::chrono::milliseconds(1));
                }
                continue;
            }
            if (saw_io) {
                if (!help_or_wait(lk, false)) {
                    moe_set_error("p1: layer %d: slots busy with reads that cannot finish", layer);
                    return -1;
                }
                continue;
            }
            if (any_free >= 0) {
                *prev = evict(x, any_free);
                return any_free;
            }
            moe_set_error("p1: layer %d has no slot to give", layer);
            return -1;
        }
    }

    // The layer's GPU reader has finished with its slots: the callback, or the reader event + unpin.
    void wait_reader(int layer) {
        if (reader_fn) {
            reader_fn(layer, reader_user);
            return;
        }
        Layer& x = L[layer];
        if (x.read_rec && x.read_ev) {
            if (hipEventSynchronize(x.read_ev) != hipSuccess) (void)hipGetLastError();
            x.read_rec = false;
        }
        unpin_layer(layer);
    }

    void unpin_layer(int layer) {
        std::lock_guard<std::mutex> g(mu);
        Layer& x = L[layer];
        if (x.gpu_pinned.empty()) return;
        for (int16_t s : x.gpu_pinned)
            if (s >= 0 && s < kExperts && x.pins[s] > 0) x.pins[s]--;
        x.gpu_pinned.clear();
        done_cv.notify_all();
    }

    // An unstarted prefetch dropped: its slot returns to the expert it displaced (whose bytes
    // are still there: nothing was read) or to the free stack.
    void cancel(Layer& x, ReadOp& op, bool mark_snapshot) {
        op.cancelled = true;
        x.st[S_PF_CANCELLED]++;
        if (x.eid_of[op.slot] != op.eid) return;
        unlink(x, op.slot);
        x.slot_of[op.eid] = -1;
        x.eid_of[op.slot] = -1;
        x.active[op.slot].reset();
        if (op.prev_eid >= 0 && op.prev_eid < kExperts && x.slot_of[op.prev_eid] < 0) {
            to_head(x, op.prev_eid, op.slot);
            if (mark_snapshot) x.snap[op.prev_eid >> 6] |= 1ull << (op.prev_eid & 63);
        } else {
            x.free_stack.push_back(op.slot);
        }
    }

    // ---- API ---------------------------------------------------------------------------------
    void layer_init(int l, int fd, int cap, int nt, const uint64_t* offs, const uint64_t* rbs, const uint64_t* ptrs,
                    uint64_t slot_inds) {
        if (l < 0 || l >= kLayers) return;
        wait_layer_all(l);
        std::lock_guard<std::mutex> g(mu);
        Layer& x = L[l];
        x.init = true;
        x.fd = fd;
        x.cap = std::min(std::max(cap, 1), kExperts);
        x.nt = std::min(std::max(nt, 1), kTensors);
        uint64_t sum = 0;
        for (int t = 0; t < x.nt; ++t) {
            x.off[t] = offs ? offs[t] : 0;
            x.rb[t] = rbs ? rbs[t] : 0;
            x.dst[t] = ptrs ? reinterpret_cast<uint8_t*>(ptrs[t]) : nullptr;
            sum += x.rb[t];
        }
        x.expert_bytes = sum ? sum : kDefaultExpertBytes;
        x.dst_device = device_ptr(x.dst[0], &x.dev);
        x.slot_inds = reinterpret_cast<uint32_t*>(slot_inds);
        x.slot_inds_device = device_ptr(x.slot_inds, nullptr);
        clear_table(x, true);
        x.free_stack.clear();
        for (int i = 0; i < x.cap; ++i) x.free_stack.push_back((int16_t)(x.cap - 1 - i));
        x.has_snap = false;
        memset(x.snap, 0, sizeof(x.snap));
        x.last_pf.clear();
        x.pending.clear();
        memset(x.st, 0, sizeof(x.st));
        x.bytes.store(0);
        x.read_rec = false;
    }

    void resize_layer(int l, int cap, const uint64_t* ptrs, uint64_t slot_inds, const int32_t* eids,
                      const int32_t* slots, int n) {
        if (l < 0 || l >= kLayers) return;
        wait_layer_all(l);
        std::lock_guard<std::mutex> g(mu);
        Layer& x = L[l];
        x.cap = std::min(std::max(cap, 1), kExperts);
        for (int t = 0; t < x.nt; ++t) x.dst[t] = ptrs ? reinterpret_cast<uint8_t*>(ptrs[t]) : nullptr;
        x.dst_device = device_ptr(x.dst[0], &x.dev);
        x.slot_inds = reinterpret_cast<uint32_t*>(slot_inds);
        x.slot_inds_device = device_ptr(x.slot_inds, nullptr);
        clear_table(x, true);
        x.has_snap = false;
        memset(x.snap, 0, sizeof(x.snap));
        x.last_pf.clear();
        x.pending.clear();
        rebuild(x, eids, slots, std::max(n, 0));
    }

    void reset_cache(int l) {
        if (l < 0 || l >= kLayers) return;
        wait_layer_all(l);
        std::lock_guard<std::mutex> g(mu);
        Layer& x = L[l];
        clear_table(x, true);
        x.free_stack.clear();
        for (int i = 0; i < x.cap; ++i) x.free_stack.push_back((int16_t)(x.cap - 1 - i));
        x.has_snap = false;
        memset(x.snap, 0, sizeof(x.snap));
        x.last_pf.clear();
        x.pending.clear();
    }

    void reset_stats(int l) {
        if (l < 0 || l >= kLayers) return;
        std::lock_guard<std::mutex> g(mu);
        memset(L[l].st, 0, sizeof(L[l].st));
        L[l].bytes.store(0);
    }

    void start_prefetch(int l, const int32_t* preds, int n, int max_fetch) {
        if (l < 0 || l >= kLayers || !preds || n <= 0 || max_fetch <= 0) return;
        std::unique_lock<std::mutex> lk(mu);
        Layer& x = L[l];
        if (!x.init) return;
        for (OpRef& op : x.last_pf) {                  // the previous prediction's reads, unused
            if (!op || op->resolved) continue;
            op->resolved = true;
            if (op->started == 0) cancel(x, *op, false);
            else x.st[S_PF_WASTED]++;
        }
        x.last_pf.clear();
        memset(x.snap, 0, sizeof(x.snap));
        for (int e = 0; e < kExperts; ++e)
            if (x.slot_of[e] >= 0) x.snap[e >> 6] |= 1ull << (e & 63);
        x.has_snap = true;
        uint64_t protect[kExperts / 64] = {};
        int32_t missing[32];
        int nm = 0;
        const int cap_fetch = std::min(max_fetch, 32);
        for (int i = 0; i < n; ++i) {
            const int32_t e = preds[i];
            if (e < 0 || e >= kExperts) continue;
            const bool seen = (protect[e >> 6] >> (e & 63)) & 1;
            protect[e >> 6] |= 1ull << (e & 63);
            if (!seen && x.slot_of[e] < 0 && nm < cap_fetch) missing[nm++] = e;
        }
        for (int i = nm - 1; i >= 0; --i) {            // lowest-ranked first: the best ends MRU
            const int32_t e = missing[i];
            if (x.slot_of[e] >= 0) continue;
            int16_t prev;
            const int s = alloc(l, lk, protect, &prev);
            if (s < 0) return;
            insert(x, e, s);
            auto op = std::make_shared<ReadOp>();
            op->layer = l;
            op->eid = e;
            op->slot = (int16_t)s;
            op->prev_eid = prev;
            op->prefetch = true;
            op->total = x.nt;
            x.active[s] = op;
            x.last_pf.push_back(op);
            x.st[S_PF_ISSUED]++;
            queue_prefetch(l, x, op);
        }
        if (nm) work_cv.notify_all();
    }

    int step_decode(int l, const uint32_t* eids, int k, uint32_t* out) {
        if (l < 0 || l >= kLayers || !eids || k <= 0) return 0;
        for (int i = 0; i < k; ++i)
            if (eids[i] >= (uint32_t)kExperts) {
                moe_set_error("p1 step_decode: expert id %u out of range", eids[i]);
                return -1;
            }
        std::unique_lock<std::mutex> lk(mu);
        Layer& x = L[l];
        if (!x.init) return 0;
        x.st[S_DECODE_REQ] += (uint64_t)k;
        uint64_t want[kExperts / 64] = {};
        for (int i = 0; i < k; ++i) want[eids[i] >> 6] |= 1ull << (eids[i] & 63);
        auto needed = [&](int32_t e) { return (want[e >> 6] >> (e & 63)) & 1; };
        std::vector<OpRef> reads;
        if (!x.last_pf.empty()) {
            for (OpRef& op : x.last_pf) {              // predicted but not routed: drop or waste
                if (!op || op->resolved || needed(op->eid)) continue;
                op->resolved = true;
                if (op->started == 0) cancel(x, *op, true);
                else x.st[S_PF_WASTED]++;
            }
            for (OpRef& op : x.last_pf) {              // predicted and routed: promote
                if (!op || op->resolved || !needed(op->eid)) continue;
                op->resolved = true;
                x.st[S_PF_USED]++;
                if (op->started == 0) {
                    op->promoted = true;
                    op->prefetch = false;
                    x.st[S_PF_PROMOTED]++;
                    reads.push_back(op);
                } else if (!op->done) {                 // its remaining tensors jump the queue
                    std::deque<Task> keep;
                    for (Task& t : prefetchq) {
                        if (t.ops[0] == op) urgent.push_back(std::move(t));
                        else keep.push_back(std::move(t));
                    }
                    prefetchq.swap(keep);
                }
            }
            x.last_pf.clear();
        }
        {
            std::deque<Task> keep;
            for (Task& t : prefetchq)
                if (t.ops[0] && !t.ops[0]->cancelled && !t.ops[0]->promoted) keep.push_back(std::move(t));
            prefetchq.swap(keep);
        }
        for (int i = 0; i < k; ++i) {
            const int32_t e = (int32_t)eids[i];
            if (x.slot_of[e] >= 0) {
                if (!x.has_snap || ((x.snap[e >> 6] >> (e & 63)) & 1)) x.st[S_LRU_HITS]++;
                continue;
            }
            x.st[S_URGENT]++;
            int16_t prev;
            const int s = alloc(l, lk, want, &prev);
            if (s < 0) return -1;
            insert(x, e, s);
            auto op = std::make_shared<ReadOp>();
            op->layer = l;
            op->eid = e;
            op->slot = (int16_t)s;
            op->prev_eid = prev;
            op->total = x.nt;
            x.active[s] = op;
            reads.push_back(op);
        }
        x.has_snap = false;
        queue_urgent(l, x, reads, false);
        x.pending.clear();
        uint32_t slots[kExperts];
        for (int i = 0; i < k; ++i) {
            const int s = x.slot_of[eids[i]];
            to_tail(x, s);
            slots[i] = (uint32_t)s;
            if (out) out[i] = (uint32_t)s;
            x.pins[s]++;
            x.gpu_pinned.push_back((int16_t)s);
            if (busy(x, s)) x.pending.push_back(x.active[s]);
        }
        if (x.slot_inds) {
            if (!x.slot_inds_device) {
                memcpy(x.slot_inds, slots, sizeof(uint32_t) * k);
            } else if (hipMemcpyAsync(x.slot_inds, slots, sizeof(uint32_t) * k, hipMemcpyHostToDevice, compute) !=
                       hipSuccess) {
                moe_set_error("p1 step_decode: slot ids to device memory failed");
            }
        }
        if (!x.pending.empty() || !reads.empty()) work_cv.notify_all();
        return (int)x.pending.size();
    }

    void wait_layer_urgent(int l) {
        if (l < 0 || l >= kLayers) return;
        std::unique_lock<std::mutex> lk(mu);
        Layer& x = L[l];
        if (x.pending.empty()) return;
        auto all_done = [&] {
            for (const OpRef& op : x.pending)
                if (op && !op->done) return false;
            return true;
        };
        if (all_done()) {
            x.pending.clear();
            return;
        }
        const auto t0 = std::chrono::steady_clock::now();
        const std::vector<OpRef> ops = x.pending;
        for (;;) {
            bool fin = true;
            for (const OpRef& op : ops)
                if (op && !op->done) fin = false;
            if (fin) break;
            if (!help_or_wait(lk, true)) {
                moe_set_error("p1: layer %d waits for reads that are not queued", l);
                break;
            }
        }
        x.st[S_IO_WAIT_NS] += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                                  std::chrono::steady_clock::now() - t0).count();
        x.pending.clear();
    }

    void wait_layer_all(int l) {
        if (l < 0 || l >= kLayers) return;
        wait_layer_urgent(l);
        std::unique_lock<std::mutex> lk(mu);
        Layer& x = L[l];
        if (!x.init) return;
        for (;;) {
            bool fin = true;
            for (int s = 0; s < x.cap && fin; ++s)
                if (x.active[s] && !x.active[s]->done && !x.active[s]->cancelled) fin = false;
            if (fin) break;
            if (!help_or_wait(lk, false)) {
                moe_set_error("p1: layer %d has reads that are not queued", l);
                break;
            }
        }
    }

    void pin(int l, const uint32_t* s, int n, int d) {
        if (l < 0 || l >= kLayers || !s || n <= 0) return;
        std::lock_guard<std::mutex> g(mu);
        for (int i = 0; i < n; ++i)
            if (s[i] < (uint32_t)kExperts && (d > 0 || L[l].pins[s[i]] > 0)) L[l].pins[s[i]] += d;
        if (d < 0) done_cv.notify_all();
    }

    int force_invalidate(int l, double rate, moe_p1_uniform_fn draw, void* user) {
        if (l < 0 || l >= kLayers || rate <= 0.0) return 0;
        std::unique_lock<std::mutex> lk(mu);
        Layer& x = L[l];
        if (!x.init) return 0;
        std::vector<int16_t> chosen;
        for (int16_t s : ordered(x)) {
            if (x.pins[s] > 0 || x.eid_of[s] < 0) continue;
            if (rate >= 1.0 || (draw && draw(user) < rate)) chosen.push_back(s);
        }
        int n = 0;
        for (int16_t s : chosen) {
            if (x.pins[s] > 0 || x.eid_of[s] < 0) continue;
            OpRef a = x.active[s];
            if (a && !a->done && !a->cancelled) {
                if (a->prefetch && a->started == 0) {
                    a->resolved = true;
                    a->cancelled = true;
                    x.st[S_PF_CANCELLED]++;
                } else {
                    while (!a->done && !a->cancelled)
                        if (!help_or_wait(lk, false)) break;
                }
            }
            if (x.pins[s] > 0) continue;
            const int16_t e = x.eid_of[s];
            if (e < 0) continue;
            for (OpRef& op : x.last_pf)
                if (op && !op->resolved && op->slot == s) {
                    op->resolved = true;
                    x.st[S_PF_WASTED]++;
                }
            unlink(x, s);
            x.slot_of[e] = -1;
            x.eid_of[s] = -1;
            x.active[s].reset();
            x.snap[e >> 6] &= ~(1ull << (e & 63));
            if (x.dst[0] && x.rb[0]) {                 // scrub: a slot not reloaded shows it
                const size_t nb = (size_t)std::min<uint64_t>(64, x.rb[0]);
                uint8_t* p = x.dst[0] + (uint64_t)s * x.rb[0];
                if (!x.dst_device) memset(p, 0xA5, nb);
                else if (hipMemset(p, 0xA5, nb) != hipSuccess) (void)hipGetLastError();
            }
            x.free_stack.push_back(s);
            ++n;
        }
        x.st[S_FORCED] += (uint64_t)n;
        return n;
    }

    void load_sync(int l, const int32_t* eids, const int32_t* slots, int n, bool prefill) {
        if (l < 0 || l >= kLayers || n <= 0 || !eids || !slots) return;
        wait_layer_all(l);
        {
            std::lock_guard<std::mutex> g(mu);
            Layer& x = L[l];
            if (!x.init) return;
            for (int i = 0; i < n; ++i)
                if (eids[i] < 0 || eids[i] >= kExperts || slots[i] < 0 || slots[i] >= x.cap) {
                    moe_set_error("p1 load_sync: pair (%d, %d) out of range", eids[i], slots[i]);
                    return;
                }
            if (prefill) x.st[S_PRE_BYTES] += (uint64_t)n * x.expert_bytes;
            std::vector<OpRef> ops;
            for (int i = 0; i < n; ++i) {
                auto op = std::make_shared<ReadOp>();
                op->layer = l;
                op->eid = eids[i];
                op->slot = (int16_t)slots[i];
                op->total = x.nt;
                x.active[slots[i]] = op;
                ops.push_back(op);
            }
            queue_urgent(l, x, ops, prefill);
            x.pending = ops;
            work_cv.notify_all();
        }
        wait_layer_urgent(l);
    }

    void get_lru_state(int l, int32_t* eids, int32_t* slots, int* count) {
        if (l < 0 || l >= kLayers) {
            if (count) *count = 0;
            return;
        }
        wait_layer_all(l);
        std::lock_guard<std::mutex> g(mu);
        int c = 0;
        for (int16_t s : ordered(L[l])) {
            if (eids) eids[c] = L[l].eid_of[s];
            if (slots) slots[c] = s;
            ++c;
        }
        if (count) *count = c;
    }

    void set_lru_state(int l, const int32_t* eids, const int32_t* slots, int n, uint64_t add_req, uint64_t add_hits,
                       uint64_t add_miss) {
        if (l < 0 || l >= kLayers) return;
        wait_layer_all(l);
        std::lock_guard<std::mutex> g(mu);
        Layer& x = L[l];
        x.st[S_PRE_REQ] += add_req;
        x.st[S_PRE_HITS] += add_hits;
        x.st[S_PRE_MISSES] += add_miss;
        clear_table(x, false);
        x.has_snap = false;
        x.last_pf.clear();
        x.pending.clear();
        rebuild(x, eids, slots, (eids && slots) ? std::max(n, 0) : 0);
    }

    void stats(int l, uint64_t* out) {
        for (int i = 0; i < S_COUNT; ++i) out[i] = 0;
        if (l < 0 || l >= kLayers) return;
        std::lock_guard<std::mutex> g(mu);
        for (int i = 0; i < S_COUNT; ++i) out[i] = L[l].st[i];
        out[S_BYTES] = L[l].bytes.load(std::memory_order_relaxed);
    }

    void total(int n, uint64_t* out) {
        for (int i = 0; i < S_COUNT; ++i) out[i] = 0;
        std::lock_guard<std::mutex> g(mu);
        for (int l = 1; l < std::min(n, kLayers); ++l) {
            if (!L[l].init) continue;
            for (int i = 0; i < S_COUNT; ++i) out[i] += L[l].st[i];   // st[S_BYTES] stays 0
            out[S_BYTES] += L[l].bytes.load(std::memory_order_relaxed);
        }
    }

    int mark_read(int l, hipStream_t s) {
        if (l < 0 || l >= kLayers) { moe_set_error("p1 mark_read: bad layer %d", l); return -1; }
        Layer& x = L[l];
        if (!x.read_ev) HIP_TRY(hipEventCreateWithFlags(&x.read_ev, hipEventDisableTiming));
        HIP_TRY(hipEventRecord(x.read_ev, s));
        x.read_rec = true;
        return 0;
    }
};

extern "C" {

moe_p1* moe_p1_create(void) { return new moe_p1(); }
void moe_p1_destroy(moe_p1* p) { delete p; }
void moe_p1_init(moe_p1* p, int num_threads) { p->init(num_threads); }
void moe_p1_shutdown(moe_p1* p) { p->shutdown(); }
int moe_p1_num_threads(moe_p1* p) { return p->nthreads; }
void moe_p1_set_wait_reader_callback(moe_p1* p, moe_p1_reader_fn fn, void* user) {
    std::lock_guard<std::mutex> g(p->mu);
    p->reader_fn = fn;
    p->reader_user = user;
}
void moe_p1_set_compute_stream(moe_p1* p, void* stream) { p->compute = (hipStream_t)stream; }
int moe_p1_mark_read(moe_p1* p, int layer_idx, void* stream) { return p->mark_read(layer_idx, (hipStream_t)stream); }
void moe_p1_layer_init(moe_p1* p, int layer_idx, int fd, int capacity, int num_tensors, const uint64_t* base_offsets,
                       const uint64_t* row_bytes, const uint64_t* base_ptrs, uint64_t slot_inds_ptr) {
    p->layer_init(layer_idx, fd, capacity, num_tensors, base_offsets, row_bytes, base_ptrs, slot_inds_ptr);
}
void moe_p1_resize_layer(moe_p1* p, int layer_idx, int new_capacity, const uint64_t* new_base_ptrs,
                         uint64_t slot_inds_ptr, const int32_t* ordered_eids, const int32_t* ordered_slots, int count) {
    p->resize_layer(layer_idx, new_capacity, new_base_ptrs, slot_inds_ptr, ordered_eids, ordered_slots, count);
}
void moe_p1_reset_cache(moe_p1* p, int layer_idx) { p->reset_cache(layer_idx); }
void moe_p1_reset_stats(moe_p1* p, int layer_idx) { p->reset_stats(layer_idx); }
void moe_p1_start_prefetch(moe_p1* p, int layer_idx, const int32_t* pred_eids, int pred_count, int max_fetch) {
    p->start_prefetch(layer_idx, pred_eids, pred_count, max_fetch);
}
int moe_p1_step_decode(moe_p1* p, int layer_idx, const uint32_t* eids, int k, uint32_t* out_slots) {
    return p->step_decode(layer_idx, eids, k, out_slots);
}
void moe_p1_wait_layer_urgent(moe_p1* p, int layer_idx) { p->wait_layer_urgent(layer_idx); }
void moe_p1_wait_layer_all(moe_p1* p, int layer_idx) { p->wait_layer_all(layer_idx); }
void moe_p1_wait_all(moe_p1* p) {
    for (int l = 0; l < kLayers; ++l) p->wait_layer_all(l);
}
void moe_p1_unpin_layer_slots(moe_p1* p, int layer_idx) {
    if (layer_idx >= 0 && layer_idx < kLayers) p->unpin_layer(layer_idx);
}
void moe_p1_pin_slots(moe_p1* p, int layer_idx, const uint32_t* slots, int count) { p->pin(layer_idx, slots, count, 1); }
void moe_p1_unpin_slots(moe_p1* p, int layer_idx, const uint32_t* slots, int count) {
    p->pin(layer_idx, slots, count, -1);
}
int moe_p1_get_slot_pin_count(moe_p1* p, int layer_idx, int slot) {
    if (layer_idx < 0 || layer_idx >= kLayers || slot < 0 || slot >= kExperts) return 0;
    std::lock_guard<std::mutex> g(p->mu);
    return p->L[layer_idx].pins[slot];
}
int moe_p1_force_invalidate(moe_p1* p, int layer_idx, double rate, moe_p1_uniform_fn draw, void* user) {
    return p->force_invalidate(layer_idx, rate, draw, user);
}
void moe_p1_load_sync(moe_p1* p, int layer_idx, const int32_t* eids, const int32_t* slots, int count, int is_prefill) {
    p->load_sync(layer_idx, eids, slots, count, is_prefill != 0);
}
void moe_p1_get_lru_state(moe_p1* p, int layer_idx, int32_t* out_eids, int32_t* out_slots, int* out_count) {
    p->get_lru_state(layer_idx, out_eids, out_slots, out_count);
}
void moe_p1_set_lru_state(moe_p1* p, int layer_idx, const int32_t* ordered_eids, const int32_t* ordered_slots,
                          int count, uint64_t add_prefill_requests, uint64_t add_prefill_hits,
                          uint64_t add_prefill_misses) {
    p->set_lru_state(layer_idx, ordered_eids, ordered_slots, count, add_prefill_requests, add_prefill_hits,
                     add_prefill_misses);
}
void moe_p1_get_layer_stats(moe_p1* p, int layer_idx, uint64_t* out16) { p->stats(layer_idx, out16); }
void moe_p1_get_total_stats(moe_p1* p, int num_layers, uint64_t* out16) { p->total(num_layers, out16); }

void* moe_p1_mt64_create(uint64_t seed) { return new std::mt19937_64(seed); }
void moe_p1_mt64_destroy(void* g) { delete static_cast<std::mt19937_64*>(g); }
uint64_t moe_p1_mt64_next(void* g) { return (*static_cast<std::mt19937_64*>(g))(); }
double moe_p1_mt64_uniform(void* g) {
    std::uniform_real_distribution<double> d(0.0, 1.0);
    return d(*static_cast<std::mt19937_64*>(g));
}

}  // extern "C"
