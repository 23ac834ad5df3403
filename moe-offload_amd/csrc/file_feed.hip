// Device-driven staging from the on-disk tier: mailboxes, the feeder thread and the two kernels
// (see file_feed.h).  Reference behaviour being served: the misses of a step are read from the
// expert shard by the reader threads and land in their slots before the layer's matmul
// (mlx-qwen38/expert_io.c:187-356, 583-685); here the step itself runs on the GPU.
#include "file_feed.h"

#include <sched.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "file_io.h"

namespace filefeed {
namespace {

// Entry flags carry the epoch of the list they answer (so a flag left from an earlier epoch is
// never taken for this one): the epoch once the entry landed, the epoch | kFeedError when its
// read failed.  Epochs stay below 2^31.
constexpr uint32_t kFeedError = 0x80000000u;
constexpr uint64_t kAlign = 4096;             // O_DIRECT granularity (and the bounce slack)
// Page-cache reads are cut into pieces of this size, so a short list (a layer's few misses) still
// keeps every reader thread busy; O_DIRECT reads stay whole (cut the same way they were no faster
// here and slower in the host-driven reads, 11.4-11.5 -> 9.4-10.0 tok/s on one box).
constexpr uint64_t kPiece = 256 * 1024;

// One (layer, list) mailbox, host-coherent: written by k_file_publish, read by the feeder.
struct Mail {
    uint32_t epoch;                           // stored last
    int32_t n;
    int32_t eid[MOE_MAX_PREFETCH];
};

struct FeedList {
    Mail* mail = nullptr;                     // host view (mapped, host-coherent)
    Mail* mail_dev = nullptr;
    uint32_t* landed = nullptr;               // [cap] entry flags (host writes, GPU polls)
    uint32_t* landed_dev = nullptr;
    uint8_t* bounce = nullptr;                // [cap][entry_bytes] pinned, mapped
    uint8_t* bounce_dev = nullptr;
    uint32_t* epoch_dev = nullptr;            // device word: the list's current epoch
    int cap = 0;
    uint32_t seen = 0;                        // feeder: last epoch taken
    std::atomic<int> left[MOE_MAX_PREFETCH];  // reads still to land per entry
};

struct Inflight {
    std::shared_ptr<fileio::Batch> batch;
    int list;
    uint32_t epoch;
    int n;
};

struct FeedLayer {
    std::atomic<bool> active{false};
    bool unpublished[2] = {false, false};     // a table op changed the list since its publication
    LayerIO io;
    uint64_t entry_bytes = 0;
    uint64_t toff[MOE_NUM_TENSORS] = {};      // data of tensor t inside an entry
    FeedList list[2];
    std::vector<Inflight> inflight;           // the feeder's batches (under g.mu)
    void* host_block = nullptr;               // mailboxes + flags
    void* bounce_block = nullptr;
    uint32_t* epochs_dev = nullptr;           // list 0 / 1 epoch words
};

struct Feed {
    std::mutex mu;                            // the feeder holds it while it looks at the layers
    std::thread thread;
    std::atomic<bool> stop{false};
    bool running = false;
    FeedLayer layers[MOE_MAX_LAYERS];
    std::atomic<uint64_t> timeout_us{10'000'000};
    int32_t* fault = nullptr;                 // host-coherent sticky fault word (host view)
    int32_t* fault_dev = nullptr;
};

// Never destroyed: the feeder may still be running when the process exits.
Feed& G() {
    static Feed* g = new Feed;
    return *g;
}

// ---- kernels --------------------------------------------------------------------------------

struct PubArgs {
    const SlotTable* t[2];
    int list[2];
    Mail* mail[2];
    uint32_t* epoch[2];
    int cap[2];
};

// One wave: each named table's copy list (ids only; the slots stay in the table) to its
// mailbox, then the list's epoch advanced and stored last with system-scope release (a release
// store waits for every earlier store of the wave, so the ids and the count are visible first).
__global__ __launch_bounds__(64) void k_file_publish(PubArgs a) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const SlotTable* t = a.t[i];
        if (!t) continue;
        int n = a.list[i] ? t->pf_n_copy : t->n_copy;
        n = n < 0 ? 0 : (n > a.cap[i] ? a.cap[i] : n);
        if (lane < n) a.mail[i]->eid[lane] = a.list[i] ? t->pf_copy_eid[lane] : t->copy_eid[lane];
        if (lane == 0) {
            a.mail[i]->n = n;
            const uint32_t e = (*a.epoch[i] + 1) & ~kFeedError;
            *a.epoch[i] = e;
            __hip_atomic_store(&a.mail[i]->epoch, e, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

struct StageArgs {
    SlotTable* t;
    int32_t* fault;                           // the library's fault word (host-coherent)
    int list, cap;
    const uint32_t* epoch;                    // device word, advanced by k_file_publish
    const uint32_t* landed;
    const uint8_t* bounce;
    uint64_t entry_bytes, toff;
    uint8_t* pool;
    uint64_t bytes;                           // bytes per expert of this tensor (= slot stride)
    uint64_t spin_ticks;                      // longest wait per entry, in wall-clock ticks
};

// Copy c = blockIdx.y of the list: wait for its entry's flag to carry this epoch (one thread
// polls, the block waits at the barrier), then copy the entry's tensor bytes into the slot with
// blockIdx.x striding over 16-byte units, four in flight per thread (as k_stage).  The bounce
// entries are host-coherent (fine-grained) memory: the GPU caches none of their lines, so a
// rewritten entry is read fresh.  A failed read
// or a wait past spin_ticks leaves the slot alone and sets the table's sticky io_fault word and the
// library's fault word; a table that already carries a fault copies nothing more (it stays wrong
// until reset_cache, and the host reports it).
__global__ __launch_bounds__(256) void k_stage_file(StageArgs a) {
    const int c = blockIdx.y;
    const int n = a.list ? a.t->pf_n_copy : a.t->n_copy;
    if (c >= (n < a.cap ? n : a.cap)) return;
    const int slot = a.list ? a.t->pf_copy_slot[c] : a.t->copy_slot[c];
    if (slot < 0 || slot >= a.t->capacity) return;
    __shared__ int ok;
    if (threadIdx.x == 0) {
        const uint32_t e = *a.epoch;
        const uint64_t t0 = wall_clock64();
        int r = __hip_atomic_load(&a.t->io_fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ? -3 : 0;
        while (r == 0) {
            const uint32_t v = __hip_atomic_load(a.landed + c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
            if (v == e) { r = 1; break; }
            if (v == (e | kFeedError)) { r = -1; break; }
            if (wall_clock64() - t0 > a.spin_ticks) { r = -2; break; }
            __builtin_amdgcn_s_sleep(4);
        }
        if (r == -1 || r == -2) {
            const int32_t code = r == -1 ? kStatusReadFailed : kStatusTimedOut;
            atomicCAS(&a.t->io_fault, 0, code);
            // a plain store to host memory (no read-modify-write over the link)
            __hip_atomic_store(a.fault, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        ok = r;
    }
    __syncthreads();
    if (ok != 1) return;
    const uint4* src = reinterpret_cast<const uint4*>(a.bounce + (uint64_t)c * a.entry_bytes + a.toff);
    uint4* dst = reinterpret_cast<uint4*>(a.pool + (uint64_t)slot * a.bytes);
    const unsigned units = (unsigned)(a.bytes / 16);
    const unsigned step = gridDim.x * blockDim.x;
    for (unsigned u = blockIdx.x * blockDim.x + threadIdx.x; u < units; u += 4 * step) {
        const bool m1 = u + step < units, m2 = u + 2 * step < units, m3 = u + 3 * step < units;
        uint4 v0 = src[u], v1 = {}, v2 = {}, v3 = {};
        if (m1) v1 = src[u + step];
        if (m2) v2 = src[u + 2 * step];
        if (m3) v3 = src[u + 3 * step];
        dst[u] = v0;
        if (m1) dst[u + step] = v1;
        if (m2) dst[u + 2 * step] = v2;
        if (m3) dst[u + 3 * step] = v3;
    }
}

// ---- feeder ---------------------------------------------------------------------------------

// Reads of a newly published list: entry c <- expert mail.eid[c], per tensor (a blob file has
// one) the expert's bytes (through the page cache in pieces of kPiece), straight into the entry (O_DIRECT: the 4 KiB-aligned
// range around the bytes, placed so the bytes land at the entry's data offset; the entry keeps
// 4 KiB of slack on each side of every tensor for that).  The worker finishing an entry's last
// piece sets its flag.
void start_reads(FeedLayer& F, int li, uint32_t epoch, int n) {
    FeedList& Q = F.list[li];
    const LayerIO& io = F.io;
    const bool direct = io.fd_direct >= 0;
    int per = 0;                                        // tensors to read per expert
    for (int t = 0; t < MOE_NUM_TENSORS; ++t)
        if (io.row_bytes[t] && io.dst[t]) ++per;
    auto b = std::make_shared<fileio::Batch>();
    for (int c = 0; c < n; ++c) {
        const int32_t e = Q.mail->eid[c];
        if (e < 0 || e >= MOE_NUM_EXPERTS || per == 0) {
            __atomic_store_n(&Q.landed[c], epoch | kFeedError, __ATOMIC_RELEASE);
            continue;
        }
        uint8_t* entry = Q.bounce + (uint64_t)c * F.entry_bytes;
        int pieces = 0;
        for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
            const uint64_t rb = io.row_bytes[t];
            if (!rb || !io.dst[t]) continue;
            const uint64_t off = io.src[t] + (uint64_t)e * rb;
            // [a, end): the bytes read (O_DIRECT: the 4 KiB-aligned range around [off, off + rb)),
            // landing at dst + (p - a); cut into pieces of kPiece (a multiple of 4 KiB)
            const uint64_t a = direct ? off & ~(kAlign - 1) : off;
            const uint64_t end = direct ? (off + rb + kAlign - 1) & ~(kAlign - 1) : off + rb;
            uint8_t* dst = entry + F.toff[t] - (off - a);
            const uint64_t piece = direct ? end - a : kPiece;
            for (uint64_t p = a; p < end; p += piece) {
                const uint64_t pe = p + piece < end ? p + piece : end;
                const uint64_t need = (pe < off + rb ? pe : off + rb) - p;
                b->reads.push_back(fileio::Read{direct ? io.fd_direct : io.fd, p, pe - p, need, dst + (p - a), direct, c});
                ++pieces;
            }
        }
        Q.left[c].store(pieces, std::memory_order_relaxed);
    }
    if (b->reads.empty()) return;
    uint32_t* landed = Q.landed;
    std::atomic<int>* left = Q.left;
    b->on_read = [landed, left, epoch](int c) -> int {
        if (left[c].fetch_sub(1, std::memory_order_acq_rel) == 1) __atomic_store_n(&landed[c], epoch, __ATOMIC_RELEASE);
        return 0;
    };
    fileio::submit(b);
    F.inflight.push_back(Inflight{b, li, epoch, n});
}

// Batches that ended: a failed one marks its entries that never landed.
void reap(FeedLayer& F) {
    for (size_t i = 0; i < F.inflight.size();) {
        Inflight& f = F.inflight[i];
        bool done, failed;
        {
            std::lock_guard<std::mutex> g(f.batch->mu);
            done = f.batch->done;
            failed = f.batch->failed;
        }
        if (!done) { ++i; continue; }
        if (failed) {
            uint32_t* landed = F.list[f.list].landed;
            for (int c = 0; c < f.n; ++c)
                if (__atomic_load_n(&landed[c], __ATOMIC_ACQUIRE) != f.epoch)
                    __atomic_store_n(&landed[c], f.epoch | kFeedError, __ATOMIC_RELEASE);
        }
        F.inflight.erase(F.inflight.begin() + i);
    }
}

void feeder_main() {
    Feed& g = G();
    auto last = std::chrono::steady_clock::now();
    while (!g.stop.load(std::memory_order_acquire)) {
        bool work = false, busy = false;
        {
            std::lock_guard<std::mutex> lk(g.mu);
            for (int l = 0; l < MOE_MAX_LAYERS; ++l) {
                FeedLayer& F = g.layers[l];
                if (!F.active.load(std::memory_order_acquire)) continue;
                reap(F);
                for (int li = 0; li < 2; ++li) {
                    FeedList& Q = F.list[li];
                    const uint32_t e = __atomic_load_n(&Q.mail->epoch, __ATOMIC_ACQUIRE);
                    if (e == Q.seen) continue;
                    // the list's previous reads write into the same entries and counters: a new
                    // epoch starts once they have all ended (normally they have: its staging waited
                    // for every entry; after a timed-out wait they may still be landing)
                    bool reading = false;
                    for (const Inflight& f : F.inflight) reading |= f.list == li;
                    if (reading) { busy = true; continue; }
                    Q.seen = e;
                    work = true;
                    int n = Q.mail->n;
                    n = n < 0 ? 0 : (n > Q.cap ? Q.cap : n);
                    if (n) start_reads(F, li, e, n);
                }
                reap(F);
                busy |= !F.inflight.empty();
            }
        }
        const auto now = std::chrono::steady_clock::now();
        if (work || busy) last = now;
        // A decode publishes a list every few hundred microseconds: poll tightly while tokens
        // run, back off once nothing has happened for a while.
        if (now - last > std::chrono::milliseconds(20)) std::this_thread::sleep_for(std::chrono::microseconds(200));
        else if (!work) sched_yield();
    }
}

// At process exit (registered after the HIP runtime was loaded, so it runs before the runtime's
// own teardown frees the mailboxes): end the feeder's polling; reads in flight are left alone.
void stop_feeder() {
    Feed& g = G();
    std::thread t;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        if (!g.running) return;
        g.stop.store(true, std::memory_order_release);
        t.swap(g.thread);
        g.running = false;
    }
    t.join();
}

void free_layer(FeedLayer& F) {
    if (F.epochs_dev) (void)hipFree(F.epochs_dev);
    if (F.host_block) (void)hipHostFree(F.host_block);
    if (F.bounce_block) (void)hipHostFree(F.bounce_block);
    F.epochs_dev = nullptr;
    F.host_block = F.bounce_block = nullptr;
    for (auto& Q : F.list) {
        Q.mail = Q.mail_dev = nullptr;
        Q.landed = Q.landed_dev = nullptr;
        Q.bounce = Q.bounce_dev = nullptr;
        Q.epoch_dev = nullptr;
        Q.cap = 0;
        Q.seen = 0;
    }
    F.entry_bytes = 0;
}

int dev_ptr(void* host, void** dev) {
    HIP_TRY(hipHostGetDevicePointer(dev, host, 0));
    return 0;
}

}  // namespace

int attach(int layer, const LayerIO& io) {
    if (layer < 0 || layer >= MOE_MAX_LAYERS) { moe_set_error("file feed: bad layer %d", layer); return -1; }
    if (io.fd < 0) { moe_set_error("file feed: layer %d has no file", layer); return -1; }
    detach(layer);
    Feed& g = G();
    FeedLayer& F = g.layers[layer];
    F.io = io;
    uint64_t off = 0;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        F.toff[t] = 0;
        if (!io.row_bytes[t] || !io.dst[t]) continue;
        if (io.row_bytes[t] % 16) { moe_set_error("file feed: tensor %d rows of %llu bytes (multiple of 16)", t, (unsigned long long)io.row_bytes[t]); return -1; }
        F.toff[t] = off + kAlign;
        off += kAlign + ((io.row_bytes[t] + kAlign - 1) & ~(kAlign - 1)) + kAlign;
    }
    if (!off) { moe_set_error("file feed: layer %d has no tensor to stage", layer); return -1; }
    F.entry_bytes = off;
    const size_t host_bytes = 2 * (sizeof(Mail) + MOE_MAX_PREFETCH * sizeof(uint32_t));
    const size_t entries = (size_t)kListCap[0] + kListCap[1];
    auto fail = [&]() { free_layer(F); return -1; };
    if (hipHostMalloc(&F.host_block, host_bytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostMalloc(&F.bounce_block, entries * F.entry_bytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
        moe_set_error("file feed: no pinned memory for layer %d (%zu bounce bytes)", layer, entries * (size_t)F.entry_bytes);
        return fail();
    }
    if (hipMalloc((void**)&F.epochs_dev, 2 * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(F.epochs_dev, 0, 2 * sizeof(uint32_t)) != hipSuccess) {
        moe_set_error("file feed: no device memory for layer %d's epochs", layer);
        return fail();
    }
    memset(F.host_block, 0, host_bytes);
    uint8_t* hb = (uint8_t*)F.host_block;
    uint8_t* bb = (uint8_t*)F.bounce_block;
    for (int li = 0; li < 2; ++li) {
        FeedList& Q = F.list[li];
        Q.cap = kListCap[li];
        Q.mail = (Mail*)hb;
        hb += sizeof(Mail);
        Q.landed = (uint32_t*)hb;
        hb += MOE_MAX_PREFETCH * sizeof(uint32_t);
        Q.bounce = bb;
        bb += (size_t)Q.cap * F.entry_bytes;
        Q.epoch_dev = F.epochs_dev + li;
        Q.seen = 0;
        void *md, *ld, *bd;
        if (dev_ptr(Q.mail, &md) || dev_ptr(Q.landed, &ld) || dev_ptr(Q.bounce, &bd)) return fail();
        Q.mail_dev = (Mail*)md;
        Q.landed_dev = (uint32_t*)ld;
        Q.bounce_dev = (uint8_t*)bd;
    }
    std::lock_guard<std::mutex> lk(g.mu);
    if (!g.fault) {                                   // the library's fault word, kept until exit
        void *h = nullptr, *d = nullptr;
        if (hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess || dev_ptr(h, &d)) {
            if (h) (void)hipHostFree(h);
            moe_set_error("file feed: no pinned memory for the fault word");
            return fail();
        }
        memset(h, 0, 256);
        g.fault = (int32_t*)h;
        g.fault_dev = (int32_t*)d;
    }
    F.active.store(true, std::memory_order_release);
    F.unpublished[0] = F.unpublished[1] = false;
    if (!g.running) {
        g.stop.store(false);
        g.thread = std::thread(feeder_main);
        g.running = true;
        static std::once_flag at_exit;                // the feeder polls pinned memory: it stops
        std::call_once(at_exit, [] { std::atexit(stop_feeder); });   // before the runtime's teardown
    }
    return 0;
}

bool attached(int layer) {
    return layer >= 0 && layer < MOE_MAX_LAYERS && G().layers[layer].active.load(std::memory_order_acquire);
}

void detach(int layer) {
    if (layer < 0 || layer >= MOE_MAX_LAYERS) return;
    Feed& g = G();
    FeedLayer& F = g.layers[layer];
    std::vector<Inflight> fl;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        if (!F.active.load()) {
            if (F.host_block || F.bounce_block || F.epochs_dev) free_layer(F);
            return;
        }
        F.active.store(false, std::memory_order_release);
        fl.swap(F.inflight);
    }
    std::string msg;
    for (auto& f : fl) (void)fileio::wait(f.batch, msg);     // their workers write into the buffers
    free_layer(F);
}

void mark_table_op(int layer, int list) {
    if (attached(layer) && (list == 0 || list == 1)) G().layers[layer].unpublished[list] = true;
}

int32_t fault_word() {
    const int32_t* f = G().fault;
    return f ? __atomic_load_n(f, __ATOMIC_ACQUIRE) : 0;
}

void clear_fault_word() {
    if (G().fault) __atomic_store_n(G().fault, 0, __ATOMIC_RELEASE);
}

int publish(int layer, int list, SlotTable* dtab, hipStream_t s) {
    if (!attached(layer)) { moe_set_error("file feed: layer %d is not a device-driven file layer", layer); return -1; }
    if (list != 0 && list != 1) { moe_set_error("file feed: list %d (0 decode step, 1 prefetch)", list); return -1; }
    G().layers[layer].unpublished[list] = false;
    FeedList& Q = G().layers[layer].list[list];
    PubArgs a = {};
    a.t[0] = dtab;
    a.list[0] = list;
    a.mail[0] = Q.mail_dev;
    a.epoch[0] = Q.epoch_dev;
    a.cap[0] = Q.cap;
    hipLaunchKernelGGL(k_file_publish, dim3(1), dim3(64), 0, s, a);
    HIP_TRY(hipGetLastError());
    return 0;
}

int stage(int layer, int list, SlotTable* dtab, int ctas, hipStream_t s) {
    if (!attached(layer)) { moe_set_error("file feed: layer %d is not a device-driven file layer", layer); return -1; }
    if (list != 0 && list != 1) { moe_set_error("file feed: list %d (0 decode step, 1 prefetch)", list); return -1; }
    FeedLayer& F = G().layers[layer];
    if (F.unpublished[list]) {
        moe_set_error("file feed: layer %d list %d changed by a table operation since its last publication "
                      "(c_layer_publish_dev before c_layer_stage_dev)", layer, list);
        return -1;
    }
    FeedList& Q = F.list[list];
    int dev = 0, khz = 0;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    if (khz <= 0) khz = 100000;
    const uint64_t ticks = G().timeout_us.load(std::memory_order_relaxed) * (uint64_t)khz / 1000;
    if (ctas <= 0) ctas = 2;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        const uint64_t rb = F.io.row_bytes[t];
        if (!rb || !F.io.dst[t]) continue;
        if (rb / 16 > 0xFFFFFFFFull) { moe_set_error("file feed: tensor %d rows too large", t); return -1; }
        StageArgs a = {};
        a.t = dtab;
        a.fault = G().fault_dev;
        a.list = list;
        a.cap = Q.cap;
        a.epoch = Q.epoch_dev;
        a.landed = Q.landed_dev;
        a.bounce = Q.bounce_dev;
        a.entry_bytes = F.entry_bytes;
        a.toff = F.toff[t];
        a.pool = (uint8_t*)F.io.dst[t];
        a.bytes = rb;
        a.spin_ticks = ticks;
        MOE_LAUNCH(TK_STAGE, k_stage_file, dim3(ctas, Q.cap), dim3(256), 0, s, a);
        HIP_TRY(hipGetLastError());
    }
    return 0;
}

void set_timeout_us(uint64_t us) { G().timeout_us.store(us ? us : 10'000'000, std::memory_order_relaxed); }

void shutdown() {
    for (int l = 0; l < MOE_MAX_LAYERS; ++l) detach(l);
    stop_feeder();
}

}  // namespace filefeed
