// C-ABI of libmoe_offload: the expert-cache entry points of mlx-qwen38/expert_io.c
// (same names, argument meaning and silent-ignore behaviour for out-of-range layers), plus the
// gfx950 compute entry points of the routed-expert decode path.  Declarations with the
// reference interface each one replaces are in include/moe_offload.h.
//
// Storage tiers.  The reference reads experts from an SSD file into slot buffers in unified
// memory.  Here a layer's pool is device memory (HBM) and its experts live in a host expert
// store; `c_layer_init` keeps the reference signature:
//   fd == -1 : base_offsets[t] are host addresses of tensor t's store (expert e at
//              base_offsets[t] + e * row_bytes[t]); pinned memory (c_host_alloc) is required
//              for overlap and for device-driven staging.
//   fd >= 0  : base_offsets[t] are file offsets, as in the reference; a batch of misses is read
//              by the reader-thread pool (file_io.h) as one read per (tensor, run of consecutive
//              experts) into a shared pinned bounce buffer, each read's copies to the slots are
//              queued as soon as it lands, and the batch is joined where its slots are needed
//              (host-driven staging only).
//   base_ptrs[t] : device address of tensor t's slot pool (slot s at + s * row_bytes[t]).
//   A tensor with row_bytes > 0 but a zero source or destination is accounting-only.
//
// Ordering (host-driven layers).  Copies run on a library-owned non-blocking stream.  Before
// copying into a layer's pool the copy stream waits for the last kernel that read it (WAR);
// before a kernel reads the pool the compute stream waits for the copies (RAW).  Waiting is
// GPU-side: c_layer_wait_prefetch makes the compute stream wait for every pending copy and
// returns without blocking the host; the synchronous calls (c_layer_step_decode,
// c_layer_load_sync) also block the host until their copies have landed.
#include <hip/hip_fp16.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <mutex>
#include <vector>

#include <fcntl.h>

#include <algorithm>
#include <memory>
#include <numeric>
#include <string>

#include "file_feed.h"
#include "file_io.h"
#include "moe_common.h"
#include "moe_offload.h"
#include "slot_table_host.h"

namespace {

struct LayerState {
    bool init = false;
    int fd = -1;
    int capacity = 0;
    uint64_t src[MOE_NUM_TENSORS] = {};
    uint64_t row_bytes[MOE_NUM_TENSORS] = {};
    uint64_t dst[MOE_NUM_TENSORS] = {};
    uint64_t dev_src[MOE_NUM_TENSORS] = {};   // device-visible store addresses (pinned stores)
    uint32_t* slot_inds = nullptr;
    bool slot_inds_device = false;
    SlotTable tab;                            // authoritative for host-driven layers
    SlotTable* dtab = nullptr;                // authoritative for device-driven layers
    bool device_mode = false;
    hipEvent_t copy_done = nullptr, read_done = nullptr;
    // copy_pending: copies the compute stream has not been made to wait for yet.  inflight:
    // copies that may still be running on the copy streams (a GPU-side wait does not end them);
    // cleared only once copy_done is known to have completed.  inflight_slots: the slots those
    // copies write.
    bool copy_pending = false, read_recorded = false;
    bool inflight = false;
    uint64_t inflight_slots[MOE_NUM_EXPERTS / 64] = {};
    // Q2 format for the layer's GEMV: a blob pool in tensor 0 (c_layer_set_format) or the
    // reference's 9 tensors (c_layer_set_format9: fmt9, with E9 built from the pools)
    int hidden = 0, inter = 0, group = 0;
    bool fmt9 = false;
    Q2Experts E9 = {};
    // File-backed stores: the in-flight batch of reads, and an O_DIRECT descriptor of the same
    // file when direct reads are on (-1 otherwise).
    // fbatch: the layer's latest batch (each batch is queued after the one before it, so this one
    // being done means all are); fpf: its latest prefetch batch (records pf_done) until joined.
    std::shared_ptr<fileio::Batch> fbatch, fpf;
    int fd_direct = -1;
    // Prefetch copies (c_layer_start_prefetch, the scheduler's next-layer prefetch) also record
    // pf_done, so work on the step's hit slots can wait for them alone (split GLU).
    hipEvent_t pf_done = nullptr;
    bool pf_pending = false;
    uint8_t* split_dev = nullptr;             // device copy of the split lists (split GLU)
};

LayerState g_layers[MOE_MAX_LAYERS];

// Scheduler split lists, per layer, kept until the next split (c_layer_get_split_inds reads
// the last one, as cpp/third_party/expert_io.c:1062-1092 does).
SplitLists g_split[MOE_MAX_LAYERS];

// Per-token accounting (cpp/third_party/expert_io.c:98-111,1002-1038).
bool g_acct_on = false;
int32_t g_token_seq = 0, g_cur_token = -1;
uint64_t g_tok[10] = {0};

slot_host::Acct* acct_for(LayerState& L, slot_host::Acct& a) {
    if (!g_acct_on) return nullptr;
    a.cur_token = g_cur_token;
    a.evicted_at = L.tab.evicted_at;
    a.tok = g_tok;
    return &a;
}

void reset_evictions(LayerState& L) {
    for (int e = 0; e < MOE_NUM_EXPERTS; ++e) L.tab.evicted_at[e] = -1;
}

// The device-driven tables (for the accounting control and gather kernels).
TableSet device_tables() {
    TableSet ts = {};
    for (int l = 0; l < MOE_MAX_LAYERS; ++l)
        if (g_layers[l].init && g_layers[l].device_mode && g_layers[l].dtab) ts.t[ts.n++] = g_layers[l].dtab;
    return ts;
}
hipStream_t g_compute = nullptr;             // caller's stream (null stream by default)
hipStream_t g_copy = nullptr;
// More copy streams: blob copies from the pinned store go round robin over g_copy and these (one
// stream of blob-sized hipMemcpyAsync copies moves ~37 GB/s, two ~49 GB/s; three or four are
// slower, sharing the process's 4 hardware queues), and each batch joins them into g_copy, so
// every event recorded on g_copy after a batch covers all of it.
constexpr int kCopyStreams = 2;
hipStream_t g_copy_more[kCopyStreams - 1] = {};
hipEvent_t g_copy_more_done[kCopyStreams - 1] = {};
bool g_ready = false;
int g_dev = 0;                              // device of the copy streams (the reader threads set it)
bool g_direct = false;                      // file-backed layers read with O_DIRECT when possible

// Pinned bounce buffers of the file tier, shared by every layer and used in turn.  A buffer is
// reused once its last batch (`user`) has queued its copies and they have run (`free_ev`, recorded
// after them); it grows to the largest batch it has held.
struct Bounce {
    uint8_t* p = nullptr;
    size_t bytes = 0;
    hipEvent_t free_ev = nullptr;
    std::shared_ptr<fileio::Batch> user;
};
constexpr int kBounceBufs = 8;
Bounce g_bounce[kBounceBufs];
int g_bounce_next = 0;
std::mutex g_err_mu;
char g_err[1024] = {0};

bool valid_layer(int l) { return l >= 0 && l < MOE_MAX_LAYERS; }

int ensure_runtime() {
    if (g_ready) return 0;
    HIP_TRY(hipGetDevice(&g_dev));
    HIP_TRY(hipStreamCreateWithFlags(&g_copy, hipStreamNonBlocking));
    for (int i = 0; i < kCopyStreams - 1; ++i) {
        HIP_TRY(hipStreamCreateWithFlags(&g_copy_more[i], hipStreamNonBlocking));
        HIP_TRY(hipEventCreateWithFlags(&g_copy_more_done[i], hipEventDisableTiming));
    }
    g_ready = true;
    return 0;
}

int ensure_events(LayerState& L) {
    if (!L.copy_done) HIP_TRY(hipEventCreateWithFlags(&L.copy_done, hipEventDisableTiming));
    if (!L.read_done) HIP_TRY(hipEventCreateWithFlags(&L.read_done, hipEventDisableTiming));
    if (!L.pf_done) HIP_TRY(hipEventCreateWithFlags(&L.pf_done, hipEventDisableTiming));
    return 0;
}

uint64_t expert_bytes_of(const LayerState& L) {
    uint64_t b = 0;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) b += L.row_bytes[t];
    return b;
}

// Pull a device-mode table back to the host copy (blocking) / push the host copy to device.
int pull_table(LayerState& L) {
    if (!L.device_mode) return 0;
    HIP_TRY(hipMemcpyAsync(&L.tab, L.dtab, sizeof(SlotTable), hipMemcpyDeviceToHost, g_compute));
    HIP_TRY(hipStreamSynchronize(g_compute));
    return 0;
}

int push_table(LayerState& L) {
    if (!L.device_mode) return 0;
    HIP_TRY(hipMemcpyAsync(L.dtab, &L.tab, sizeof(SlotTable), hipMemcpyHostToDevice, g_compute));
    HIP_TRY(hipStreamSynchronize(g_compute));
    return 0;
}

// Host join of the layer's in-flight file batch: its reads are done and its copies queued.
int join_file(LayerState& L) {
    if (!L.fbatch) return 0;
    std::string msg;
    const int rc = fileio::wait(L.fbatch, msg);
    L.fbatch.reset();
    L.fpf.reset();
    if (rc) {
        moe_set_error("expert file read: %s", msg.c_str());
        return -1;
    }
    return 0;
}

// Host join of the layer's latest prefetch batch only (pf_done recorded).
int join_prefetch_file(LayerState& L) {
    if (!L.fpf) return 0;
    std::string msg;
    const int rc = fileio::wait(L.fpf, msg);
    L.fpf.reset();
    if (rc) {
        moe_set_error("expert file read: %s", msg.c_str());
        return -1;
    }
    return 0;
}

// Wait until bounce buffer b may be overwritten: its last batch has queued its copies (a failed
// batch may have queued part of them: the copy stream is drained) and they have run.
int bounce_idle(Bounce& b) {
    if (!b.user) return 0;
    std::string msg;                              // an error is reported by the owning layer's join
    const bool failed = fileio::wait(b.user, msg) != 0;
    b.user.reset();
    if (failed) HIP_TRY(hipStreamSynchronize(g_copy));
    else HIP_TRY(hipEventSynchronize(b.free_ev));
    return 0;
}

// Release the bounce buffers (every layer's batch joined first).
void release_bounce() {
    for (Bounce& b : g_bounce) {
        (void)bounce_idle(b);
        if (b.p) (void)hipHostFree(b.p);
        if (b.free_ev) (void)hipEventDestroy(b.free_ev);
        b = Bounce();
    }
}

// Free a layer's file-tier resources (after joining its batch).
void release_file(LayerState& L) {
    (void)join_file(L);
    if (L.fd_direct >= 0) close(L.fd_direct);
    L.fd_direct = -1;
}

// Forget the layer's in-flight copies once its last copy event has completed (non-blocking).
void settle_copies(LayerState& L) {
    if (!L.inflight) return;
    if (L.fbatch) {                                  // a file batch records copy_done when it ends
        std::lock_guard<std::mutex> g(L.fbatch->mu);
        if (!L.fbatch->done) return;
    }
    hipError_t e = hipEventQuery(L.copy_done);
    if (e == hipErrorNotReady) {
        (void)hipGetLastError();
        return;
    }
    L.inflight = false;
    memset(L.inflight_slots, 0, sizeof(L.inflight_slots));
}

// Block the host until every copy queued for the layer has landed.
int drain_copies(LayerState& L) {
    if (join_file(L)) return -1;
    if (L.inflight) HIP_TRY(hipEventSynchronize(L.copy_done));
    L.inflight = false;
    memset(L.inflight_slots, 0, sizeof(L.inflight_slots));
    return 0;
}

// A batch of misses of a file-backed layer: the (eid, slot) pairs sorted by expert id, each run of
// consecutive ids read as one contiguous range per tensor (expert_io.c:187-276) into a bounce
// buffer, longest reads first, by the reader threads.  The worker that completes a read queues its
// copies (one per run of consecutive slots) at once, so the copy engine works while the other
// reads run; the batch is queued after the layer's previous one (its copies go first: a demand
// miss may take a slot an in-flight prefetch is filling), and the worker completing the batch
// records copy_done (and pf_done for a prefetch).
// With O_DIRECT each read covers the 4 KiB-aligned range around its bytes (through the reader's
// own staging buffer: see fileio::Read::direct).
int issue_file_batch(LayerState& L, const int32_t* eids, const int32_t* slots, int n, bool prefetch) {
    constexpr uint64_t kAlign = 4096;
    const bool direct = L.fd_direct >= 0;
    std::vector<int> ord(n);
    std::iota(ord.begin(), ord.end(), 0);
    std::sort(ord.begin(), ord.end(), [&](int a, int b) { return eids[a] < eids[b]; });
    std::vector<std::pair<int, int>> runs;            // (first position in ord, length)
    for (int i = 0; i < n;) {
        int r = 1;
        while (i + r < n && eids[ord[i + r]] == eids[ord[i]] + r) ++r;
        runs.emplace_back(i, r);
        i += r;
    }
    struct Piece { int t, run; uint64_t boff, skip; };  // a tensor's run in the bounce buffer
    std::vector<Piece> pieces;
    std::vector<fileio::Read> reads;
    uint64_t total = 0;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        const uint64_t rb = L.row_bytes[t];
        if (!rb || !L.dst[t]) continue;
        for (size_t q = 0; q < runs.size(); ++q) {
            const uint64_t off = L.src[t] + (uint64_t)eids[ord[runs[q].first]] * rb, len = (uint64_t)runs[q].second * rb;
            const uint64_t a = direct ? off & ~(kAlign - 1) : off;
            const uint64_t end = direct ? (off + len + kAlign - 1) & ~(kAlign - 1) : off + len;
            pieces.push_back(Piece{t, (int)q, total, off - a});
            reads.push_back(fileio::Read{direct ? L.fd_direct : L.fd, a, end - a, off - a + len, nullptr, direct});
            total += (end - a + kAlign - 1) & ~(kAlign - 1);
        }
    }
    Bounce& B = g_bounce[g_bounce_next];
    g_bounce_next = (g_bounce_next + 1) % kBounceBufs;
    if (bounce_idle(B)) return -1;
    if (total > B.bytes) {
        if (B.p) HIP_TRY(hipHostFree(B.p));
        B.p = nullptr;
        B.bytes = 0;
        HIP_TRY(hipHostMalloc((void**)&B.p, total, hipHostMallocDefault));
        B.bytes = total;
    }
    if (!B.free_ev) HIP_TRY(hipEventCreateWithFlags(&B.free_ev, hipEventDisableTiming));
    for (size_t i = 0; i < reads.size(); ++i) reads[i].dst = B.p + pieces[i].boff;
    auto b = std::make_shared<fileio::Batch>();
    b->reads = std::move(reads);
    uint8_t* bounce = B.p;
    hipEvent_t copy_done = L.copy_done, pf_done = L.pf_done, free_ev = B.free_ev;
    std::vector<std::pair<int32_t, int32_t>> sorted(n);
    for (int i = 0; i < n; ++i) sorted[i] = {eids[ord[i]], slots[ord[i]]};
    const std::vector<uint64_t> rbv(L.row_bytes, L.row_bytes + MOE_NUM_TENSORS), dstv(L.dst, L.dst + MOE_NUM_TENSORS);
    const int dev = g_dev;
    for (size_t i = 0; i < b->reads.size(); ++i) b->reads[i].tag = (int)i;   // tag = piece index
    b->on_read = [=](int tag) -> int {
        if (hipSetDevice(dev) != hipSuccess) return -1;
        const Piece& pc = pieces[tag];
        const uint64_t rb = rbv[pc.t];
        const int first = runs[pc.run].first, len = runs[pc.run].second;
        for (int i = 0; i < len;) {                     // one copy per run of consecutive slots
            int r = 1;
            while (i + r < len && sorted[first + i + r].second == sorted[first + i].second + r) ++r;
            if (hipMemcpyAsync((void*)(dstv[pc.t] + (uint64_t)sorted[first + i].second * rb),
                               bounce + pc.boff + pc.skip + (uint64_t)i * rb, (uint64_t)r * rb,
                               hipMemcpyHostToDevice, g_copy) != hipSuccess)
                return -1;
            i += r;
        }
        return 0;
    };
    b->finish = [=]() -> int {
        if (hipSetDevice(dev) != hipSuccess) return -1;
        if (hipEventRecord(copy_done, g_copy) != hipSuccess) return -1;
        if (hipEventRecord(free_ev, g_copy) != hipSuccess) return -1;
        if (prefetch && hipEventRecord(pf_done, g_copy) != hipSuccess) return -1;
        return 0;
    };
    B.user = b;
    b->after = L.fbatch;
    L.fbatch = b;
    if (prefetch) L.fpf = b;
    fileio::submit(b);
    return 0;
}

// Queue the copies store[eid] -> pool[slot] for every tensor on the copy stream.  A prefetch's
// copies also record pf_done.
//
// Ordering between batches of one layer: copies on g_copy run in queue order, and each batch
// joins its g_copy_more copies into g_copy before copy_done is recorded.  A copy on g_copy_more
// is ordered after nothing on g_copy, so when this batch writes a slot that an earlier batch's
// copy may still be writing (a demand victim that a prefetch is filling, or a prefill chunk's
// load after an in-flight prefetch), the g_copy_more streams first wait for that batch.
// The layer's tensors as one StageSet over the device-visible store, when every tensor that is
// copied has one (a pinned store) and whole 16-byte units.
bool cu_stage_set(const LayerState& L, StageSet& S) {
    S = {};
    uint64_t units = 0;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        const uint64_t rb = L.row_bytes[t];
        if (!rb || !L.src[t] || !L.dst[t]) continue;
        if (!L.dev_src[t] || rb % 16) return false;
        S.src[S.n] = (const uint8_t*)L.dev_src[t];
        S.dst[S.n] = (uint8_t*)L.dst[t];
        S.src_stride[S.n] = S.dst_stride[S.n] = rb;
        S.first[S.n] = (uint32_t)units;
        units += rb / 16;
        ++S.n;
    }
    if (S.n == 0 || units > 0xFFFFFFFFull) return false;
    S.total = (uint32_t)units;
    return true;
}

// cu_copy: a pinned store's copies run as one CU copy kernel on g_copy (k_stage_pairs) instead of
// DMA requests, for the synchronous loads of a prefill chunk (tens of experts, each a ~1 MB run).
int issue_copies(int layer, LayerState& L, const int32_t* eids, const int32_t* slots, int n,
                 bool prefetch = false, bool cu_copy = false) {
    if (n <= 0) return 0;
    bool any = false;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) any |= (L.row_bytes[t] && L.src[t] && L.dst[t]);
    if (!any) return 0;                       // accounting-only layer
    if (g_acct_on) {
        uint64_t b = 0;
        for (int t = 0; t < MOE_NUM_TENSORS; ++t)
            if (L.row_bytes[t] && L.src[t] && L.dst[t]) b += L.row_bytes[t];
        g_tok[slot_host::AC_BYTES] += (uint64_t)n * b;
    }
    if (ensure_runtime()) return -1;
    if (ensure_events(L)) return -1;
    settle_copies(L);
    bool overlap = false;
    if (L.inflight)
        for (int i = 0; i < n && !overlap; ++i) overlap = (L.inflight_slots[slots[i] >> 6] >> (slots[i] & 63)) & 1u;
    if (L.read_recorded) HIP_TRY(hipStreamWaitEvent(g_copy, L.read_done, 0));
    StageSet S;
    if (L.fd >= 0) {
        if (issue_file_batch(L, eids, slots, n, prefetch)) return -1;
    } else if (cu_copy && cu_stage_set(L, S)) {
        // g_copy runs in queue order after the layer's earlier batches (their g_copy_more copies
        // were joined into g_copy) and after read_done
        if (launch_stage_pairs(eids, slots, n, S, g_copy)) return -1;
    } else {
        for (int i = 0; i < kCopyStreams - 1; ++i) {
            if (L.read_recorded) HIP_TRY(hipStreamWaitEvent(g_copy_more[i], L.read_done, 0));
            if (overlap) HIP_TRY(hipStreamWaitEvent(g_copy_more[i], L.copy_done, 0));
        }
        // Consecutive pairs whose expert ids and slots both step by one are contiguous in the
        // store and in the pool: one copy each run (a prefill chunk's ranked load list is mostly
        // such runs; one large copy moves ~57 GB/s).
        int c = 0;
        for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
            uint64_t rb = L.row_bytes[t];
            if (!rb || !L.src[t] || !L.dst[t]) continue;
            for (int i = 0; i < n; ++c) {
                int r = 1;
                while (i + r < n && eids[i + r] == eids[i] + r && slots[i + r] == slots[i] + r) ++r;
                HIP_TRY(hipMemcpyAsync((void*)(L.dst[t] + (uint64_t)slots[i] * rb),
                                       (const void*)(L.src[t] + (uint64_t)eids[i] * rb), (uint64_t)r * rb,
                                       hipMemcpyHostToDevice,
                                       c % kCopyStreams ? g_copy_more[c % kCopyStreams - 1] : g_copy));
                i += r;
            }
        }
        for (int i = 0; i < kCopyStreams - 1 && i + 1 < c; ++i) {
            HIP_TRY(hipEventRecord(g_copy_more_done[i], g_copy_more[i]));
            HIP_TRY(hipStreamWaitEvent(g_copy, g_copy_more_done[i], 0));
        }
    }
    if (L.fd < 0) {
        HIP_TRY(hipEventRecord(L.copy_done, g_copy));
        if (prefetch) HIP_TRY(hipEventRecord(L.pf_done, g_copy));
    }
    L.copy_pending = true;
    L.inflight = true;
    for (int i = 0; i < n; ++i) L.inflight_slots[slots[i] >> 6] |= 1ull << (slots[i] & 63);
    if (prefetch) L.pf_pending = true;
    (void)layer;
    return 0;
}

int wait_copies_gpu(LayerState& L, hipStream_t s) {
    if (!L.copy_pending) return 0;
    if (join_file(L)) return -1;
    HIP_TRY(hipStreamWaitEvent(s, L.copy_done, 0));
    L.copy_pending = false;
    L.pf_pending = false;
    return 0;
}

// SwitchGLU over a layer's pool in its format (blob or 9 tensors).
int layer_glu(const LayerState& L, const void* x, const uint32_t* slots, const void* scores, int k,
              const void* residual, void* h_ws, float* y_out, int per_expert, hipStream_t s) {
    if (L.fmt9) {
        if (launch_q2t_gate_up((const __half*)x, L.E9, L.capacity, slots, k, L.hidden, L.inter, (__half*)h_ws, s)) return -1;
        return launch_q2t_down((const __half*)h_ws, L.E9, L.capacity, slots, (const __half*)scores, k, L.hidden, L.inter,
                               (const __half*)residual, y_out, per_expert, s);
    }
    return moe_q2_switch_glu(x, (const void*)L.dst[0], L.row_bytes[0], L.capacity, slots, scores, k, L.hidden, L.inter,
                             L.group, residual, h_ws, y_out, per_expert, s);
}

int write_slot_inds(LayerState& L, const uint32_t* slots, int k) {
    if (!L.slot_inds) return 0;
    if (L.slot_inds_device) return launch_store_u32(L.slot_inds, slots, k, g_compute);
    memcpy(L.slot_inds, slots, (size_t)k * sizeof(uint32_t));
    return 0;
}

// Input checks of a decode step (the reference indexes its tables with the ids unchecked).
bool check_step_ids(const char* who, const LayerState& L, const uint32_t* eids, int k) {
    if (!L.init) { moe_set_error("%s: layer not initialised", who); return false; }
    if (k <= 0 || k > MOE_MAX_K || k > L.capacity) {
        moe_set_error("%s: k=%d must be in 1..%d and <= capacity %d", who, k, MOE_MAX_K, L.capacity);
        return false;
    }
    for (int i = 0; i < k; ++i) {
        if (eids[i] >= MOE_NUM_EXPERTS) { moe_set_error("%s: expert id %u out of range", who, eids[i]); return false; }
        for (int j = 0; j < i; ++j)
            if (eids[j] == eids[i]) { moe_set_error("%s: expert id %u repeated", who, eids[i]); return false; }
    }
    return true;
}

int step_host(int layer, const uint32_t* eids, int k, int async_io) {
    LayerState& L = g_layers[layer];
    if (!check_step_ids("step", L, eids, k)) return -1;
    if (pull_table(L)) return -1;
    uint32_t out[MOE_MAX_K];
    slot_host::Acct acct;
    int n_miss = slot_host::step(&L.tab, eids, k, out, nullptr, nullptr, acct_for(L, acct));
    if (push_table(L)) return -1;
    if (write_slot_inds(L, out, k)) return -1;
    if (issue_copies(layer, L, L.tab.copy_eid, L.tab.copy_slot, L.tab.n_copy)) return -1;
    if (!async_io && drain_copies(L)) return -1;
    return n_miss;
}

// ---- kernel timing -------------------------------------------------------------------------
struct KtSlot { int kind; hipEvent_t start, stop; };
std::vector<KtSlot> g_kt;                    // event pool (grows to the requested capacity)
size_t g_kt_used = 0, g_kt_cap = 0;
bool g_kt_on = false;

}  // namespace

bool kt_enabled() { return g_kt_on; }

void kt_events(int kind, hipEvent_t* start, hipEvent_t* stop) {
    *start = *stop = nullptr;
    if (g_kt_used >= g_kt_cap) return;
    KtSlot& k = g_kt[g_kt_used++];
    k.kind = kind;
    *start = k.start;
    *stop = k.stop;
}

void moe_set_error(const char* fmt, ...) {
    std::lock_guard<std::mutex> g(g_err_mu);
    if (g_err[0]) return;                     // keep the first failure
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" {

// ---- errors, streams, host memory ---------------------------------------------------------

const char* c_last_error(void) { return g_err; }

void c_clear_error(void) {
    std::lock_guard<std::mutex> g(g_err_mu);
    g_err[0] = 0;
}

int c_set_compute_stream(void* stream) {
    g_compute = (hipStream_t)stream;
    return 0;
}

void* c_host_alloc(uint64_t bytes) {
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, (size_t)bytes, hipHostMallocMapped);
    if (e != hipSuccess) {
        moe_set_error("hipHostMalloc(%llu) -> %s", (unsigned long long)bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

int c_host_free(void* p) {
    if (p) HIP_TRY(hipHostFree(p));
    return 0;
}

// ---- expert_io.c entry points ---------------------------------------------------------------

void c_io_init(int num_threads) {
    // Reader threads of file-backed layers (<= 0: 8); copies from host memory are queued to the DMA
    // engines.  The copy streams are created on first use so that accounting-only tables work
    // without a GPU.
    fileio::set_threads(num_threads);
}

// Read file-backed layers initialised from now on with O_DIRECT (on != 0) or through the page
// cache (0, the default).  A file system that refuses O_DIRECT leaves the layer on the page cache.
void c_io_set_direct(int on) { g_direct = on != 0; }

// 1 when the layer reads its file with O_DIRECT.
int c_layer_io_direct(int layer) { return valid_layer(layer) && g_layers[layer].fd_direct >= 0 ? 1 : 0; }

// Reader threads of the file tier.
int c_io_threads(void) { return fileio::threads(); }

// Read n ranges of a file into host memory with the reader threads (blocking): range i is
// lens[i] bytes at offs[i] into the address dsts[i].  Host code only (no GPU needed); used to fill
// host expert stores from a shard.  0, or -1 on a failed or short read.
int c_io_read_ranges(int fd, const uint64_t* offs, const uint64_t* lens, const uint64_t* dsts, int n) {
    if (n < 0 || (n > 0 && (!offs || !lens || !dsts))) { moe_set_error("io_read_ranges: bad arguments"); return -1; }
    auto b = std::make_shared<fileio::Batch>();
    for (int i = 0; i < n; ++i)
        if (lens[i]) b->reads.push_back(fileio::Read{fd, offs[i], lens[i], lens[i], (uint8_t*)dsts[i]});
    fileio::submit(b);
    std::string msg;
    if (fileio::wait(b, msg)) { moe_set_error("io_read_ranges: %s", msg.c_str()); return -1; }
    return 0;
}

void c_io_shutdown(void) {
    for (int l = 0; l < MOE_MAX_LAYERS; ++l)
        if (filefeed::attached(l)) {          // device-driven file layers: their staging kernels
            (void)hipDeviceSynchronize();     // wait on the feeder, so they end first
            break;
        }
    filefeed::shutdown();
    for (int l = 0; l < MOE_MAX_LAYERS; ++l) (void)join_file(g_layers[l]);
    fileio::shutdown();
    if (!g_ready) return;
    (void)hipStreamSynchronize(g_copy);
    release_bounce();
    for (int l = 0; l < MOE_MAX_LAYERS; ++l) {
        LayerState& L = g_layers[l];
        release_file(L);
        if (L.dtab) (void)hipFree(L.dtab);
        if (L.copy_done) (void)hipEventDestroy(L.copy_done);
        if (L.read_done) (void)hipEventDestroy(L.read_done);
        if (L.pf_done) (void)hipEventDestroy(L.pf_done);
        if (L.split_dev) (void)hipFree(L.split_dev);
        L = LayerState();
    }
    for (int i = 0; i < kCopyStreams - 1; ++i) {
        (void)hipStreamSynchronize(g_copy_more[i]);
        (void)hipStreamDestroy(g_copy_more[i]);
        (void)hipEventDestroy(g_copy_more_done[i]);
        g_copy_more[i] = nullptr;
        g_copy_more_done[i] = nullptr;
    }
    (void)hipStreamDestroy(g_copy);
    g_copy = nullptr;
    g_ready = false;
}

void c_layer_reset_cache(int layer) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    if (pull_table(L)) return;
    slot_host::reset_cache(&L.tab);
    reset_evictions(L);
    if (layer == 1) {                         // layer 1's reset restarts the token numbering
        g_token_seq = 0;
        g_cur_token = -1;
        L.tab.acct_token = -1;
        L.tab.acct_seq = 0;
    }
    if (push_table(L)) return;
    if (layer == 1) {                         // ... of the device-driven tables too
        const TableSet ts = device_tables();
        if (ts.n && launch_acct_ctl(ts, 3, g_compute) == 0) (void)hipStreamSynchronize(g_compute);
    }
}

void c_layer_reset_stats(int layer) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    if (pull_table(L)) return;
    slot_host::reset_stats(&L.tab);
    push_table(L);
}

void c_layer_init(int layer, int fd, int capacity, const uint64_t* base_offsets, const uint64_t* row_bytes,
                  const uint64_t* base_ptrs, uint64_t slot_inds_ptr) {
    if (!valid_layer(layer)) return;
    if (capacity < 1 || capacity > MOE_NUM_EXPERTS) {
        moe_set_error("c_layer_init: capacity %d out of range 1..%d", capacity, MOE_NUM_EXPERTS);
        return;
    }
    LayerState& L = g_layers[layer];
    if (filefeed::attached(layer)) {
        (void)hipDeviceSynchronize();         // its staging kernels wait on the feeder
        filefeed::detach(layer);
    }
    (void)join_file(L);
    if (L.inflight) (void)hipEventSynchronize(L.copy_done);
    release_file(L);
    if (L.dtab) (void)hipFree(L.dtab);
    hipEvent_t cd = L.copy_done, rd = L.read_done, pd = L.pf_done;
    uint8_t* sd = L.split_dev;
    L = LayerState();
    L.copy_done = cd;
    L.read_done = rd;
    L.pf_done = pd;
    L.split_dev = sd;
    reset_evictions(L);
    if (layer == 1) {
        g_token_seq = 0;
        g_cur_token = -1;
    }
    L.fd = fd;
    if (fd >= 0 && g_direct) {                // a second descriptor of the same file, page cache bypassed
        char path[64];
        snprintf(path, sizeof(path), "/proc/self/fd/%d", fd);
        L.fd_direct = open(path, O_RDONLY | O_DIRECT | O_CLOEXEC);
    }
    L.capacity = capacity;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        L.src[t] = base_offsets ? base_offsets[t] : 0;
        L.row_bytes[t] = row_bytes ? row_bytes[t] : 0;
        L.dst[t] = base_ptrs ? base_ptrs[t] : 0;
        L.dev_src[t] = 0;
        if (fd < 0 && L.src[t]) {
            void* dp = nullptr;
            if (hipHostGetDevicePointer(&dp, (void*)L.src[t], 0) == hipSuccess) L.dev_src[t] = (uint64_t)dp;
            else (void)hipGetLastError();
        }
    }
    L.slot_inds = (uint32_t*)slot_inds_ptr;
    L.slot_inds_device = false;
    if (L.slot_inds) {
        hipPointerAttribute_t a;
        if (hipPointerGetAttributes(&a, L.slot_inds) == hipSuccess) L.slot_inds_device = (a.type == hipMemoryTypeDevice);
        else (void)hipGetLastError();
    }
    slot_host::init(&L.tab, capacity, expert_bytes_of(L));
    L.init = true;
}

int c_layer_step_decode_ex(int layer, const uint32_t* eids, int k, int async_io) {
    if (!valid_layer(layer)) return 0;
    return step_host(layer, eids, k, async_io);
}

int c_layer_step_decode(int layer, const uint32_t* eids, int k) {
    return c_layer_step_decode_ex(layer, eids, k, 0);
}

int c_layer_step_decode10(int layer, uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, uint32_t e4,
                          uint32_t e5, uint32_t e6, uint32_t e7, uint32_t e8, uint32_t e9) {
    uint32_t e[10] = {e0, e1, e2, e3, e4, e5, e6, e7, e8, e9};
    return c_layer_step_decode_ex(layer, e, 10, 0);
}

int c_layer_step_decode10_async(int layer, uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, uint32_t e4,
                                uint32_t e5, uint32_t e6, uint32_t e7, uint32_t e8, uint32_t e9) {
    uint32_t e[10] = {e0, e1, e2, e3, e4, e5, e6, e7, e8, e9};
    return c_layer_step_decode_ex(layer, e, 10, 1);
}

void c_layer_start_prefetch(int layer, const int32_t* preds, int n, int max_fetch) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    if (!L.init) { moe_set_error("layer %d not initialised", layer); return; }
    if (n < 0 || n > MOE_MAX_PREFETCH) { moe_set_error("prefetch: %d predictions (max %d)", n, MOE_MAX_PREFETCH); return; }
    if (pull_table(L)) return;
    slot_host::Acct acct;
    slot_host::prefetch(&L.tab, preds, n, max_fetch, false, acct_for(L, acct));
    if (push_table(L)) return;
    issue_copies(layer, L, L.tab.pf_copy_eid, L.tab.pf_copy_slot, L.tab.pf_n_copy, true);
}

void c_layer_start_prefetch10(int layer, int max_fetch, int32_t e0, int32_t e1, int32_t e2, int32_t e3,
                              int32_t e4, int32_t e5, int32_t e6, int32_t e7, int32_t e8, int32_t e9) {
    int32_t p[10] = {e0, e1, e2, e3, e4, e5, e6, e7, e8, e9};
    c_layer_start_prefetch(layer, p, 10, max_fetch);
}

void c_layer_start_prefetch12(int layer, int max_fetch, int32_t e0, int32_t e1, int32_t e2, int32_t e3,
                              int32_t e4, int32_t e5, int32_t e6, int32_t e7, int32_t e8, int32_t e9,
                              int32_t e10, int32_t e11) {
    int32_t p[12] = {e0, e1, e2, e3, e4, e5, e6, e7, e8, e9, e10, e11};
    c_layer_start_prefetch(layer, p, 12, max_fetch);
}

void c_layer_wait_prefetch(int layer) {
    (void)layer;                              // joins every layer's in-flight copies
    for (int l = 0; l < MOE_MAX_LAYERS; ++l)
        if (g_layers[l].init) wait_copies_gpu(g_layers[l], g_compute);
}

void c_layer_load_sync(int layer, const int32_t* eids, const int32_t* slots, int n, int is_prefill) {
    if (!valid_layer(layer) || n <= 0) return;
    LayerState& L = g_layers[layer];
    if (!L.init) { moe_set_error("layer %d not initialised", layer); return; }
    for (int i = 0; i < n; ++i)
        if (eids[i] < 0 || eids[i] >= MOE_NUM_EXPERTS || slots[i] < 0 || slots[i] >= L.capacity) {
            moe_set_error("load_sync: pair (%d, %d) out of range", eids[i], slots[i]);
            return;
        }
    if (pull_table(L)) return;
    if (is_prefill) L.tab.stats[ST_PRE_BYTES] += (uint64_t)n * L.tab.expert_bytes;
    slot_host::count_runs(&L.tab, eids, n);
    if (push_table(L)) return;
    // Copied one after the other, the last pair naming a slot decides what it holds; the copies
    // here run concurrently, so only that pair is copied.
    std::vector<int32_t> ce, cs;
    ce.reserve(n);
    cs.reserve(n);
    uint64_t seen[MOE_NUM_EXPERTS / 64] = {};
    for (int i = n - 1; i >= 0; --i) {
        uint64_t& w = seen[slots[i] >> 6];
        const uint64_t bit = 1ull << (slots[i] & 63);
        if (w & bit) continue;
        w |= bit;
        ce.push_back(eids[i]);
        cs.push_back(slots[i]);
    }
    std::reverse(ce.begin(), ce.end());
    std::reverse(cs.begin(), cs.end());
    if (issue_copies(layer, L, ce.data(), cs.data(), (int)ce.size(), false, true)) return;
    if (drain_copies(L)) return;
    wait_copies_gpu(L, g_compute);
}

void c_layer_get_lru_state(int layer, int32_t* out_eids, int32_t* out_slots, int* out_count) {
    if (!valid_layer(layer)) { *out_count = 0; return; }
    LayerState& L = g_layers[layer];
    if (pull_table(L)) { *out_count = 0; return; }
    *out_count = slot_host::get_state(&L.tab, out_eids, out_slots);
}

void c_layer_set_lru_state(int layer, const int32_t* eids, const int32_t* slots, int n, uint64_t add_req,
                           uint64_t add_hits, uint64_t add_miss) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    for (int i = 0; i < n; ++i)
        if (eids[i] < 0 || eids[i] >= MOE_NUM_EXPERTS || slots[i] < 0 || slots[i] >= L.capacity) {
            moe_set_error("set_lru_state: pair (%d, %d) out of range", eids[i], slots[i]);
            return;
        }
    if (pull_table(L)) return;
    slot_host::set_state(&L.tab, eids, slots, n, add_req, add_hits, add_miss);
    for (int i = 0; i < n; ++i) L.tab.evicted_at[eids[i]] = -1;
    push_table(L);
}

void c_layer_get_stats(int layer, uint64_t* out) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    if (pull_table(L)) return;
    memcpy(out, L.tab.stats, sizeof(L.tab.stats));
}

void c_get_decode_totals(int num_layers, uint64_t* out6) {
    uint64_t t[6] = {0};
    if (num_layers > MOE_MAX_LAYERS) num_layers = MOE_MAX_LAYERS;
    for (int l = 1; l < num_layers; ++l) {
        LayerState& L = g_layers[l];
        if (!L.init) continue;
        if (pull_table(L)) break;
        const uint64_t* st = L.tab.stats;
        t[0] += st[ST_DEC_LRU_HIT];
        t[1] += st[ST_DEC_PREF_HIT];
        t[2] += st[ST_DEC_MISS];
        t[3] += st[ST_DEC_REQ];
        t[4] += st[ST_DEC_BYTES];
        t[5] += st[ST_PREF_BYTES];
    }
    memcpy(out6, t, sizeof(t));
}

// ---- scheduler variant and per-token accounting (cpp/third_party/expert_io.c) --------------

// GPU-side join of a layer's copies: the compute stream waits for every copy queued for the
// layer (its prefetch and its demand misses) before later work reads the pool.
void c_layer_wait_demand(int layer) {
    if (!valid_layer(layer) || !g_layers[layer].init) return;
    wait_copies_gpu(g_layers[layer], g_compute);
}

int c_layer_decode_step_sched(int layer, const int32_t* eids, int k, const int32_t* pred, int n_pred, int next_layer,
                              int prefetch_cap, int flags) {
    int n_miss = 0;
    // 1: the step of `layer` (layer 0 is resident and never stepped)
    if (layer > 0 && layer < MOE_MAX_LAYERS && eids && k > 0) {
        if (k > MOE_MAX_K) k = MOE_MAX_K;
        LayerState& L = g_layers[layer];
        if (!check_step_ids("decode_step_sched", L, reinterpret_cast<const uint32_t*>(eids), k)) return -1;
        if (pull_table(L)) return -1;
        uint64_t extra[8] = {0};
        if (L.tab.snap_valid) memcpy(extra, L.tab.snap_fetched, sizeof(extra));
        uint32_t out[MOE_MAX_K];
        uint8_t hit[MOE_MAX_K];
        slot_host::Acct acct;
        n_miss = slot_host::step(&L.tab, reinterpret_cast<const uint32_t*>(eids), k, out, extra, hit,
                                 acct_for(L, acct));
        if (push_table(L)) return -1;
        if (write_slot_inds(L, out, k)) return -1;
        if ((flags & MOE_SCHED_SPLIT) && n_miss > 0 && n_miss < k) {
            SplitLists& S = g_split[layer];
            const int n_hit = k - n_miss;
            int h = 0, m = 0;
            for (int i = 0; i < k; ++i) {
                if (hit[i]) { S.hit[h] = out[i]; S.inv[i] = h++; }
                else { S.miss[m] = out[i]; S.inv[i] = n_hit + m++; }
            }
            S.n_hit = n_hit;
            S.n_miss = n_miss;
            S.k = k;
        }
        if (issue_copies(layer, L, L.tab.copy_eid, L.tab.copy_slot, L.tab.n_copy)) return -1;
    }
    // 2: the prefetch of `next_layer`, queued behind the demand copies
    if (!(flags & MOE_SCHED_NO_PREFETCH) && next_layer > 0 && next_layer < MOE_MAX_LAYERS && pred && n_pred > 0 &&
        prefetch_cap > 0) {
        LayerState& N = g_layers[next_layer];
        if (!N.init) { moe_set_error("decode_step_sched: next layer %d not initialised", next_layer); return -1; }
        if (pull_table(N)) return -1;
        slot_host::Acct acct;
        slot_host::prefetch(&N.tab, pred, n_pred, prefetch_cap, true, acct_for(N, acct));
        if (push_table(N)) return -1;
        if (issue_copies(next_layer, N, N.tab.pf_copy_eid, N.tab.pf_copy_slot, N.tab.pf_n_copy, true)) return -1;
    }
    // 3: joins.  SYNC_DEMAND blocks the host until the layer's copies have landed; with no miss
    // the layer's (prefetch) copies are joined on the GPU so the GEMV needs no further call.
    if (layer > 0 && layer < MOE_MAX_LAYERS && g_layers[layer].init) {
        LayerState& L = g_layers[layer];
        if (flags & MOE_SCHED_SYNC_DEMAND) {
            if (drain_copies(L)) return -1;
            wait_copies_gpu(L, g_compute);
        } else if (n_miss == 0) {
            wait_copies_gpu(L, g_compute);
        }
    }
    return n_miss;
}

void c_layer_get_split_inds(int layer, uint32_t* out_hit_slots, uint32_t* out_miss_slots, int32_t* out_inv_order) {
    if (!valid_layer(layer)) return;
    LayerState& L = g_layers[layer];
    if (L.device_mode && pull_table(L)) return;
    const SplitLists& S = L.device_mode ? L.tab.split : g_split[layer];
    if (S.n_hit > 0 && out_hit_slots) memcpy(out_hit_slots, S.hit, (size_t)S.n_hit * sizeof(uint32_t));
    if (S.n_miss > 0 && out_miss_slots) memcpy(out_miss_slots, S.miss, (size_t)S.n_miss * sizeof(uint32_t));
    if (S.k > 0 && out_inv_order) memcpy(out_inv_order, S.inv, (size_t)S.k * sizeof(int32_t));
}

// Device-driven tables count on the device: these queue small control kernels on the compute
// stream (so a captured token replays them), and c_end_decode_token adds the tables' counters.
void c_set_io_accounting(int enabled) {
    g_acct_on = enabled != 0;
    if (!g_acct_on) g_cur_token = -1;
    const TableSet ts = device_tables();
    if (ts.n) (void)launch_acct_ctl(ts, g_acct_on ? 1 : 0, g_compute);
}

void c_begin_decode_token(int token_idx) {
    (void)token_idx;                          // tokens are numbered by the library, as in the reference
    g_cur_token = g_token_seq++;
    memset(g_tok, 0, sizeof(g_tok));
    const TableSet ts = device_tables();
    if (ts.n) (void)launch_acct_ctl(ts, 2, g_compute);
}

void c_end_decode_token(uint64_t* out10) {
    memcpy(out10, g_tok, sizeof(g_tok));
    const TableSet ts = device_tables();
    if (!ts.n) return;
    static uint64_t* sums = nullptr;          // 10 device counters, kept until the process ends
    if (!sums && hipMalloc((void**)&sums, 10 * sizeof(uint64_t)) != hipSuccess) {
        moe_set_error("end_decode_token: no device memory for the sums");
        sums = nullptr;
        return;
    }
    uint64_t dev[10];
    if (launch_acct_sum(ts, sums, g_compute) ||
        hipMemcpyAsync(dev, sums, sizeof(dev), hipMemcpyDeviceToHost, g_compute) != hipSuccess ||
        hipStreamSynchronize(g_compute) != hipSuccess) {
        moe_set_error("end_decode_token: reading the device tables' counters failed");
        return;
    }
    for (int i = 0; i < 10; ++i) out10[i] += dev[i];
}

uint64_t c_get_native_buffer_bytes(void) {
    uint64_t b = sizeof(g_layers) + sizeof(g_split);
    for (int l = 0; l < MOE_MAX_LAYERS; ++l) {
        if (g_layers[l].dtab) b += sizeof(SlotTable);
    }
    for (const Bounce& bb : g_bounce) b += bb.bytes;
    return b;
}

int c_layer_set_sched(int layer, int on) {
    if (!valid_layer(layer) || !g_layers[layer].init) { moe_set_error("set_sched: bad layer %d", layer); return -1; }
    LayerState& L = g_layers[layer];
    if (pull_table(L)) return -1;
    L.tab.sched = on & 3;                     // bit 0 the variant, bit 1 device split lists
    return push_table(L);
}

// ---- device-driven slot tables ----------------------------------------------------------------

int c_layer_set_device_mode(int layer, int on) {
    if (!valid_layer(layer) || !g_layers[layer].init) { moe_set_error("set_device_mode: bad layer %d", layer); return -1; }
    LayerState& L = g_layers[layer];
    if (on && !L.device_mode) {
        for (int t = 0; t < MOE_NUM_TENSORS && L.fd < 0; ++t)
            if (L.row_bytes[t] && L.src[t] && L.dst[t] && !L.dev_src[t]) {
                moe_set_error("device-driven staging: tensor %d store is not pinned host memory", t);
                return -1;
            }
        if (!L.slot_inds || !L.slot_inds_device) { moe_set_error("device-driven layers need a device slot_inds buffer"); return -1; }
        if (L.fd >= 0) {                      // file-backed: misses published to the feeder
            if (drain_copies(L)) return -1;
            filefeed::LayerIO io;
            io.fd = L.fd;
            io.fd_direct = L.fd_direct;
            for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
                io.src[t] = L.src[t];
                io.row_bytes[t] = L.row_bytes[t];
                io.dst[t] = L.dst[t];
            }
            if (filefeed::attach(layer, io)) return -1;
        }
        if (!L.dtab) HIP_TRY(hipMalloc((void**)&L.dtab, sizeof(SlotTable)));
        // per-token accounting now runs on the device: the open token, the switch, and the bytes
        // a copied expert moves (none for an accounting-only layer)
        L.tab.acct_on = g_acct_on ? 1 : 0;
        L.tab.acct_token = g_cur_token;
        L.tab.acct_seq = g_token_seq;
        L.tab.stage_bytes = 0;
        for (int t = 0; t < MOE_NUM_TENSORS; ++t)
            if (L.row_bytes[t] && L.src[t] && L.dst[t]) L.tab.stage_bytes += L.row_bytes[t];
        L.device_mode = true;
        return push_table(L);
    }
    if (!on && L.device_mode) {
        if (L.fd >= 0) {
            HIP_TRY(hipDeviceSynchronize());  // staging kernels still waiting on the feeder end first
            filefeed::detach(layer);
        }
        if (pull_table(L)) return -1;
        L.device_mode = false;
    }
    return 0;
}

uint64_t c_layer_device_table(int layer) {
    if (!valid_layer(layer)) return 0;
    return (uint64_t)g_layers[layer].dtab;
}

static int stage_device(int layer, LayerState& L, int list, hipStream_t s, int ctas) {
    if (L.fd >= 0) return filefeed::stage(layer, list, L.dtab, ctas, s);
    StageSet S = {};
    uint64_t units = 0;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        const uint64_t rb = L.row_bytes[t];
        if (!rb || !L.dev_src[t] || !L.dst[t]) continue;
        if (rb % 16) { S.n = 0; break; }              // (the per-tensor kernel reports it)
        S.src[S.n] = (const uint8_t*)L.dev_src[t];
        S.dst[S.n] = (uint8_t*)L.dst[t];
        S.src_stride[S.n] = S.dst_stride[S.n] = rb;
        S.first[S.n] = (uint32_t)units;
        units += rb / 16;
        ++S.n;
    }
    if (S.n > 1 && units <= 0xFFFFFFFFull) {          // several tensors: one launch for all of them
        S.total = (uint32_t)units;
        return launch_stage_set(L.dtab, list, S, ctas, s);
    }
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        uint64_t rb = L.row_bytes[t];
        if (!rb || !L.dev_src[t] || !L.dst[t]) continue;
        if (launch_stage(L.dtab, list, (const uint8_t*)L.dev_src[t], rb, (uint8_t*)L.dst[t], rb, rb, ctas, s)) return -1;
    }
    return 0;
}

// stage_ctas < 0: update the table only (the copies are queued later with c_layer_stage_dev).
int c_layer_step_decode_dev(int layer, const uint32_t* ids_dev, int k, int stage_ctas, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].device_mode) {
        moe_set_error("step_decode_dev: layer %d is not a device-driven layer", layer);
        return -1;
    }
    LayerState& L = g_layers[layer];
    if (k <= 0 || k > MOE_MAX_K || k > L.capacity) { moe_set_error("step_decode_dev: k=%d out of range", k); return -1; }
    hipStream_t s = (hipStream_t)stream;
    if (launch_slot_step(L.dtab, ids_dev, k, L.slot_inds, s)) return -1;
    filefeed::mark_table_op(layer, 0);
    if (stage_ctas < 0) return 0;
    if (L.fd >= 0 && filefeed::publish(layer, 0, L.dtab, s)) return -1;
    return stage_device(layer, L, 0, s, stage_ctas);
}

int c_layer_start_prefetch_dev(int layer, const int32_t* preds_dev, int m, int max_fetch, int stage_ctas,
                               void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].device_mode) {
        moe_set_error("start_prefetch_dev: layer %d is not a device-driven layer", layer);
        return -1;
    }
    LayerState& L = g_layers[layer];
    hipStream_t s = (hipStream_t)stream;
    if (launch_slot_prefetch(L.dtab, preds_dev, m, max_fetch, s)) return -1;
    filefeed::mark_table_op(layer, 1);
    if (stage_ctas < 0) return 0;
    if (L.fd >= 0 && filefeed::publish(layer, 1, L.dtab, s)) return -1;
    return stage_device(layer, L, 1, s, stage_ctas);
}

// Queue the copies listed by the layer's last device-side decode step (list 0) or prefetch
// (list 1).
int c_layer_stage_dev(int layer, int list, int stage_ctas, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].device_mode) {
        moe_set_error("stage_dev: layer %d is not a device-driven layer", layer);
        return -1;
    }
    if (list != 0 && list != 1) { moe_set_error("stage_dev: list %d (0 = decode step, 1 = prefetch)", list); return -1; }
    return stage_device(layer, g_layers[layer], list, (hipStream_t)stream, stage_ctas < 0 ? 0 : stage_ctas);
}

// File-backed device-driven layers: hand the list of the layer's last device-side decode step
// (list 0) or prefetch (list 1) to the feeder thread, which reads those experts into the layer's
// bounce entries while the stream goes on; c_layer_stage_dev then waits for each entry and copies
// it into its slot.
int c_layer_publish_dev(int layer, int list, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].device_mode || g_layers[layer].fd < 0) {
        moe_set_error("publish_dev: layer %d is not a device-driven file-backed layer", layer);
        return -1;
    }
    return filefeed::publish(layer, list, g_layers[layer].dtab, (hipStream_t)stream);
}

void c_io_set_feed_timeout_us(uint64_t us) { filefeed::set_timeout_us(us); }

int c_layer_table_status(int layer) {
    if (!valid_layer(layer)) return -1;
    LayerState& L = g_layers[layer];
    if (pull_table(L)) return -1;
    return L.tab.io_fault ? L.tab.io_fault : L.tab.status;   // a sticky file-tier fault first
}

int c_io_fault(void) { return filefeed::fault_word(); }

void c_io_clear_fault(void) { filefeed::clear_fault_word(); }

// ---- compute entry points ---------------------------------------------------------------------

uint64_t moe_router_workspace_bytes(int n_exp) { return (uint64_t)(2 * n_exp) * sizeof(float) + 256; }

int moe_router_logits(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out, const void* w,
                      int hidden, int n_exp, float* logits_out, void* stream) {
    return launch_router_logits(h_in, (const __half*)norm_w, eps, (const __half*)x_in, (__half*)x_out,
                                (const __half*)w, hidden, n_exp, logits_out, (hipStream_t)stream);
}

int moe_q2_gate_up_routed(const void* x, const float* logits, int n_exp, int k, const void* pool, uint64_t stride,
                          int hidden, int inter, int group, uint32_t* ids_out, void* scores_out, void* h_out,
                          void* stream) {
    return launch_q2_gate_up_routed((const __half*)x, logits, n_exp, k, (const uint8_t*)pool, stride, hidden, inter,
                                    group, ids_out, (__half*)scores_out, (__half*)h_out, (hipStream_t)stream);
}

int moe_router(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out, const void* w,
               const void* w_next, int hidden, int n_exp, int k, int m, void* workspace, uint32_t* ids_out,
               void* scores_out, int32_t* pred_out, void* stream) {
    float* scratch = (float*)workspace;
    unsigned* counter = (unsigned*)((uint8_t*)workspace + (size_t)(2 * n_exp) * sizeof(float));
    return launch_router(h_in, (const __half*)norm_w, eps, (const __half*)x_in, (__half*)x_out,
                         (const __half*)w, (const __half*)w_next, hidden, n_exp, k, m, scratch, counter,
                         ids_out, (__half*)scores_out, pred_out, nullptr, nullptr, nullptr, 0, (hipStream_t)stream);
}

int moe_router_noalloc(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out, const void* w,
                       const void* w_next, int hidden, int n_exp, int k, int m, uint32_t* ids_out, void* scores_out,
                       int32_t* pred_out, void* stream) {
    return launch_router_noalloc(h_in, (const __half*)norm_w, eps, (const __half*)x_in, (__half*)x_out,
                                 (const __half*)w, (const __half*)w_next, hidden, n_exp, k, m, ids_out,
                                 (__half*)scores_out, pred_out, (hipStream_t)stream);
}

// Router whose last block also runs the decode step of layer step_layer (its selected ids, slot
// ids into that layer's slot_inds) and the prefetch of layer pf_layer (the prediction); either
// layer may be -1.  Both must be device-driven layers.  Same decisions as
// c_layer_step_decode_dev + c_layer_start_prefetch_dev after moe_router.
int c_router_tables_dev(int step_layer, int pf_layer, int max_fetch, const float* h_in, const void* norm_w, float eps,
                        const void* x_in, void* x_out, const void* w, const void* w_next, int hidden, int n_exp, int k,
                        int m, void* workspace, uint32_t* ids_out, void* scores_out, int32_t* pred_out, void* stream) {
    SlotTable* st = nullptr;
    SlotTable* pt = nullptr;
    uint32_t* slots = nullptr;
    if (step_layer >= 0) {
        if (!valid_layer(step_layer) || !g_layers[step_layer].init || !g_layers[step_layer].device_mode) {
            moe_set_error("router_tables_dev: layer %d is not a device-driven layer", step_layer);
            return -1;
        }
        LayerState& L = g_layers[step_layer];
        if (k > L.capacity) { moe_set_error("router_tables_dev: k=%d > capacity %d", k, L.capacity); return -1; }
        if (!L.slot_inds || !L.slot_inds_device) {
            moe_set_error("router_tables_dev: layer %d slot_inds must be device memory", step_layer);
            return -1;
        }
        st = L.dtab;
        slots = L.slot_inds;
    }
    if (pf_layer >= 0) {
        if (!valid_layer(pf_layer) || !g_layers[pf_layer].init || !g_layers[pf_layer].device_mode) {
            moe_set_error("router_tables_dev: layer %d is not a device-driven layer", pf_layer);
            return -1;
        }
        if (!w_next || m <= 0) { moe_set_error("router_tables_dev: prefetch needs the next router and m > 0"); return -1; }
        pt = g_layers[pf_layer].dtab;
    }
    if (st && st == pt) {                  // two waves would race on one table
        moe_set_error("router_tables_dev: step and prefetch name the same layer %d", step_layer);
        return -1;
    }
    float* scratch = (float*)workspace;
    unsigned* counter = (unsigned*)((uint8_t*)workspace + (size_t)(2 * n_exp) * sizeof(float));
    if (launch_router(h_in, (const __half*)norm_w, eps, (const __half*)x_in, (__half*)x_out, (const __half*)w,
                      (const __half*)w_next, hidden, n_exp, k, m, scratch, counter, ids_out, (__half*)scores_out,
                      pred_out, st, slots, pt, max_fetch, (hipStream_t)stream))
        return -1;
    if (st) filefeed::mark_table_op(step_layer, 0);
    if (pt) filefeed::mark_table_op(pf_layer, 1);
    return 0;
}

int moe_f64_to_f16(const double* in, uint16_t* out, int n, void* stream) {
    return launch_f64_to_f16(in, out, n, (hipStream_t)stream);
}

int moe_rmsnorm(const float* h_in, const void* norm_w, float eps, int hidden, void* x_out, void* stream) {
    return launch_rmsnorm(h_in, (const __half*)norm_w, eps, hidden, (__half*)x_out, (hipStream_t)stream);
}

int moe_rmsnorm_bf16(const float* h_in, const void* norm_w, float eps, int hidden, void* x_bf16_out, void* x_f16_out,
                     void* stream) {
    return launch_rmsnorm_bf16(h_in, (const uint16_t*)norm_w, eps, hidden, (uint16_t*)x_bf16_out, (__half*)x_f16_out,
                               (hipStream_t)stream);
}

uint64_t moe_q2_expert_bytes(int hidden, int inter, int group) {
    return (uint64_t)blob_layout(hidden, inter, group).bytes;
}

int moe_q2_gate_up(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots, int k,
                   int hidden, int inter, int group, void* h_out, void* stream) {
    return launch_q2_gate_up((const __half*)x, (const uint8_t*)pool, stride, n_slots, slots, k, hidden, inter, group,
                             (__half*)h_out, (hipStream_t)stream);
}

int moe_q2_down(const void* h, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
                const void* scores, int k, int hidden, int inter, int group, const void* residual, float* y_out,
                int per_expert, void* stream) {
    return launch_q2_down((const __half*)h, (const uint8_t*)pool, stride, n_slots, slots, (const __half*)scores, k, hidden,
                          inter, group, (const __half*)residual, y_out, per_expert, (hipStream_t)stream);
}

int moe_q2_switch_glu(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
                      const void* scores, int k, int hidden, int inter, int group, const void* residual, void* h_ws,
                      float* y_out, int per_expert, void* stream) {
    if (moe_q2_gate_up(x, pool, stride, n_slots, slots, k, hidden, inter, group, h_ws, stream)) return -1;
    return moe_q2_down(h_ws, pool, stride, n_slots, slots, scores, k, hidden, inter, group, residual, y_out, per_expert,
                       stream);
}

int c_layer_set_format(int layer, int hidden, int inter, int group) {
    if (!valid_layer(layer) || !g_layers[layer].init) { moe_set_error("set_format: bad layer %d", layer); return -1; }
    LayerState& L = g_layers[layer];
    uint64_t want = blob_layout(hidden, inter, group).bytes;
    if (L.row_bytes[0] != want) {
        moe_set_error("set_format: tensor 0 row bytes %llu != Q2 blob bytes %llu", (unsigned long long)L.row_bytes[0],
                      (unsigned long long)want);
        return -1;
    }
    L.hidden = hidden;
    L.inter = inter;
    L.group = group;
    L.fmt9 = false;
    return 0;
}

// The layer's 9 tensors (c_layer_init order, which the reference sorts by file offset,
// loader.py:381-385) are the Q2 projections: roles[t] names tensor t (Q2T_* in moe_offload.h).
int c_layer_set_format9(int layer, int hidden, int inter, int group, const int32_t* roles, int scale_bf16) {
    if (!valid_layer(layer) || !g_layers[layer].init) { moe_set_error("set_format9: bad layer %d", layer); return -1; }
    if (!q2t_shape_ok("set_format9", 1, hidden, inter, group)) return -1;
    if (!roles) { moe_set_error("set_format9: null roles"); return -1; }
    LayerState& L = g_layers[layer];
    int tensor_of[9];
    for (int r = 0; r < 9; ++r) tensor_of[r] = -1;
    for (int t = 0; t < MOE_NUM_TENSORS; ++t) {
        if (roles[t] < 0 || roles[t] >= 9 || tensor_of[roles[t]] >= 0) {
            moe_set_error("set_format9: roles must name each of the 9 tensors once (tensor %d: %d)", t, roles[t]);
            return -1;
        }
        tensor_of[roles[t]] = t;
    }
    Q2Experts E = {};
    for (int p = 0; p < 3; ++p) {
        const uint64_t out = p == 2 ? hidden : inter, in = p == 2 ? inter : hidden;
        const uint64_t want[3] = {out * in / 4, out * (in / 64) * 2, out * (in / 64) * 2};
        for (int c = 0; c < 3; ++c) {
            const int t = tensor_of[3 * p + c];
            if (L.row_bytes[t] != want[c] || !L.dst[t]) {
                moe_set_error("set_format9: tensor %d (role %d) has %llu bytes per expert, expected %llu", t, 3 * p + c,
                              (unsigned long long)L.row_bytes[t], (unsigned long long)want[c]);
                return -1;
            }
        }
        E.p[p].w = (const uint8_t*)L.dst[tensor_of[3 * p]];
        E.p[p].s = (const uint8_t*)L.dst[tensor_of[3 * p + 1]];
        E.p[p].b = (const uint8_t*)L.dst[tensor_of[3 * p + 2]];
        E.p[p].w_stride = L.row_bytes[tensor_of[3 * p]];
        E.p[p].s_stride = L.row_bytes[tensor_of[3 * p + 1]];
        E.p[p].b_stride = L.row_bytes[tensor_of[3 * p + 2]];
        E.p[p].sb_step = 2;
    }
    E.bf16 = scale_bf16 & 1;
    E.scores_bf16 = (scale_bf16 >> 1) & 1;
    L.hidden = hidden;
    L.inter = inter;
    L.group = group;
    L.E9 = E;
    L.fmt9 = true;
    return 0;
}

// The 9 tensors as plain arguments: ptrs / slot_bytes in role order (gate w, s, b, up w, s, b,
// down w, s, b).
static bool experts9(const char* who, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int hidden,
                     int inter, Q2Experts& E) {
    if (!ptrs || !slot_bytes) { moe_set_error("%s: null tensor arrays", who); return false; }
    for (int p = 0; p < 3; ++p) {
        const uint64_t out = p == 2 ? hidden : inter, in = p == 2 ? inter : hidden;
        const uint64_t want[3] = {out * in / 4, out * (in / 64) * 2, out * (in / 64) * 2};
        for (int c = 0; c < 3; ++c)
            if (!ptrs[3 * p + c] || slot_bytes[3 * p + c] < want[c]) {
                moe_set_error("%s: tensor %d: %llu bytes per expert < %llu", who, 3 * p + c,
                              (unsigned long long)slot_bytes[3 * p + c], (unsigned long long)want[c]);
                return false;
            }
        E.p[p].w = (const uint8_t*)ptrs[3 * p];
        E.p[p].s = (const uint8_t*)ptrs[3 * p + 1];
        E.p[p].b = (const uint8_t*)ptrs[3 * p + 2];
        E.p[p].w_stride = slot_bytes[3 * p];
        E.p[p].s_stride = slot_bytes[3 * p + 1];
        E.p[p].b_stride = slot_bytes[3 * p + 2];
        E.p[p].sb_step = 2;
    }
    E.bf16 = scale_bf16 & 1;
    E.scores_bf16 = (scale_bf16 >> 1) & 1;
    return true;
}

int moe_q2t_gate_up(const void* x, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                    const uint32_t* slots, int k, int hidden, int inter, int group, void* h_out, void* stream) {
    Q2Experts E;
    if (!q2t_shape_ok("q2t_gate_up", k, hidden, inter, group)) return -1;
    if (!experts9("q2t_gate_up", ptrs, slot_bytes, scale_bf16, hidden, inter, E)) return -1;
    return launch_q2t_gate_up((const __half*)x, E, n_slots, slots, k, hidden, inter, (__half*)h_out, (hipStream_t)stream);
}

int moe_q2t_gate_up_routed(const void* x, const void* logits, int n_exp, int k, const uint64_t* ptrs,
                           const uint64_t* slot_bytes, int scale_bf16, int hidden, int inter, int group,
                           uint32_t* ids_out, void* scores_out, void* h_out, void* stream) {
    Q2Experts E;
    if (!q2t_shape_ok("q2t_gate_up_routed", k, hidden, inter, group)) return -1;
    if (!experts9("q2t_gate_up_routed", ptrs, slot_bytes, scale_bf16, hidden, inter, E)) return -1;
    return launch_q2t_gate_up_routed((const __half*)x, E, (const uint16_t*)logits, n_exp, k, hidden, inter, ids_out,
                                     (uint16_t*)scores_out, (__half*)h_out, (hipStream_t)stream);
}

int moe_q2t_down(const void* h, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                 const uint32_t* slots, const void* scores, int k, int hidden, int inter, int group,
                 const void* residual, float* y_out, int per_expert, void* stream) {
    Q2Experts E;
    if (!q2t_shape_ok("q2t_down", k, hidden, inter, group)) return -1;
    if (!experts9("q2t_down", ptrs, slot_bytes, scale_bf16, hidden, inter, E)) return -1;
    return launch_q2t_down((const __half*)h, E, n_slots, slots, (const __half*)scores, k, hidden, inter,
                           (const __half*)residual, y_out, per_expert, (hipStream_t)stream);
}

int moe_q2t_switch_glu(const void* x, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                       const uint32_t* slots, const void* scores, int k, int hidden, int inter, int group,
                       const void* residual, void* h_ws, float* y_out, int per_expert, void* stream) {
    if (moe_q2t_gate_up(x, ptrs, slot_bytes, scale_bf16, n_slots, slots, k, hidden, inter, group, h_ws, stream)) return -1;
    return moe_q2t_down(h_ws, ptrs, slot_bytes, scale_bf16, n_slots, slots, scores, k, hidden, inter, group, residual,
                        y_out, per_expert, stream);
}

// SwitchGLU over the layer's slot pool with the slot ids of its last decode step.  Orders the
// compute stream after the layer's pending copies and records the read for later copies.
int c_layer_switch_glu(int layer, const void* x, const void* scores, const void* residual, void* h_ws,
                       float* y_out, int per_expert, int k, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].hidden) {
        moe_set_error("layer_switch_glu: layer %d has no Q2 format (c_layer_set_format)", layer);
        return -1;
    }
    LayerState& L = g_layers[layer];
    if (!L.slot_inds_device) { moe_set_error("layer_switch_glu: slot_inds must be device memory"); return -1; }
    hipStream_t s = (hipStream_t)stream;
    if (wait_copies_gpu(L, s)) return -1;
    if (ensure_events(L)) return -1;
    if (layer_glu(L, x, L.slot_inds, scores, k, residual, h_ws, y_out, per_expert, s)) return -1;
    HIP_TRY(hipEventRecord(L.read_done, s));
    L.read_recorded = true;
    return 0;
}

// Half of a split SwitchGLU over the layer's pool after a scheduler step with SPLIT:
// part 0 runs the step's hit experts as soon as the layer's prefetch copies have landed and
// writes y = residual + sum over hits; part 1 waits for the demand copies and adds the sum over
// the missed experts.  Both parts must run on the same stream, part 0 first.
int c_layer_switch_glu_split(int layer, int part, const void* x, const void* scores, const void* residual,
                             void* h_ws, float* y_out, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].hidden) {
        moe_set_error("layer_switch_glu_split: layer %d has no Q2 format (c_layer_set_format)", layer);
        return -1;
    }
    if (part != 0 && part != 1) { moe_set_error("layer_switch_glu_split: part %d (0 hits, 1 misses)", part); return -1; }
    LayerState& L = g_layers[layer];
    const SplitLists& S = g_split[layer];
    if (S.n_hit <= 0 || S.n_miss <= 0) {
        moe_set_error("layer_switch_glu_split: layer %d has no split (scheduler step with SPLIT and 0 < misses < k)",
                      layer);
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    if (ensure_events(L)) return -1;
    if (!L.split_dev) HIP_TRY(hipMalloc((void**)&L.split_dev, 256));
    uint32_t* dslots = reinterpret_cast<uint32_t*>(L.split_dev);
    __half* dscores = reinterpret_cast<__half*>(L.split_dev + 128);
    int rc;
    if (part == 0) {
        if (L.pf_pending && join_prefetch_file(L)) return -1;
        if (L.pf_pending) HIP_TRY(hipStreamWaitEvent(s, L.pf_done, 0));
        if (launch_split_lists(S, (const __half*)scores, dslots, dscores, s)) return -1;
        rc = layer_glu(L, x, dslots, dscores, S.n_hit, residual, h_ws, y_out, 0, s);
    } else {
        if (wait_copies_gpu(L, s)) return -1;
        rc = layer_glu(L, x, dslots + MOE_MAX_K, dscores + MOE_MAX_K, S.n_miss, nullptr, h_ws, y_out, 2, s);
    }
    if (rc) return -1;
    HIP_TRY(hipEventRecord(L.read_done, s));
    L.read_recorded = true;
    return 0;
}

int moe_q2_grouped_gate_up(const void* x, int n_tokens, const int32_t* row_token, int n_rows, const int32_t* seg_start,
                           const int32_t* seg_slot, int n_seg, const void* pool, uint64_t stride, int n_slots,
                           int hidden, int inter, int group, void* h_out, void* stream) {
    return launch_q2_grouped_gate_up((const __half*)x, n_tokens, row_token, n_rows, seg_start, seg_slot, n_seg,
                                     (const uint8_t*)pool, stride, n_slots, hidden, inter, group, (__half*)h_out,
                                     (hipStream_t)stream);
}

int moe_q2_grouped_down(const void* h, int n_rows, const int32_t* row_out, int n_out_rows, const int32_t* seg_start,
                        const int32_t* seg_slot, int n_seg, const void* pool, uint64_t stride, int n_slots, int hidden,
                        int inter, int group, void* y_out, void* stream) {
    return launch_q2_grouped_down((const __half*)h, n_rows, row_out, n_out_rows, seg_start, seg_slot, n_seg,
                                  (const uint8_t*)pool, stride, n_slots, hidden, inter, group, (__half*)y_out,
                                  (hipStream_t)stream);
}

int moe_q2_grouped_switch_glu(const void* x, int n_tokens, const int32_t* row_token, const int32_t* row_out, int n_rows,
                              int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                              const void* pool, uint64_t stride, int n_slots, int hidden, int inter, int group,
                              void* h_ws, void* y_out, void* stream) {
    if (moe_q2_grouped_gate_up(x, n_tokens, row_token, n_rows, seg_start, seg_slot, n_seg, pool, stride, n_slots, hidden,
                               inter, group, h_ws, stream))
        return -1;
    return moe_q2_grouped_down(h_ws, n_rows, row_out, n_out_rows, seg_start, seg_slot, n_seg, pool, stride, n_slots,
                               hidden, inter, group, y_out, stream);
}

int moe_q2t_grouped_switch_glu(const void* x, int n_tokens, const int32_t* row_token, const int32_t* row_out,
                               int n_rows, int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                               const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots, int hidden,
                               int inter, int group, void* h_ws, void* y_out, void* stream) {
    Q2Experts E;
    if (!experts9("q2t_grouped_switch_glu", ptrs, slot_bytes, scale_bf16, hidden, inter, E)) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (launch_q2t_grouped_gate_up((const __half*)x, n_tokens, row_token, n_rows, seg_start, seg_slot, n_seg, E, n_slots,
                                   hidden, inter, group, (__half*)h_ws, s))
        return -1;
    return launch_q2t_grouped_down((const __half*)h_ws, n_rows, row_out, n_out_rows, seg_start, seg_slot, n_seg, E,
                                   n_slots, hidden, inter, group, (__half*)y_out, s);
}

uint64_t moe_cb_expert_bytes(int hidden, int inter) {
    if (hidden <= 0 || inter <= 0 || hidden % 256 || inter % 256) return 0;
    return cb_layout(hidden, inter).bytes;
}

int moe_cb_up(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots, int k, int hidden,
              int inter, const void* grid, void* h_out, void* stream) {
    return launch_cb_up((const __half*)x, (const uint8_t*)pool, stride, n_slots, slots, k, hidden, inter,
                        (const uint8_t*)grid, (uint16_t*)h_out, (hipStream_t)stream);
}

int moe_cb_down(const void* h, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
                const void* scores, int k, int hidden, int inter, const void* grid, const void* residual, float* y_out,
                int per_expert, void* stream) {
    return launch_cb_down((const uint16_t*)h, (const uint8_t*)pool, stride, n_slots, slots, (const __half*)scores, k,
                          hidden, inter, (const uint8_t*)grid, (const __half*)residual, y_out, per_expert,
                          (hipStream_t)stream);
}

int moe_cb_moe(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
               const void* scores, int k, int hidden, int inter, const void* grid, const void* residual, void* h_ws,
               float* y_out, int per_expert, void* stream) {
    if (moe_cb_up(x, pool, stride, n_slots, slots, k, hidden, inter, grid, h_ws, stream)) return -1;
    return moe_cb_down(h_ws, pool, stride, n_slots, slots, scores, k, hidden, inter, grid, residual, y_out, per_expert,
                       stream);
}

int moe_cb_moe_norm(const float* h_in, const void* norm_w, float eps, void* x_out, const void* pool, uint64_t stride,
                    int n_slots, const uint32_t* slots, const void* scores, int k, int hidden, int inter,
                    const void* grid, void* h_ws, float* y_out, void* stream) {
    if (launch_cb_up_norm(h_in, (const __half*)norm_w, eps, (__half*)x_out, (const uint8_t*)pool, stride, n_slots,
                          slots, k, hidden, inter, (const uint8_t*)grid, (uint16_t*)h_ws, (hipStream_t)stream))
        return -1;
    return moe_cb_down(h_ws, pool, stride, n_slots, slots, scores, k, hidden, inter, grid, x_out, y_out, 0, stream);
}

int moe_pair_combine(const void* y, const void* scores, const void* residual, int n_tokens, int k, int hidden,
                     float* out, void* stream) {
    return launch_pair_combine((const __half*)y, (const __half*)scores, (const __half*)residual, n_tokens, k, hidden, out,
                               (hipStream_t)stream);
}

// Grouped SwitchGLU over the layer's slot pool, segment u reading slot u (the chunk-local slot =
// rank of the expert in the chunk).  Orders `stream` after the layer's pending copies and records
// the read, so copies queued for the next chunk wait for it.
int c_layer_grouped_switch_glu(int layer, const void* x, int n_tokens, const int32_t* row_token,
                               const int32_t* row_out, int n_rows, int n_out_rows, const int32_t* seg_start,
                               int n_seg, void* h_ws, void* y_out, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init || !g_layers[layer].hidden) {
        moe_set_error("layer_grouped_switch_glu: layer %d has no Q2 format (c_layer_set_format)", layer);
        return -1;
    }
    LayerState& L = g_layers[layer];
    if (!L.dst[0]) { moe_set_error("layer_grouped_switch_glu: layer %d has no pool", layer); return -1; }
    if (n_seg > L.capacity) {
        moe_set_error("layer_grouped_switch_glu: %d segments > capacity %d", n_seg, L.capacity);
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    if (wait_copies_gpu(L, s)) return -1;
    if (ensure_events(L)) return -1;
    if (L.fmt9) {
        if (launch_q2t_grouped_gate_up((const __half*)x, n_tokens, row_token, n_rows, seg_start, nullptr, n_seg, L.E9,
                                       L.capacity, L.hidden, L.inter, L.group, (__half*)h_ws, s) ||
            launch_q2t_grouped_down((const __half*)h_ws, n_rows, row_out, n_out_rows, seg_start, nullptr, n_seg, L.E9,
                                    L.capacity, L.hidden, L.inter, L.group, (__half*)y_out, s))
            return -1;
    } else if (moe_q2_grouped_switch_glu(x, n_tokens, row_token, row_out, n_rows, n_out_rows, seg_start, nullptr, n_seg,
                                         (const void*)L.dst[0], L.row_bytes[0], L.capacity, L.hidden, L.inter, L.group,
                                         h_ws, y_out, stream)) {
        return -1;
    }
    HIP_TRY(hipEventRecord(L.read_done, s));
    L.read_recorded = true;
    return 0;
}

// Record that work queued so far on `stream` reads the layer's pool (later copies wait for it).
int c_layer_mark_read(int layer, void* stream) {
    if (!valid_layer(layer) || !g_layers[layer].init) { moe_set_error("mark_read: bad layer %d", layer); return -1; }
    LayerState& L = g_layers[layer];
    if (ensure_events(L)) return -1;
    HIP_TRY(hipEventRecord(L.read_done, (hipStream_t)stream));
    L.read_recorded = true;
    return 0;
}

// Host-blocking join of every copy queued so far.
int c_sync_copies(void) {
    for (int l = 0; l < MOE_MAX_LAYERS; ++l)
        if (join_file(g_layers[l])) return -1;
    if (!g_ready) return 0;
    HIP_TRY(hipStreamSynchronize(g_copy));
    return 0;
}

// Start timing every kernel launch of this library (up to `capacity` launches).
int c_timing_begin(int capacity) {
    if (capacity <= 0) { moe_set_error("timing_begin: capacity %d", capacity); return -1; }
    while (g_kt.size() < (size_t)capacity) {
        KtSlot k{0, nullptr, nullptr};
        HIP_TRY(hipEventCreate(&k.start));
        HIP_TRY(hipEventCreate(&k.stop));
        g_kt.push_back(k);
    }
    g_kt_cap = (size_t)capacity;
    g_kt_used = 0;
    g_kt_on = true;
    return 0;
}

// Stop timing; blocks until the timed kernels finished.  out_ms[kind] = summed kernel
// durations (ms), out_n[kind] = launches, for the MOE_TIMING_KINDS kinds.
static_assert(TK_KINDS == MOE_TIMING_KINDS, "kernel kinds out of step with the header");
int c_timing_end(double* out_ms, int* out_n) {
    g_kt_on = false;
    for (int i = 0; i < TK_KINDS; ++i) { out_ms[i] = 0.0; out_n[i] = 0; }
    for (size_t i = 0; i < g_kt_used; ++i) {
        KtSlot& k = g_kt[i];
        HIP_TRY(hipEventSynchronize(k.stop));
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, k.start, k.stop));
        out_ms[k.kind] += ms;
        out_n[k.kind] += 1;
    }
    g_kt_used = 0;
    return 0;
}

int moe_calibrate_copy(void* dst, const void* src, uint64_t bytes, void* stream) {
    return launch_copy_calib(dst, src, (size_t)bytes, (hipStream_t)stream);
}

int moe_calibrate_stream(const void* src, uint64_t bytes, int grid, float* out, void* stream) {
    return launch_stream_calib(src, (size_t)bytes, grid, out, (hipStream_t)stream);
}

int c_abi_version(void) { return 1; }

}  // extern "C"
