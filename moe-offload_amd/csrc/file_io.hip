// Reader-thread pool of the on-disk expert tier (host code only; see file_io.h).
#include "file_io.h"

#include <errno.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <deque>
#include <thread>

namespace fileio {
namespace {

struct Item {
    std::shared_ptr<Batch> batch;
    size_t idx;
};

// The pool's state lives in a heap object that is never destroyed: reader threads still waiting
// on it when the process exits must not see it torn down (nor may a joinable std::thread be
// destroyed, which would call std::terminate).
struct Pool {
    std::mutex mu;
    std::condition_variable cv;
    std::deque<Item> queue;
    std::vector<std::thread> threads;
    int want = 8;
    bool stop = false;
};

Pool& P() {
    static Pool* p = new Pool;
    return *p;
}

void fail(Batch& b, const std::string& why) {
    std::lock_guard<std::mutex> g(b.mu);
    if (!b.failed) {
        b.failed = true;
        b.error = why;
    }
}

bool failed(Batch& b) {
    std::lock_guard<std::mutex> g(b.mu);
    return b.failed;
}

// Wait for the batch this one is queued after; its failure becomes this batch's.
void wait_after(Batch& b) {
    if (!b.after) return;
    std::string msg;
    if (wait(b.after, msg)) fail(b, "an earlier batch of the layer failed: " + msg);
}

void complete(Batch& b) {
    wait_after(b);
    b.after.reset();                                  // every on_read step has run: nothing else reads it
    const int rc = (!failed(b) && b.finish) ? b.finish() : 0;
    if (rc) fail(b, "copy issue failed");
    std::lock_guard<std::mutex> g(b.mu);
    b.done = true;
    b.cv.notify_all();
}

constexpr uint64_t kDirectChunk = 8ull << 20;

struct Stage {                                        // a worker's aligned buffer for O_DIRECT
    uint8_t* p = nullptr;
    ~Stage() { free(p); }
};

void do_read(Batch& b, const Read& r) {
    thread_local Stage st;
    if (r.direct && !st.p && posix_memalign((void**)&st.p, 4096, kDirectChunk)) {
        st.p = nullptr;
        std::lock_guard<std::mutex> g(b.mu);
        if (!b.failed) {
            b.failed = true;
            b.error = "no memory for the O_DIRECT staging buffer";
        }
        return;
    }
    uint64_t got = 0;
    while (got < r.len) {
        const uint64_t want = r.direct ? std::min(r.len - got, kDirectChunk) : r.len - got;
        const ssize_t n = pread(r.fd, r.direct ? st.p : r.dst + got, want, (off_t)(r.off + got));
        if (n < 0) {
            if (errno == EINTR) continue;
            std::lock_guard<std::mutex> g(b.mu);
            if (!b.failed) {
                b.failed = true;
                b.error = "pread(fd=" + std::to_string(r.fd) + ", off=" + std::to_string(r.off + got) + "): " + strerror(errno);
            }
            return;
        }
        if (n == 0) break;                        // end of file
        if (r.direct) memcpy(r.dst + got, st.p, (size_t)n);
        got += (uint64_t)n;
        if (r.direct && (uint64_t)n < want) break;    // end of file inside this chunk
    }
    if (got < r.need) {
        std::lock_guard<std::mutex> g(b.mu);
        if (!b.failed) {
            b.failed = true;
            b.error = "short read at offset " + std::to_string(r.off) + ": " + std::to_string(got) + " of " +
                      std::to_string(r.need) + " bytes";
        }
    }
}

void worker() {
    for (;;) {
        Item it;
        {
            Pool& p = P();
            std::unique_lock<std::mutex> lk(p.mu);
            p.cv.wait(lk, [&] { return p.stop || !p.queue.empty(); });
            if (p.queue.empty()) return;          // stopping and drained
            it = std::move(p.queue.front());
            p.queue.pop_front();
        }
        Batch& b = *it.batch;
        const Read& r = b.reads[it.idx];
        do_read(b, r);
        if (b.on_read && !failed(b)) {
            wait_after(b);
            if (!failed(b) && b.on_read(r.tag)) fail(b, "copy issue failed");
        }
        if (b.left.fetch_sub(1) == 1) complete(b);
    }
}

void stop_locked(std::unique_lock<std::mutex>& lk) {
    Pool& p = P();
    p.stop = true;
    p.cv.notify_all();
    std::vector<std::thread> ts;
    ts.swap(p.threads);
    lk.unlock();
    for (auto& t : ts) t.join();
    lk.lock();
    p.stop = false;
}

}  // namespace

void set_threads(int n) {
    Pool& p = P();
    std::unique_lock<std::mutex> lk(p.mu);
    const int want = n > 0 ? n : 8;
    if (want == p.want) return;
    p.want = want;
    if (!p.threads.empty()) stop_locked(lk);      // restarted with the new count on the next batch
}

int threads() {
    Pool& p = P();
    std::lock_guard<std::mutex> g(p.mu);
    return p.want;
}

void submit(const std::shared_ptr<Batch>& b) {
    // largest reads first, so the batch's longest read does not start last
    std::stable_sort(b->reads.begin(), b->reads.end(), [](const Read& x, const Read& y) { return x.len > y.len; });
    b->left.store((int)b->reads.size());
    if (b->reads.empty()) {
        complete(*b);
        return;
    }
    Pool& p = P();
    std::lock_guard<std::mutex> g(p.mu);
    while ((int)p.threads.size() < p.want) p.threads.emplace_back(worker);
    for (size_t i = 0; i < b->reads.size(); ++i) p.queue.push_back(Item{b, i});
    p.cv.notify_all();
}

int wait(const std::shared_ptr<Batch>& b, std::string& msg) {
    std::unique_lock<std::mutex> lk(b->mu);
    b->cv.wait(lk, [&] { return b->done; });
    if (b->failed) {
        msg = b->error;
        return -1;
    }
    return 0;
}

void shutdown() {
    Pool& p = P();
    std::unique_lock<std::mutex> lk(p.mu);
    if (!p.threads.empty()) stop_locked(lk);
}

}  // namespace fileio
