// Reads of the on-disk expert tier: a pool of reader threads (host code).
//
// The reference reads its experts-XX.safetensors shard with a pthread pool and one preadv per
// (tensor, run of consecutive experts), longest reads first (mlx-qwen38/expert_io.c:95-276); a
// batch runs in the background and every later entry point joins it first (:312-356).  Here a
// batch is a list of contiguous reads into pinned host memory, an `on_read` step run by the worker
// that completed a read (it queues that read's host-to-device copies, so copies overlap the reads
// still running) and a `finish` step run once every read is done (it records the batch's events);
// `wait` is the join.  A batch may name an earlier one (`after`) whose copies must be queued before
// any of its own: its on_read and finish steps wait for that batch first, so a batch being done
// means every batch before it is done too, and an earlier batch's failure fails the later one.
#pragma once
#include <stdint.h>

#include <atomic>
#include <condition_variable>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace fileio {

struct Read {
    int fd;
    uint64_t off;        // file offset
    uint64_t len;        // bytes to read (len >= need; the tail may lie past the end of the file)
    uint64_t need;       // bytes that must be read
    uint8_t* dst;
    // fd was opened with O_DIRECT (off and len 4 KiB multiples): the kernel cannot read straight
    // into pinned GPU-visible host memory (its pages cannot be pinned again: EFAULT), so the read
    // goes through the worker's own aligned buffer, 8 MiB at a time, and is copied to dst.
    bool direct = false;
    int tag = -1;        // passed to the batch's on_read step
};

struct Batch {
    std::vector<Read> reads;
    std::function<int(int tag)> on_read;  // after each successful read; 0 or -1
    std::function<int()> finish;          // 0 or -1 (then `error` says why)
    std::shared_ptr<Batch> after;         // queued before this batch (may be null)
    std::atomic<int> left{0};
    std::mutex mu;
    std::condition_variable cv;
    bool done = false;
    bool failed = false;
    std::string error;
};

// Reader threads (<= 0: 8, the reference's default, loader.py:219-223); takes effect for later
// batches (the pool drains first).
void set_threads(int n);
int threads();
// Start the batch's reads (largest first); returns at once.
void submit(const std::shared_ptr<Batch>& b);
// Block until the batch's reads and its finish step are done; 0, or -1 with the error in `msg`.
int wait(const std::shared_ptr<Batch>& b, std::string& msg);
// Stop the reader threads (after the queued work).
void shutdown();

}  // namespace fileio
