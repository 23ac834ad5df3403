// Builds against include/moe_io_sched.hpp the way the C++ runner uses the reference class
// (cpp/src/loader.cpp:728-731,907-908, engine.cpp:547-607): writes a small expert file, runs the
// cancel/promote scenario of cpp/tests/test_io_sched.cpp:150-200 and a forced invalidation with a
// std::mt19937_64, and prints what it observed as one JSON line for tests/test_p1_sched.py.
#include <fcntl.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "moe_io_sched.hpp"

namespace {
constexpr int kExp = 32, kNt = 9;
const uint64_t kRow[kNt] = {1024, 256, 256, 1024, 256, 256, 1024, 256, 256};

uint8_t byte_of(int eid, int t, uint64_t i) { return (uint8_t)(eid * 7 + t * 31 + i * 13); }
}  // namespace

int main(int argc, char** argv) {
    const std::string path = argc > 1 ? argv[1] : "/tmp/p1_class_test.bin";
    uint64_t offs[kNt], pos = 0;
    {
        FILE* f = fopen(path.c_str(), "wb");
        if (!f) return 2;
        for (int t = 0; t < kNt; ++t) {
            offs[t] = pos;
            for (int e = 0; e < kExp; ++e)
                for (uint64_t i = 0; i < kRow[t]; ++i) fputc(byte_of(e, t, i), f);
            pos += kExp * kRow[t];
        }
        fclose(f);
    }
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return 2;
    const int cap = 4;
    std::vector<std::vector<uint8_t>> pool(kNt);
    uint64_t ptrs[kNt];
    for (int t = 0; t < kNt; ++t) {
        pool[t].assign(cap * kRow[t], 0xCD);
        ptrs[t] = (uint64_t)(uintptr_t)pool[t].data();
    }
    std::vector<uint32_t> slot_inds(16, 0);

    moe::P1IoScheduler sched;
    sched.init(0);
    sched.set_wait_reader_callback([&](int l) { sched.unpin_layer_slots(l); });
    sched.layer_init(1, fd, cap, kNt, offs, kRow, ptrs, (uint64_t)(uintptr_t)slot_inds.data());
    int32_t e0[4] = {0, 1, 2, 3}, s0[4] = {0, 1, 2, 3};
    sched.load_sync(1, e0, s0, 4, true);
    sched.set_lru_state(1, e0, s0, 4, 4, 0, 4);
    sched.unpin_layer_slots(1);
    int32_t preds[3] = {10, 11, 12};
    sched.start_prefetch(1, preds, 3, 3);
    uint32_t route[4] = {0, 10, 20, 21}, out[4] = {};
    const int pending = sched.step_decode(1, route, 4, out);
    sched.wait_layer_urgent(1);
    bool bytes_ok = true;
    for (int i = 0; i < 4; ++i)
        for (int t = 0; t < kNt; ++t)
            for (uint64_t b = 0; b < kRow[t]; ++b)
                bytes_ok &= pool[t][out[i] * kRow[t] + b] == byte_of((int)route[i], t, b);
    moe::P1LayerStats st = sched.get_layer_stats(1);
    sched.unpin_layer_slots(1);
    std::mt19937_64 rng(7);
    const int inv = sched.force_invalidate(1, 0.5, rng);
    int32_t le[512], ls[512];
    int n = 0;
    sched.get_lru_state(1, le, ls, &n);
    printf("{\"pending\": %d, \"slots\": [%u, %u, %u, %u], \"bytes_ok\": %s, \"issued\": %llu, \"cancelled\": %llu, "
           "\"promoted\": %llu, \"used\": %llu, \"urgent\": %llu, \"invalidated\": %d, \"next_draw\": %llu, \"lru\": [",
           pending, out[0], out[1], out[2], out[3], bytes_ok ? "true" : "false",
           (unsigned long long)st.prefetch_issued, (unsigned long long)st.prefetch_cancelled,
           (unsigned long long)st.prefetch_promoted, (unsigned long long)st.prefetch_used,
           (unsigned long long)st.urgent_reads, inv, (unsigned long long)rng());
    for (int i = 0; i < n; ++i) printf("%s[%d, %d]", i ? ", " : "", le[i], ls[i]);
    printf("], \"threads\": %d}\n", sched.num_threads());
    sched.shutdown();
    close(fd);
    unlink(path.c_str());
    return 0;
}
