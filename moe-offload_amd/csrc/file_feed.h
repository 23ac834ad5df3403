// Device-driven staging from the on-disk tier (host side + kernels in file_feed.hip).
//
// A device-driven layer decides its misses on the GPU (the slot table in device memory), so the
// host cannot know what to read before the router has run.  Here the table's copy list of a layer
// (list 0: the decode step's misses, list 1: the prefetch) is published by a one-wave kernel,
// right after the table operation, to a mailbox in host-coherent memory: the expert ids, their
// count and an epoch (stored last, with system-scope release).  A feeder thread polls the
// mailboxes and hands each new list to the reader threads (fileio): entry c of the list is read
// into bounce entry c of the (layer, list), and when all of its tensors have landed the entry's
// flag is set to the epoch.  The staging kernel waits for each entry's flag (bounded: an error
// marker or a timeout sets the table's status word and the kernel ends) and copies the entry
// from pinned host memory into its slot, like the pinned-store staging kernel.
//
// A bounce entry is rewritten only after the next publication of its (layer, list), which the
// stream orders after the previous staging of that list has finished (the next token's router of
// the layer runs after its GEMV, which waits for both lists' copies), and the feeder starts a
// publication's reads only once every read of that list's previous publication has ended (after a
// staging wait that timed out, the late reads would otherwise land in the reused entries).
//
// Failures are sticky: a failed read or a wait past its limit leaves the slot alone, sets the
// table's io_fault word (cleared only by reset_cache) and the library's fault word (host memory,
// read without a GPU synchronisation: fault_word()); later stagings of that table copy nothing.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_common.h"

namespace filefeed {

// The file layout of one layer (c_layer_init's arguments) and where its experts go.
struct LayerIO {
    int fd = -1, fd_direct = -1;
    uint64_t src[MOE_NUM_TENSORS] = {};        // file offset of expert 0 of tensor t
    uint64_t row_bytes[MOE_NUM_TENSORS] = {};  // bytes per expert of tensor t
    uint64_t dst[MOE_NUM_TENSORS] = {};        // HBM slot pool of tensor t
};

constexpr int kListCap[2] = {MOE_MAX_K, MOE_MAX_PREFETCH};   // entries per list
constexpr int32_t kStatusReadFailed = 16;                       // table status words
constexpr int32_t kStatusTimedOut = 17;

// Attach a device-driven file-backed layer (allocates its mailboxes and bounce entries, starts
// the feeder on first use); 0 or -1 with the error set.
int attach(int layer, const LayerIO& io);
// Detach it (waits for its reads in flight, frees its buffers); a no-op for an unattached layer.
void detach(int layer);
bool attached(int layer);
// Queue the publication of the layer's list (0 decode step, 1 prefetch) from its device table.
int publish(int layer, int list, SlotTable* dtab, hipStream_t s);
// Queue the staging kernel of the layer's list: ctas blocks per copied expert and tensor.
int stage(int layer, int list, SlotTable* dtab, int ctas, hipStream_t s);
// Longest a staging block waits for one entry (0: the default, 10 s).
void set_timeout_us(uint64_t us);
// The library's sticky fault word (the first io_fault code any table took; 0 none) and its clear.
int32_t fault_word();
void clear_fault_word();
// The layer's list was changed by a table operation (mark_table_op) or handed to the feeder
// (publish): stage() refuses a list changed since its last publication.
void mark_table_op(int layer, int list);
// Detach every layer and stop the feeder.
void shutdown();

}  // namespace filefeed
