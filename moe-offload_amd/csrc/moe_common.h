// Shared definitions for libmoe_offload (gfx950).
//
// Expert blob: every routed expert of a layer is one contiguous byte range, in the slot pool
// (HBM) and in the host expert store alike, so that one miss is one copy.  For hidden H,
// intermediate I and group G (2-bit codes, 16 per uint32, LSB first, MLX affine format):
//
//   gate codes [I][H/16] u32 | up codes [I][H/16] u32 | down codes [H][I/16] u32 |
//   gate sb [I][H/G] | up sb [I][H/G] | down sb [H][I/G]
//
// where each sb entry is the pair (scale, bias) as two fp16 halves of one 32-bit word.  The
// code arrays are byte-for-byte the MLX `weight` arrays of one expert; the sb arrays
// interleave MLX's separate `scales`/`biases`.  At H=2048, I=512, G=64 an expert is
// 983,040 bytes (786,432 of codes, 196,608 of scale/bias).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stddef.h>
#include <stdint.h>

#define MOE_MAX_LAYERS 64
#define MOE_NUM_EXPERTS 512
#define MOE_NUM_TENSORS 9
#define MOE_MAX_K 16
#define MOE_MAX_PREFETCH 32

struct BlobLayout {
    int hidden, inter, group;
    size_t gate_codes, up_codes, down_codes, gate_sb, up_sb, down_sb, bytes;
};

static inline __host__ __device__ BlobLayout blob_layout(int hidden, int inter, int group) {
    BlobLayout L;
    L.hidden = hidden;
    L.inter = inter;
    L.group = group;
    size_t gu = (size_t)inter * hidden / 4;          // 2-bit codes: 4 per byte
    size_t dn = (size_t)hidden * inter / 4;
    size_t gsb = (size_t)inter * (hidden / group) * 4;
    size_t dsb = (size_t)hidden * (inter / group) * 4;
    L.gate_codes = 0;
    L.up_codes = gu;
    L.down_codes = 2 * gu;
    L.gate_sb = 2 * gu + dn;
    L.up_sb = L.gate_sb + gsb;
    L.down_sb = L.up_sb + gsb;
    L.bytes = L.down_sb + dsb;
    return L;
}

// The Q2 experts of a pool addressed per projection (gate, up, down): code rows [out][in/16] u32 at
// w + slot * w_stride, scales and biases at s / b + slot * s_stride / b_stride with sb_step bytes
// between consecutive (row, group) entries -- 2 for separate scale and bias arrays (the
// reference's 9 pools, loader.py:332-406), 4 for the interleaved (scale, bias) words of a blob.
// bf16 != 0: scales and biases are bf16, else fp16.
struct Q2Proj {
    const uint8_t* w;
    const uint8_t* s;
    const uint8_t* b;
    uint64_t w_stride, s_stride, b_stride;
    int sb_step;
};
struct Q2Experts {
    Q2Proj p[3];
    int bf16;
    int scores_bf16;      // the down kernel's expert scores are bf16 (the 8-bit router's), else fp16
};

// Roles of the 9 tensors of a reference layer (c_layer_set_format9).
enum { Q2T_GATE_W = 0, Q2T_GATE_S, Q2T_GATE_B, Q2T_UP_W, Q2T_UP_S, Q2T_UP_B, Q2T_DOWN_W, Q2T_DOWN_S, Q2T_DOWN_B };

// 2-bit codebook expert blob (IQ2_XXS-style super-blocks of 256 weights, seeded 256-entry grid):
//   up_qs [I][H/256][8][8 B] | down_qs [H][I/256][8][8 B] | up_d [I][H/256] fp16 | down_d [H][I/256] fp16
// Each 8-byte sub-block entry (32 weights) = 4 grid indices (one per 8-weight group) and a u32
// aux = sign7_0 | sign7_1 << 7 | sign7_2 << 14 | sign7_3 << 21 | sub_scale << 28.
struct CbLayout {
    int hidden, inter;
    size_t up_qs, down_qs, up_d, down_d, bytes;
};

static inline __host__ __device__ CbLayout cb_layout(int hidden, int inter) {
    CbLayout L;
    L.hidden = hidden;
    L.inter = inter;
    const size_t uq = (size_t)inter * (hidden / 256) * 64, dq = (size_t)hidden * (inter / 256) * 64;
    const size_t ud = (size_t)inter * (hidden / 256) * 2, dd = (size_t)hidden * (inter / 256) * 2;
    L.up_qs = 0;
    L.down_qs = uq;
    L.up_d = uq + dq;
    L.down_d = uq + dq + ud;
    L.bytes = uq + dq + ud + dd;
    return L;
}

// Hit/miss split of one scheduler step (c_layer_get_split_inds): slots of the ids that were
// resident, slots of the missed ids (both in id order), and each id's position in hits ++ misses.
struct SplitLists {
    uint32_t hit[MOE_MAX_K], miss[MOE_MAX_K];
    int32_t inv[MOE_MAX_K];
    int32_t n_hit, n_miss, k;
};

// Per-layer slot table.  The reference keeps a doubly linked list over slots
// (mlx-qwen38/expert_io.c:43-91); this keeps the same order as recency stamps: a resident
// slot carries stamp > 0, the LRU end is the smallest stamp, moving a slot to the MRU end
// gives it the next clock value.  Every list operation of the reference maps to a stamp
// operation with the same resulting order, so decisions are identical; the stamp form lets
// the device kernel pick victims with wave-wide reductions instead of pointer chasing.
// The same struct lives in host memory (host-driven layers) or device memory (device-driven
// layers) so tables can be copied either way.
struct SlotTable {
    int32_t capacity;
    int32_t n_free;
    uint32_t clock;
    int32_t snap_valid;
    uint64_t snap_resident[8];
    uint64_t snap_pred[8];
    uint64_t snap_fetched[8];
    uint64_t stats[18];
    uint64_t expert_bytes;
    // (16-byte aligned so the device kernels copy them with 128-bit loads)
    alignas(16) int16_t slot_of[MOE_NUM_EXPERTS];   // expert id -> slot, -1 when not resident
    alignas(16) int16_t eid_of[MOE_NUM_EXPERTS];    // slot -> expert id, -1 when empty
    alignas(16) int16_t free_stack[MOE_NUM_EXPERTS];
    alignas(16) uint32_t stamp[MOE_NUM_EXPERTS];    // 0 = slot not on the recency list
    // Copies the last decode step (list 0) and the last prefetch (list 1) need: (eid, slot).
    // Two lists, so a step may run while the previous prefetch's copies are still queued.
    int32_t n_copy;
    int32_t copy_eid[MOE_MAX_PREFETCH];
    int32_t copy_slot[MOE_MAX_PREFETCH];
    int32_t pf_n_copy;
    int32_t pf_copy_eid[MOE_MAX_PREFETCH];
    int32_t pf_copy_slot[MOE_MAX_PREFETCH];
    int32_t status;                     // 0 ok; nonzero: rejected input (device kernels)
    int32_t sched;                      // bit 0: device-driven ops follow the scheduler variant
                                        // (cpp/third_party/expert_io.c:1094-1394); bit 1: they
                                        // record the step's split lists (split below)
    int32_t io_fault;                   // sticky: 16 a file read failed, 17 a staging wait timed
                                        // out (the slot kept its old bytes); set by the file
                                        // tier's staging kernel, cleared only by reset_cache
    // Per-token accounting (cpp/third_party/expert_io.c:98-111,1002-1038).  Host tables keep the
    // open token and the counters in the library; device-driven tables keep them here, so the
    // table kernels can count without the host: acct_on / acct_token / acct_seq set by control
    // kernels on the compute stream (c_set_io_accounting, c_begin_decode_token, layer 1's
    // reset), acct[10] the table's share
    // of the open token's counters, stage_bytes the bytes one copied expert moves (0 for an
    // accounting-only layer).  evicted_at (both kinds): per expert, the token of its last
    // eviction, -1 none.
    int32_t acct_on;
    int32_t acct_token;                 // -1: no token open
    int32_t acct_seq;                   // the next token's number
    int32_t acct_pad;
    uint64_t stage_bytes;
    uint64_t acct[10];
    int32_t evicted_at[MOE_NUM_EXPERTS];
    // Device-driven tables in scheduler mode with sched bit 1: the split of the last step that
    // had 0 < misses < k (cpp/third_party/expert_io.c:1062-1092 keeps the last one the same way).
    SplitLists split;
};

// A set of device tables for the accounting control and gather kernels.
struct TableSet {
    SlotTable* t[MOE_MAX_LAYERS];
    int n;
};
int launch_acct_ctl(const TableSet& ts, int mode, hipStream_t s);        // 0 off, 1 on, 2 begin a token,
                                                                          // 3 restart the token numbering
int launch_acct_sum(const TableSet& ts, uint64_t* out10, hipStream_t s);  // out10 = sum of the tables' acct


// Stats word indices (same order as c_layer_get_stats, expert_io.c:791-812).
enum {
    ST_DEC_REQ = 0, ST_DEC_LRU_HIT, ST_DEC_PREF_HIT, ST_DEC_MISS, ST_DEC_BYTES, ST_PREF_BYTES,
    ST_PRE_REQ, ST_PRE_HIT, ST_PRE_MISS, ST_PRE_BYTES,
    ST_PRED_HITS, ST_PRED_ACTUAL, ST_PRED_TOTAL,
    ST_MISS_PREF_HITS, ST_MISS_ACTUAL, ST_MISS_FETCHED,
    ST_UNCOAL, ST_COAL
};

#define STAMP_RENORM_AT 0xF0000000u

// Error reporting: entry points record the first failure; c_last_error() returns it.
void moe_set_error(const char* fmt, ...);

#define HIP_TRY(expr)                                                                  \
    do {                                                                               \
        hipError_t _e = (expr);                                                        \
        if (_e != hipSuccess) {                                                        \
            moe_set_error("%s:%d %s -> %s", __FILE__, __LINE__, #expr, hipGetErrorString(_e)); \
            return -1;                                                                 \
        }                                                                              \
    } while (0)

// Optional per-launch kernel timing: when enabled, launchers dispatch through
// hipExtLaunchKernelGGL with a start/stop event pair, which the runtime stamps at the kernel's
// own begin/end; kinds index the accumulated totals.
enum { TK_ROUTER = 0, TK_GATE_UP, TK_DOWN, TK_STAGE, TK_SLOT, TK_PF_GATE_UP, TK_PF_DOWN, TK_COMBINE, TK_CB_UP,
       TK_CB_DOWN, TK_STREAM_CALIB, TK_KINDS };
bool kt_enabled();
void kt_events(int kind, hipEvent_t* start, hipEvent_t* stop);   // both null when disabled / full

#define MOE_LAUNCH(kind, kernel, grid, block, shmem, stream, ...)                            \
    do {                                                                                     \
        hipEvent_t _ks = nullptr, _ke = nullptr;                                             \
        if (kt_enabled()) kt_events(kind, &_ks, &_ke);                                       \
        if (_ks)                                                                             \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, _ks, _ke, 0, __VA_ARGS__); \
        else                                                                                 \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);             \
    } while (0)

// Kernel launchers implemented in the .hip translation units (return 0 / -1).
int launch_router(const float* h_in, const __half* norm_w, float eps, const __half* x_in,
                  __half* x_out, const __half* w, const __half* w_next, int hidden, int n_exp,
                  int k, int m, float* scratch, unsigned* counter, uint32_t* ids_out,
                  __half* scores_out, int32_t* pred_out, SlotTable* step_tab, uint32_t* slot_inds,
                  SlotTable* pf_tab, int max_fetch, hipStream_t s);
// launch_router with its scratch and arrival counter in a static device array of the library
// (no allocation, no caller workspace); n_exp <= 1024.  Overlapping calls on one GPU race.
int launch_router_noalloc(const float* h_in, const __half* norm_w, float eps, const __half* x_in, __half* x_out,
                          const __half* w, const __half* w_next, int hidden, int n_exp, int k, int m, uint32_t* ids_out,
                          __half* scores_out, int32_t* pred_out, hipStream_t s);
// The router's [RMSNorm +] GEMV alone: logits_out[n_exp] = fp16-rounded logits (as floats).
int launch_router_logits(const float* h_in, const __half* norm_w, float eps, const __half* x_in, __half* x_out,
                         const __half* w, int hidden, int n_exp, float* logits_out, hipStream_t s);
// Gate/up whose blocks first select the top-k experts from the logits (the router's rule, bit
// for bit) over a pool holding every expert (slot = id); ids/scores also go to ids_out /
// scores_out for the down product.
int launch_q2_gate_up_routed(const __half* x, const float* logits, int n_exp, int k, const uint8_t* pool,
                             size_t expert_stride, int hidden, int inter, int group, uint32_t* ids_out,
                             __half* scores_out, __half* h_out, hipStream_t s);
int launch_f64_to_f16(const double* in, uint16_t* out, int n, hipStream_t s);
int launch_rmsnorm(const float* h_in, const __half* norm_w, float eps, int hidden, __half* x_out,
                   hipStream_t s);
int launch_rmsnorm_bf16(const float* h_in, const uint16_t* norm_w, float eps, int hidden, uint16_t* x_bf16,
                        __half* x_f16, hipStream_t s);
int launch_q2_gate_up(const __half* x, const uint8_t* pool, size_t expert_stride, int n_slots,
                      const uint32_t* slots, int k, int hidden, int inter, int group,
                      __half* h_out, hipStream_t s);
int launch_q2_down(const __half* h, const uint8_t* pool, size_t expert_stride, int n_slots,
                   const uint32_t* slots, const __half* scores, int k, int hidden, int inter,
                   int group, const __half* residual, float* y_out, int per_expert,
                   hipStream_t s);
// Tensor-form Q2 GEMV (q2_gemv_t.hip): any hidden <= 4096 / inter <= 1024, multiples of 64.
bool q2t_shape_ok(const char* who, int k, int hidden, int inter, int group);
Q2Experts q2_experts_from_blob(const uint8_t* pool, size_t stride, const BlobLayout& L);
int launch_q2t_gate_up(const __half* x, const Q2Experts& E, int n_slots, const uint32_t* slots, int k, int hidden,
                       int inter, __half* h_out, hipStream_t s);
int launch_q2t_gate_up_routed(const __half* x, const Q2Experts& E, const uint16_t* logits, int n_exp, int k,
                              int hidden, int inter, uint32_t* ids_out, uint16_t* scores_out, __half* h_out,
                              hipStream_t s);
int launch_q2t_down(const __half* h, const Q2Experts& E, int n_slots, const uint32_t* slots, const __half* scores,
                    int k, int hidden, int inter, const __half* residual, float* y_out, int per_expert, hipStream_t s);
int launch_slot_step(SlotTable* t, const uint32_t* ids, int k, uint32_t* slot_inds,
                     hipStream_t s);
int launch_slot_prefetch(SlotTable* t, const int32_t* preds, int m, int max_fetch,
                         hipStream_t s);
int launch_stage(const SlotTable* t, int list, const uint8_t* store, size_t store_stride,
                 uint8_t* pool, size_t pool_stride, size_t bytes, int ctas, hipStream_t s);
// The listed experts' n tensors in one launch: tensor i of expert e is src_stride[i] bytes at
// src[i] + e * src_stride[i] (units[i] = its bytes / 16 copied), slot row s at dst[i] +
// s * dst_stride[i]; first[i] = the units of tensors 0..i-1, total = all units.
struct StageSet {
    const uint8_t* src[MOE_NUM_TENSORS];
    uint8_t* dst[MOE_NUM_TENSORS];
    uint64_t src_stride[MOE_NUM_TENSORS], dst_stride[MOE_NUM_TENSORS];
    uint32_t first[MOE_NUM_TENSORS];
    uint32_t total;
    int n;
};
int launch_stage_set(const SlotTable* t, int list, const StageSet& S, int ctas, hipStream_t s);
// Copies store[eids[i]] -> pool[slots[i]] for i < n over the tensors of S with CU loads from the
// mapped pinned store (the pairs travel in the kernel arguments, kStagePairsMax per launch).
int launch_stage_pairs(const int32_t* eids, const int32_t* slots, int n, const StageSet& S, hipStream_t s);
int launch_store_u32(uint32_t* dst, const uint32_t* vals, int n, hipStream_t s);
// slots_out[0..n_hit) / [16..16+n_miss): hit / miss slots; scores_out likewise, gathered from
// the step's scores (router order) through inv.
int launch_split_lists(const SplitLists& a, const __half* scores, uint32_t* slots_out, __half* scores_out,
                       hipStream_t s);
int launch_copy_calib(void* dst, const void* src, size_t bytes, hipStream_t s);
int launch_stream_calib(const void* src, size_t bytes, int grid, float* out, hipStream_t s);
int launch_q2_grouped_gate_up(const __half* x, int n_tokens, const int32_t* row_token, int n_rows,
                              const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                              const uint8_t* pool, size_t stride, int n_slots, int hidden, int inter,
                              int group, __half* h_out, hipStream_t s);
int launch_q2_grouped_down(const __half* h, int n_rows, const int32_t* row_out, int n_out_rows,
                           const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                           const uint8_t* pool, size_t stride, int n_slots, int hidden, int inter,
                           int group, __half* y_out, hipStream_t s);
int launch_q2t_grouped_gate_up(const __half* x, int n_tokens, const int32_t* row_token, int n_rows,
                               const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const Q2Experts& E,
                               int n_slots, int hidden, int inter, int group, __half* h_out, hipStream_t s);
int launch_q2t_grouped_down(const __half* h, int n_rows, const int32_t* row_out, int n_out_rows,
                            const int32_t* seg_start, const int32_t* seg_slot, int n_seg, const Q2Experts& E,
                            int n_slots, int hidden, int inter, int group, __half* y_out, hipStream_t s);
int launch_cb_up(const __half* x, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots, int k,
                 int hidden, int inter, const uint8_t* grid, uint16_t* h_out, hipStream_t s);
int launch_cb_up_norm(const float* h_in, const __half* norm_w, float eps, __half* x_out, const uint8_t* pool,
                      size_t stride, int n_slots, const uint32_t* slots, int k, int hidden, int inter,
                      const uint8_t* grid, uint16_t* h_out, hipStream_t s);
int launch_cb_down(const uint16_t* h, const uint8_t* pool, size_t stride, int n_slots, const uint32_t* slots,
                   const __half* scores, int k, int hidden, int inter, const uint8_t* grid, const __half* residual,
                   float* y_out, int per_expert, hipStream_t s);
int launch_pair_combine(const __half* y, const __half* scores, const __half* residual, int n_tokens,
                        int k, int hidden, float* out, hipStream_t s);
