/*
 * moe_offload.h -- C-ABI of libmoe_offload.so, the MI355X (gfx950) routed-expert decode path.
 *
 * Part 1 replaces the reference's native expert cache, mlx-qwen38/expert_io.c, symbol for
 * symbol (the ctypes bindings of mlx-qwen38/loader.py:100-220 bind them unchanged).  Part 2 is
 * the compute the reference gets from MLX built-ins (gather_qmm, softmax, argpartition), as
 * hand-written HIP kernels.  Part 3 has no counterpart in the reference (device-driven slot
 * tables, streams, pinned host memory, error reporting).
 *
 * Conventions: plain pointers and sizes only.  Device pointers are HIP device addresses
 * (e.g. torch tensors' data_ptr()); `stream` is a hipStream_t (0 = null stream).  As in the
 * reference, entry points given an out-of-range layer return silently; every other failure is
 * recorded and reported by c_last_error() (int-returning entry points also return -1).
 */
#ifndef MOE_OFFLOAD_H
#define MOE_OFFLOAD_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Part 1: expert cache (expert_io.c) -------------------------------------------------- */

/* expert_io.c:430-448.  num_threads: reader threads of file-backed layers (<= 0: 8), started on
 * the first file batch; copies from host memory go to the DMA engines. */
void c_io_init(int num_threads);
/* cpp/src/expert_io.h:15 (superset ABI).  Joins file batches, stops the reader threads, drains
 * copies and releases every layer. */
void c_io_shutdown(void);
/* No counterpart in the reference (its files are read through the page cache).  on != 0: file-backed
 * layers initialised from now on also open their file with O_DIRECT, reading 4 KiB-aligned ranges
 * that bypass the page cache; a file system that refuses it leaves the layer on the page cache
 * (c_layer_io_direct says which). */
void c_io_set_direct(int on);
/* 1 when the layer reads its file with O_DIRECT, else 0. */
int c_layer_io_direct(int layer_idx);
/* Reader threads the file tier uses (c_io_init). */
int c_io_threads(void);
/* No counterpart in the reference (loader.py reads a shard through mx.load).  Reads n ranges of
 * the file (lens[i] bytes at offs[i] into host address dsts[i]) with the reader threads and
 * returns when all are done: 0, or -1 on a failed or short read (c_last_error).  Host only. */
int c_io_read_ranges(int fd, const uint64_t* offs, const uint64_t* lens, const uint64_t* dsts, int n);
/* expert_io.c:497-520.  fd == -1: base_offsets[t] are host addresses of tensor t's expert store
 * (pinned via c_host_alloc for overlap / device staging); fd >= 0: file offsets as in the
 * reference, each batch of misses read by the reader threads as one read per (tensor, run of
 * consecutive experts) and joined where its slots are used (host-driven staging only; the caller
 * keeps fd open until the layer is re-initialised or c_io_shutdown).  base_ptrs[t] are device slot pools; slot_inds_ptr receives slot ids (device or
 * host memory).  capacity in 1..512. */
void c_layer_init(int layer_idx, int fd, int capacity, const uint64_t* base_offsets,
                  const uint64_t* row_bytes, const uint64_t* base_ptrs, uint64_t slot_inds_ptr);
/* expert_io.c:450-468 */
void c_layer_reset_cache(int layer_idx);
/* expert_io.c:470-495 */
void c_layer_reset_stats(int layer_idx);
/* expert_io.c:583-685.  Returns the number of demand misses; writes k slot ids to slot_inds.
 * async_io != 0 leaves the copies in flight (join: c_layer_wait_prefetch). k in 1..16. */
int c_layer_step_decode_ex(int layer_idx, const uint32_t* eids, int k, int async_io);
/* expert_io.c:687-689 (synchronous) */
int c_layer_step_decode(int layer_idx, const uint32_t* eids, int k);
/* expert_io.c:692-699 */
int c_layer_step_decode10(int layer_idx, uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3,
                          uint32_t e4, uint32_t e5, uint32_t e6, uint32_t e7, uint32_t e8,
                          uint32_t e9);
/* expert_io.c:701-708 */
int c_layer_step_decode10_async(int layer_idx, uint32_t e0, uint32_t e1, uint32_t e2,
                                uint32_t e3, uint32_t e4, uint32_t e5, uint32_t e6, uint32_t e7,
                                uint32_t e8, uint32_t e9);
/* expert_io.c:527-581.  n <= 32. */
void c_layer_start_prefetch(int layer_idx, const int32_t* pred_eids, int pred_count, int max_fetch);
/* expert_io.c:814-822 */
void c_layer_start_prefetch10(int layer_idx, int max_fetch, int32_t e0, int32_t e1, int32_t e2,
                              int32_t e3, int32_t e4, int32_t e5, int32_t e6, int32_t e7,
                              int32_t e8, int32_t e9);
/* expert_io.c:824-832 */
void c_layer_start_prefetch12(int layer_idx, int max_fetch, int32_t e0, int32_t e1, int32_t e2,
                              int32_t e3, int32_t e4, int32_t e5, int32_t e6, int32_t e7,
                              int32_t e8, int32_t e9, int32_t e10, int32_t e11);
/* expert_io.c:522-525.  Joins every in-flight copy on the GPU side: the compute stream waits;
 * the host does not block (c_sync_copies blocks). */
void c_layer_wait_prefetch(int layer_idx);
/* expert_io.c:710-724.  Blocking copy of (eid -> slot) pairs; counts prefill bytes.  From a
 * pinned store the copies run as a CU copy kernel (reads of the mapped store) on the copy
 * stream; from a file-backed store through the reader threads. */
void c_layer_load_sync(int layer_idx, const int32_t* eids, const int32_t* slots, int count,
                       int is_prefill);
/* expert_io.c:726-747.  LRU -> MRU order. */
void c_layer_get_lru_state(int layer_idx, int32_t* out_eids, int32_t* out_slots, int* out_count);
/* expert_io.c:749-789 */
void c_layer_set_lru_state(int layer_idx, const int32_t* ordered_eids, const int32_t* ordered_slots,
                           int count, uint64_t add_prefill_requests, uint64_t add_prefill_hits,
                           uint64_t add_prefill_misses);
/* expert_io.c:791-812.  out[18]; byte counters use the layer's real expert bytes. */
void c_layer_get_stats(int layer_idx, uint64_t* out_stats);
/* expert_io.c:834-852.  out[6] summed over layers 1..num_layers-1. */
void c_get_decode_totals(int num_layers, uint64_t* out6);

/* Superset ABI of the reference's C++ runner (cpp/src/expert_io.h:8-108, implemented in
 * cpp/third_party/expert_io.c).  These act on host-driven layers. */
enum { MOE_SCHED_SYNC_DEMAND = 1, MOE_SCHED_NO_PREFETCH = 2, MOE_SCHED_SPLIT = 4 };
/* cpp/third_party/expert_io.c:1094-1394.  One call per layer: the decode step of layer_idx
 * (skipped for layer 0 or null eids; k > 16 is cut to 16) whose victim choice also protects
 * the experts the layer's last prefetch fetched, then the prefetch of next_layer (only when
 * next_layer > 0, pred given, n_pred > 0, prefetch_cap > 0 and not NO_PREFETCH) taking each
 * predicted expert at most once, its copies queued behind the demand copies.  SPLIT records
 * the hit / miss slot lists when 0 < misses < k; SYNC_DEMAND blocks the host until the layer's
 * copies land; with no miss the layer's copies are joined on the GPU.  Returns the misses. */
int c_layer_decode_step_sched(int layer_idx, const int32_t* eids, int k, const int32_t* pred,
                              int n_pred, int next_layer, int prefetch_cap, int flags);
/* cpp/third_party/expert_io.c:1062-1092.  The last recorded split of the layer: hit slots,
 * miss slots (id order) and each id's position in hits ++ misses (kept until the next split).
 * A device-driven layer's split is the one its table kernels recorded (c_layer_set_sched bit 1);
 * reading it waits for the compute stream. */
void c_layer_get_split_inds(int layer_idx, uint32_t* out_hit_slots, uint32_t* out_miss_slots,
                            int32_t* out_inv_order);
/* cpp/third_party/expert_io.c:1048-1060.  Joins the layer's copies on the GPU side (the
 * compute stream waits; the host does not block). */
void c_layer_wait_demand(int layer_idx);
/* cpp/third_party/expert_io.c:1002-1038.  Per-token accounting: out10 = lru hits, demand
 * misses, prefetch loads, prefetch hits, wasted prefetches, demand re-reads within 16 / 64
 * tokens, prefetch re-reads within 16 / 64 tokens, bytes staged.  Tokens are numbered by the
 * library (token_idx is ignored, as in the reference); layer 1's reset restarts the numbering.
 * Host tables count in the library; device-driven tables count in their table kernels: for
 * them the three calls queue small control kernels on the compute stream (so they order with
 * the token's kernels and a captured token's table work counts at replay), and
 * c_end_decode_token adds the device tables' counters, waiting for the compute stream. */
void c_set_io_accounting(int enabled);
void c_begin_decode_token(int token_idx);
void c_end_decode_token(uint64_t* out10);
/* cpp/third_party/expert_io.c:1040-1042.  Host bytes held by the library's tables and
 * buffers. */
uint64_t c_get_native_buffer_bytes(void);

/* ---- Part 2: compute (MLX built-ins of the reference) ------------------------------------- */

/* loader.py:903-908 + loader.py:237-242,950-958 (cpp/src/layers.cpp:311-341).  Optional
 * RMSNorm of an fp32 residual h_in (norm_w fp16, may be null) into x_out, else fp16 x_in;
 * logits = x.W^T (fp16 [n_exp][hidden]); softmax; top-k ids (ascending gate) and fp16 scores;
 * when w_next != null, the next layer's top-m prediction (descending).  workspace:
 * moe_router_workspace_bytes(n_exp) bytes of device memory, zeroed once before first use. */
int moe_router(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out,
               const void* w, const void* w_next, int hidden, int n_exp, int k, int m,
               void* workspace, uint32_t* ids_out, void* scores_out, int32_t* pred_out,
               void* stream);
uint64_t moe_router_workspace_bytes(int n_exp);
/* The real checkpoint's router / predictor (loader.py:903-908, 237-242, 950-958;
 * cpp/src/kernels.cpp:997-1019 QLinear::forward with bits 8, group 64): an 8-bit affine quantized
 * linear layer over a bf16 vector x [hidden] -- codes u32 [n_rows][hidden / 4] (4 bytes per word,
 * LSB first), scales and biases bf16 [n_rows][hidden / 64] -- with logits rounded to bf16 once
 * (fp64 accumulation).  Route mode (k > 0, m == 0): ids_out u32 [k] and scores_out bf16 [k] in
 * ascending gate order (gates = bf16(softmax), scores = bf16(g / s), s the left-to-right bf16 sum).
 * Predict mode (m > 0, k == 0): pred_out i32 [m], the top m logits by descending value (equal
 * values by ascending id).  logits_out (bf16 [n_rows], optional; required when k == m == 0).
 * hidden a multiple of 64 up to 4096, n_rows <= 1024.  workspace: moe_router_q8_workspace_bytes,
 * zero-filled before its first use (the kernel leaves it reusable). */
uint64_t moe_router_q8_workspace_bytes(int n_rows);
int moe_router_q8(const void* x, const uint32_t* codes, const void* scales, const void* biases, int hidden,
                  int n_rows, int group, int k, int m, void* workspace, uint32_t* ids_out, void* scores_out,
                  int32_t* pred_out, void* logits_out, void* stream);
/* moe_rmsnorm_bf16 + moe_router_q8 in one launch (no reference counterpart: the glue is the
 * builder's): every block normalises h_in (fp32 [hidden], norm_w bf16 or null) with
 * moe_rmsnorm_bf16's arithmetic while its weight loads fly and multiplies the bf16 result; block 0
 * also writes x_bf16_out / x_f16_out (either may be null), bit-identical to moe_rmsnorm_bf16's.
 * Other arguments, modes and outputs as moe_router_q8; hidden a multiple of 64 up to 4096. */
int moe_router_q8_norm(const float* h_in, const void* norm_w, float eps, void* x_bf16_out, void* x_f16_out,
                       const uint32_t* codes, const void* scales, const void* biases, int hidden, int n_rows,
                       int group, int k, int m, void* workspace, uint32_t* ids_out, void* scores_out,
                       int32_t* pred_out, void* logits_out, void* stream);
/* No counterpart in the reference.  moe_router for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): no workspace argument;
 * the logits and the arrival counter live in a static device array of the library (8,448 bytes
 * per GPU, held until the process ends).  Allocates nothing.  n_exp <= 1024 (larger is rejected
 * with an error).  Every call on one GPU shares that array: calls that overlap on one GPU (other
 * streams, other threads) race. */
int moe_router_noalloc(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out,
                       const void* w, const void* w_next, int hidden, int n_exp, int k, int m,
                       uint32_t* ids_out, void* scores_out, int32_t* pred_out, void* stream);
/* moe_router split at the logits, for a pool that holds every expert (the resident path; no
 * slot table has to run once per layer): moe_router_logits writes logits_out fp32 [n_exp] (each
 * the fp16-rounded logit moe_router computes), and moe_q2_gate_up_routed's blocks select the
 * top-k from them with moe_router's rule (same ids, order and scores, bit for bit; ids_out and
 * scores_out as moe_router's) before their moe_q2_gate_up over pool[id].  Together they replace
 * moe_router + moe_q2_gate_up without the router's last-block hand-off.  n_exp <= 1024. */
int moe_router_logits(const float* h_in, const void* norm_w, float eps, const void* x_in, void* x_out,
                      const void* w, int hidden, int n_exp, float* logits_out, void* stream);
int moe_q2_gate_up_routed(const void* x, const float* logits, int n_exp, int k, const void* pool,
                          uint64_t stride, int hidden, int inter, int group, uint32_t* ids_out,
                          void* scores_out, void* h_out, void* stream);
/* The single f64 -> f16 rounding every kernel uses (exposed so tests can check it directly). */
int moe_f64_to_f16(const double* in, uint16_t* out, int n, void* stream);
/* Builder-defined glue between stacked MoE layers (no reference counterpart: the reference
 * mixes hyper-connections there, loader.py:61,992): x_out fp16 = RMSNorm(h_in fp32) * norm_w,
 * the same arithmetic as moe_router's prologue. */
int moe_rmsnorm(const float* h_in, const void* norm_w, float eps, int hidden, void* x_out,
                void* stream);
/* The same glue for the reference's bf16 checkpoint (no reference counterpart): norm_w bf16 (or
 * null), x_bf16_out = bf16(RMSNorm(h_in) * norm_w) rounded once from fp64 -- moe_router_q8's input
 * -- and x_f16_out = that bf16 value as fp16, the tensor-form expert kernels' input. */
int moe_rmsnorm_bf16(const float* h_in, const void* norm_w, float eps, int hidden, void* x_bf16_out,
                     void* x_f16_out, void* stream);
/* Bytes of one Q2 expert blob (layout in csrc/moe_common.h). */
uint64_t moe_q2_expert_bytes(int hidden, int inter, int group);
/* gather_qmm gate+up + SwiGLU (loader.py:564, kernels.cpp:1027-1040,1090-1094):
 * h_out[k][inter] fp16 from x fp16 [hidden] over pool blobs selected by slots[k]; pool holds
 * n_slots blobs of `stride` bytes (a slot id >= n_slots contributes zeros).  hidden, inter:
 * multiples of 64, hidden <= 4096, inter <= 1024. */
int moe_q2_gate_up(const void* x, const void* pool, uint64_t stride, int n_slots,
                   const uint32_t* slots, int k, int hidden, int inter, int group, void* h_out,
                   void* stream);
/* gather_qmm down + weighted combine (loader.py:964-965).  per_expert 0: y_out fp32 [hidden] =
 * residual + sum_j scores[j] * down_j(h_j); 1: per-expert rows y_out[k][hidden]; 2: y_out +=
 * sum_j scores[j] * down_j(h_j) (residual ignored). */
int moe_q2_down(const void* h, const void* pool, uint64_t stride, int n_slots,
                const uint32_t* slots, const void* scores, int k, int hidden, int inter, int group,
                const void* residual, float* y_out, int per_expert, void* stream);
/* Both of the above (h_ws: k*inter fp16 workspace). */
int moe_q2_switch_glu(const void* x, const void* pool, uint64_t stride, int n_slots,
                      const uint32_t* slots, const void* scores, int k, int hidden, int inter,
                      int group, const void* residual, void* h_ws, float* y_out, int per_expert,
                      void* stream);

/* The same SwitchGLU over experts held as the reference's 9 tensors (loader.py:332-406: per
 * projection a code pool [slots][out][in/16] u32 and scale and bias pools [slots][out][in/64]),
 * each tensor at its own base address with its own bytes per slot.  ptrs / slot_bytes: 9 entries
 * in role order -- gate weight, scales, biases, up weight, scales, biases, down weight, scales,
 * biases; scale_bf16 bit 0: scales and biases are bf16 (the reference's checkpoints), else fp16;
 * bit 1: the down product's scores are bf16 (as moe_router_q8 and moe_q2t_gate_up_routed write
 * them), else fp16.
 * Any hidden <= 4096 and inter <= 1024 that are multiples of 64 (the real model: 2560 / 640);
 * other arguments as moe_q2_gate_up / moe_q2_down / moe_q2_switch_glu, which also take these
 * shapes for blob pools. */
int moe_q2t_gate_up(const void* x, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                    const uint32_t* slots, int k, int hidden, int inter, int group, void* h_out, void* stream);
/* No counterpart in the reference: moe_q2t_gate_up for a pool holding every expert (slot = id),
 * whose blocks select the top k themselves from the bf16 logits of moe_router_q8 (logits-only
 * mode, k == m == 0) by the router's own rule and code -- ids u32 [k] and bf16 scores [k] out,
 * bit-identical to moe_router_q8 in route mode -- so a resident layer of the real checkpoint
 * needs no router selection pass (loader.py:903-908 + 557-564 fused). */
int moe_q2t_gate_up_routed(const void* x, const void* logits, int n_exp, int k, const uint64_t* ptrs,
                           const uint64_t* slot_bytes, int scale_bf16, int hidden, int inter, int group,
                           uint32_t* ids_out, void* scores_out, void* h_out, void* stream);
int moe_q2t_down(const void* h, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                 const uint32_t* slots, const void* scores, int k, int hidden, int inter, int group,
                 const void* residual, float* y_out, int per_expert, void* stream);
int moe_q2t_switch_glu(const void* x, const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots,
                       const uint32_t* slots, const void* scores, int k, int hidden, int inter, int group,
                       const void* residual, void* h_ws, float* y_out, int per_expert, void* stream);

/* Prefill grouped GEMM (loader.py:566-699 sorted gather_qmm via prefill_qproj.py:18-40;
 * cpp/src/layers.cpp:364-600).  The n_rows (token, k) rows are sorted by expert; segment u
 * covers sorted rows [seg_start[u], seg_start[u+1]) and uses pool blob seg_slot[u] (seg_slot
 * null: blob u, the reference's chunk-local slot = rank in chunk).  All index arrays are
 * device memory.  gate_up: h_out[r][inter] fp16 = silu(G x_{row_token[r]}) * (U x_{row_token[r]});
 * down: y_out[row_out[r]][hidden] fp16 = D h[r] (row_out null: row r).  A row whose token is
 * out of range computes from zeros; rows whose output row or slot is out of range are not
 * written.  Requires hidden, inter multiples of 64 and
 * <= 2560, group 64.  MFMA (v_mfma_f32_16x16x32_f16), fp32 accumulation. */
int moe_q2_grouped_gate_up(const void* x, int n_tokens, const int32_t* row_token, int n_rows,
                           const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                           const void* pool, uint64_t stride, int n_slots, int hidden, int inter,
                           int group, void* h_out, void* stream);
int moe_q2_grouped_down(const void* h, int n_rows, const int32_t* row_out, int n_out_rows,
                        const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                        const void* pool, uint64_t stride, int n_slots, int hidden, int inter,
                        int group, void* y_out, void* stream);
/* Both of the above (h_ws: n_rows*inter fp16 workspace). */
int moe_q2_grouped_switch_glu(const void* x, int n_tokens, const int32_t* row_token,
                              const int32_t* row_out, int n_rows, int n_out_rows,
                              const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                              const void* pool, uint64_t stride, int n_slots, int hidden,
                              int inter, int group, void* h_ws, void* y_out, void* stream);
/* Score-weighted sum of per-(token, k) rows (loader.py:964-965): out fp32 [n_tokens][hidden] =
 * residual + sum_j scores[t][j] * y[t*k + j] (fp16 y, scores, residual; residual may be null). */
int moe_pair_combine(const void* y, const void* scores, const void* residual, int n_tokens, int k,
                     int hidden, float* out, void* stream);

/* 2-bit codebook experts: the Nemotron model of README.md:37 (IQ2_XXS GGUF, 240 experts, top-9),
 * run by the reference only inside llama.cpp's Metal backend (llama-moe-cache.patch:1-12 adds the
 * mul_mm_id map for 9 experts per token; format in csrc/moe_common.h CbLayout): non-gated up ->
 * squared ReLU -> down.
 * grid: device uint8 [256][8] magnitudes (the workload's seeded grid holds {1, 3, 5}).
 * hidden, inter multiples of 256 (hidden <= 4096, inter <= 2048), k <= 16. */
uint64_t moe_cb_expert_bytes(int hidden, int inter);
/* h_out bf16 [k][inter] = relu(U_j x)^2 for x fp16 [hidden]; a slot id >= n_slots yields 0. */
int moe_cb_up(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots, int k,
              int hidden, int inter, const void* grid, void* h_out, void* stream);
/* per_expert 0: y_out fp32 [hidden] = residual + sum_j scores[j] * D_j h_j; 1: rows y_out[k][hidden]. */
int moe_cb_down(const void* h, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
                const void* scores, int k, int hidden, int inter, const void* grid, const void* residual,
                float* y_out, int per_expert, void* stream);
/* Both of the above (h_ws: k*inter bf16 workspace). */
int moe_cb_moe(const void* x, const void* pool, uint64_t stride, int n_slots, const uint32_t* slots,
               const void* scores, int k, int hidden, int inter, const void* grid, const void* residual,
               void* h_ws, float* y_out, int per_expert, void* stream);
/* One layer of the codebook stack from the previous layer's fp32 output: x = RMSNorm(h_in) * norm_w
 * (fp64, one fp16 rounding; the arithmetic of moe_rmsnorm), written to x_out [hidden] fp16, then
 * y_out = x + sum_j scores[j] * D_j relu(U_j x)^2.  The norm runs inside the up-projection (every
 * block normalises h while its weight loads are in flight), so the layer is two launches, not three.
 * norm_w may be null (no weight). */
int moe_cb_moe_norm(const float* h_in, const void* norm_w, float eps, void* x_out, const void* pool,
                    uint64_t stride, int n_slots, const uint32_t* slots, const void* scores, int k,
                    int hidden, int inter, const void* grid, void* h_ws, float* y_out, void* stream);

/* ---- Part 3: no counterpart in the reference ----------------------------------------------- */

/* Last recorded failure ("" if none) / clear it. */
const char* c_last_error(void);
void c_clear_error(void);
/* Stream that Part-1 entry points order their slot-id writes and waits on. */
int c_set_compute_stream(void* stream);
/* Pinned, device-mapped host memory for expert stores. */
void* c_host_alloc(uint64_t bytes);
int c_host_free(void* p);
/* Declare tensor 0 of a layer as a Q2 blob pool (row_bytes[0] == moe_q2_expert_bytes). */
int c_layer_set_format(int layer_idx, int hidden, int inter, int group);
/* Declare the layer's 9 tensors, as loader.py:332-406 passes them to c_layer_init (sorted by file
 * offset), to be the Q2 projections: roles[t] is the role of tensor t (MOE_Q2T_*); each tensor's
 * row_bytes must be its size per expert; scale_bf16 as moe_q2t_switch_glu.  c_layer_switch_glu and
 * c_layer_switch_glu_split then read the 9 pools in place. */
enum { MOE_Q2T_GATE_W = 0, MOE_Q2T_GATE_S, MOE_Q2T_GATE_B, MOE_Q2T_UP_W, MOE_Q2T_UP_S, MOE_Q2T_UP_B,
       MOE_Q2T_DOWN_W, MOE_Q2T_DOWN_S, MOE_Q2T_DOWN_B };
int c_layer_set_format9(int layer_idx, int hidden, int inter, int group, const int32_t* roles, int scale_bf16);
/* The prefill grouped SwitchGLU (as moe_q2_grouped_switch_glu) over the 9 tensors' pools (as
 * moe_q2t_switch_glu: ptrs / slot_bytes in MOE_Q2T_* role order, scale_bf16); hidden and inter
 * multiples of 64 up to 2560.  c_layer_grouped_switch_glu takes this path for format9 layers. */
int moe_q2t_grouped_switch_glu(const void* x, int n_tokens, const int32_t* row_token, const int32_t* row_out,
                               int n_rows, int n_out_rows, const int32_t* seg_start, const int32_t* seg_slot, int n_seg,
                               const uint64_t* ptrs, const uint64_t* slot_bytes, int scale_bf16, int n_slots, int hidden,
                               int inter, int group, void* h_ws, void* y_out, void* stream);
/* SwitchGLU over the layer's pool with its current slot ids; orders after pending copies. */
int c_layer_switch_glu(int layer_idx, const void* x, const void* scores, const void* residual,
                       void* h_ws, float* y_out, int per_expert, int k, void* stream);
/* Prefill grouped SwitchGLU over the layer's pool, segment u reading slot u (the chunk-local
 * slot of loader.py:653-664); orders after pending copies and records the read so the next
 * chunk's copies (c_layer_load_sync) wait for it.  Arguments as moe_q2_grouped_switch_glu. */
int c_layer_grouped_switch_glu(int layer_idx, const void* x, int n_tokens, const int32_t* row_token,
                               const int32_t* row_out, int n_rows, int n_out_rows,
                               const int32_t* seg_start, int n_seg, void* h_ws, void* y_out,
                               void* stream);
/* Split SwitchGLU after c_layer_decode_step_sched with MOE_SCHED_SPLIT (the purpose of the
 * reference's split lists, cpp/third_party/expert_io.c:1257-1276,1380-1390: hit experts start
 * before the misses land).  part 0: the hit experts, after the layer's prefetch copies only,
 * y_out = residual + their sum; part 1: after the demand copies, y_out += the missed experts'
 * sum.  scores in router order; both parts on one stream, part 0 first. */
int c_layer_switch_glu_split(int layer_idx, int part, const void* x, const void* scores,
                             const void* residual, void* h_ws, float* y_out, void* stream);
/* Device-driven tables follow the scheduler variant's decisions (bit 0 of on) or the published
 * ones (the default); with bit 1 also set, their steps record the split lists as
 * MOE_SCHED_SPLIT does (read with c_layer_get_split_inds). */
int c_layer_set_sched(int layer_idx, int on);
/* Record that work queued on `stream` so far reads the layer's pool (copies into it wait). */
int c_layer_mark_read(int layer_idx, void* stream);
/* Move a layer's slot table to device memory (on != 0) or back.  Device-driven layers take
 * their ids from device memory and stage misses with a kernel that reads the pinned store, or,
 * for a file-backed layer (fd >= 0), the bounce entries the feeder thread reads the published
 * misses into (c_layer_publish_dev).  No reference counterpart: the reference's tables live on
 * the host (expert_io.c:583-708). */
int c_layer_set_device_mode(int layer_idx, int on);
/* Device-driven decode step / prefetch (same decisions as c_layer_step_decode_ex /
 * c_layer_start_prefetch), queued on `stream`; stage_ctas == 0 picks a default staging grid,
 * stage_ctas < 0 updates the table only (queue the copies with c_layer_stage_dev). */
int c_layer_step_decode_dev(int layer_idx, const uint32_t* ids_dev, int k, int stage_ctas,
                            void* stream);
int c_layer_start_prefetch_dev(int layer_idx, const int32_t* preds_dev, int m, int max_fetch,
                               int stage_ctas, void* stream);
/* moe_router whose last block also runs the decode step of device-driven layer step_layer with
 * the selected ids (slot ids into its slot_inds) and the prefetch of device-driven layer
 * pf_layer with the prediction (-1: none).  Same decisions as moe_router followed by
 * c_layer_step_decode_dev(step_layer, ids) and c_layer_start_prefetch_dev(pf_layer, pred),
 * without their two launches; copies are then queued with c_layer_stage_dev. */
int c_router_tables_dev(int step_layer, int pf_layer, int max_fetch, const float* h_in,
                        const void* norm_w, float eps, const void* x_in, void* x_out, const void* w,
                        const void* w_next, int hidden, int n_exp, int k, int m, void* workspace,
                        uint32_t* ids_out, void* scores_out, int32_t* pred_out, void* stream);
/* Queue the copies of the layer's last device-side decode step (list 0) or prefetch (list 1)
 * on `stream` (the two lists are kept apart so a step may run while prefetch copies queue). */
int c_layer_stage_dev(int layer_idx, int list, int stage_ctas, void* stream);
/* File-backed device-driven layers: publish the copy list of the layer's last device-side decode
 * step (list 0) or prefetch (list 1) to the feeder thread, queued on `stream` after that table
 * operation and before c_layer_stage_dev of the same list.  The feeder reads the listed experts
 * (the reader threads, one read per expert and tensor, O_DIRECT when c_io_set_direct was on at
 * c_layer_init) into the layer's bounce entries; the staging kernel waits for each entry and
 * copies it into its slot.  Replaces the reference's step-time reads of the misses
 * (expert_io.c:187-356, 583-685) for tables that run on the GPU. */
int c_layer_publish_dev(int layer_idx, int list, void* stream);
/* No counterpart in the reference (its reads block the calling thread, expert_io.c:312-356).
 * Longest a file-backed staging kernel waits for one expert's read (0: 10 s); past it the
 * layer's table status becomes 17 (a failed read: 16).  Applies to copies queued afterwards.
 * Both faults are sticky: the slot keeps its old bytes, so the table stays faulted (and its
 * later stagings copy nothing) until c_layer_reset_cache.  Staging a list that a table
 * operation changed since its last c_layer_publish_dev fails with -1. */
void c_io_set_feed_timeout_us(uint64_t us);
/* No counterpart in the reference (its reads report nothing: expert_io.c:118-127).  The
 * library-wide sticky fault word of the device-driven file tier: 0, or the code (16 / 17) a
 * staging kernel last stored on a failed read or a timed-out wait.  Host memory, so it is read
 * without synchronising the GPU (it reflects the kernels that have run); cleared by
 * c_io_clear_fault. */
int c_io_fault(void);
void c_io_clear_fault(void);
/* Device address of a device-driven layer's table; 0 otherwise. */
uint64_t c_layer_device_table(int layer_idx);
/* Status word of a device-driven table: the sticky file-tier fault if any (16 a file-backed
 * layer's read failed, 17 its staging wait timed out; cleared by c_layer_reset_cache), else that
 * of the last device-side table operation (0 ok, 1 id out of range, 2 repeated id); blocks.  (The reference accepts repeated ids and leaks a slot; both paths here reject them.) */
int c_layer_table_status(int layer_idx);
/* Block the host until every queued copy has landed. */
int c_sync_copies(void);
/* Per-kernel timing: launches between begin and end are dispatched with start/stop events
 * stamped at the kernel's own begin/end; end() sums durations per kind (0 router, 1 gate/up,
 * 2 down, 3 staging, 4 slot table, 5 grouped gate/up, 6 grouped down, 7 pair combine,
 * 8 codebook up, 9 codebook down, 10 streaming calibration) into out_ms[MOE_TIMING_KINDS] and
 * counts into out_n[MOE_TIMING_KINDS]. */
#define MOE_TIMING_KINDS 11
int c_timing_begin(int capacity);
int c_timing_end(double* out_ms, int* out_n);
/* Plain device-to-device copy of `bytes` (multiple of 16): the known-size reference for scaling
 * per-dispatch memory counters (FETCH_SIZE, WRITE_SIZE) to bytes. */
int moe_calibrate_copy(void* dst, const void* src, uint64_t bytes, void* stream);
/* Read-only streaming of `bytes` (multiple of 16) with `grid` blocks of 256 threads: the
 * single-launch floor for a kernel of that many HBM bytes (out: 4-byte device scratch). */
int moe_calibrate_stream(const void* src, uint64_t bytes, int grid, float* out, void* stream);
int c_abi_version(void);

/* ---- Part 3b: native host-driven decode token ---------------------------------------------- */
/* No counterpart in the reference's C ABI: the C++ runner's per-layer loop (cpp/src/engine.cpp:
 * 572-660, loader.py:920-977) over the entry points above, for host-driven layers.  Layer 0's
 * experts are all resident in pool0 (slot == expert id); layers 1.. are cached layers
 * layer_base + l set up with c_layer_init / c_layer_set_format.  Per layer the router writes its
 * ids and next-layer predictions into pinned host memory (ids_host, pred_host: c_host_alloc), the
 * host steps the table (copies queued to the DMA engines), launches the SwitchGLU and the next
 * layer's prefetch.  Shapes of the buffers (fp16 unless noted):
 *   xs [n_layers + 1][hidden] (xs[0] is the token's input, xs[n_layers] its output), hs fp32
 *   [n_layers][hidden], router_w [n_layers][n_exp][hidden], norm_w [n_layers][hidden], scores
 *   [n_layers][top_k], ids0 u32 [top_k] (device), ids_host u32 [n_layers][top_k], pred_host i32
 *   [n_layers][top_m], router_ws n_layers x router_ws_bytes (moe_router_workspace_bytes), h_ws
 *   [top_k * inter]. */
typedef struct moe_stack_desc {
    int n_layers, layer_base, hidden, n_exp, top_k, top_m, inter, group, prefetch, prefetch_cap;
    float eps;
    void* xs;
    float* hs;
    const void* router_w;
    const void* norm_w;
    void* scores;
    uint32_t* ids0;
    uint32_t* ids_host;
    int32_t* pred_host;
    void* router_ws;
    uint64_t router_ws_bytes;
    const void* pool0;
    uint64_t blob_bytes;
    void* h_ws;
} moe_stack_desc;
int moe_stack_token_host(const moe_stack_desc* d, void* stream);

/* ---- Part 4: P1 I/O scheduler (mlx-qwen38/cpp/src/io_sched.h:46-245) ---------------------- */
/* The C++ runner's `--io p1` cache: urgent and prefetch read queues served by reader threads,
 * cancel / promote of queued prefetches, slots pinned while a GPU reader uses them, resize and
 * forced invalidation.  One handle per scheduler (the reference's class instance); each function
 * below is the method of the same name (include/moe_io_sched.hpp wraps them in that class).
 * Slot pools may be HBM (reads are staged in pinned memory and copied by DMA; a read is done once
 * its copy has completed) or host memory (read into directly).  Counters: 16 values in the order of
 * P1LayerStats (io_sched.h:23-44). */
typedef struct moe_p1 moe_p1;
typedef void (*moe_p1_reader_fn)(int layer_idx, void* user);
typedef double (*moe_p1_uniform_fn)(void* user);
/* io_sched.h:48-49 (constructor, destructor: shuts the readers down) */
moe_p1* moe_p1_create(void);
void moe_p1_destroy(moe_p1* p);
/* io_sched.h:54.  num_threads in 0..32; 0 runs every read inside the waits (the reference
 * clamps to at least 1 thread). */
void moe_p1_init(moe_p1* p, int num_threads);
/* io_sched.h:55 */
void moe_p1_shutdown(moe_p1* p);
/* io_sched.h:146 */
int moe_p1_num_threads(moe_p1* p);
/* io_sched.h:57.  Called (without the scheduler's lock) when an allocation meets slots pinned by
 * a GPU reader; it must end that reader and unpin (moe_p1_unpin_layer_slots).  fn == NULL: the
 * scheduler waits for the layer's moe_p1_mark_read event and unpins the layer's slots itself. */
void moe_p1_set_wait_reader_callback(moe_p1* p, moe_p1_reader_fn fn, void* user);
/* No counterpart: the stream on which slot ids are written to device memory (default: null
 * stream), and the event marking the end of layer l's GPU reader (recorded on `stream`). */
void moe_p1_set_compute_stream(moe_p1* p, void* stream);
int moe_p1_mark_read(moe_p1* p, int layer_idx, void* stream);
/* io_sched.h:59-67 */
void moe_p1_layer_init(moe_p1* p, int layer_idx, int fd, int capacity, int num_tensors,
                       const uint64_t* base_offsets, const uint64_t* row_bytes, const uint64_t* base_ptrs,
                       uint64_t slot_inds_ptr);
/* io_sched.h:69-76 */
void moe_p1_resize_layer(moe_p1* p, int layer_idx, int new_capacity, const uint64_t* new_base_ptrs,
                         uint64_t slot_inds_ptr, const int32_t* ordered_eids, const int32_t* ordered_slots,
                         int count);
/* io_sched.h:78-79 */
void moe_p1_reset_cache(moe_p1* p, int layer_idx);
void moe_p1_reset_stats(moe_p1* p, int layer_idx);
/* io_sched.h:82-86 */
void moe_p1_start_prefetch(moe_p1* p, int layer_idx, const int32_t* pred_eids, int pred_count, int max_fetch);
/* io_sched.h:88-98.  Pending reads the GPU must wait for (moe_p1_wait_layer_urgent); -1 with an
 * error for an expert id >= 512 or when no slot can be freed. */
int moe_p1_step_decode(moe_p1* p, int layer_idx, const uint32_t* eids, int k, uint32_t* out_slots);
/* io_sched.h:100-106 */
void moe_p1_wait_layer_urgent(moe_p1* p, int layer_idx);
void moe_p1_wait_layer_all(moe_p1* p, int layer_idx);
void moe_p1_wait_all(moe_p1* p);
/* io_sched.h:108-114 */
void moe_p1_unpin_layer_slots(moe_p1* p, int layer_idx);
void moe_p1_pin_slots(moe_p1* p, int layer_idx, const uint32_t* slots, int count);
void moe_p1_unpin_slots(moe_p1* p, int layer_idx, const uint32_t* slots, int count);
int moe_p1_get_slot_pin_count(moe_p1* p, int layer_idx, int slot);
/* io_sched.h:116-117.  The reference takes a std::mt19937_64&; here `draw(user)` returns one
 * uniform [0, 1) value per candidate slot (moe_p1_mt64_uniform over a moe_p1_mt64_create handle
 * draws exactly what std::uniform_real_distribution<double>(0, 1) does over that generator). */
int moe_p1_force_invalidate(moe_p1* p, int layer_idx, double rate, moe_p1_uniform_fn draw, void* user);
void* moe_p1_mt64_create(uint64_t seed);
void moe_p1_mt64_destroy(void* rng);
uint64_t moe_p1_mt64_next(void* rng);
double moe_p1_mt64_uniform(void* rng);
/* io_sched.h:119-125 */
void moe_p1_load_sync(moe_p1* p, int layer_idx, const int32_t* eids, const int32_t* slots, int count,
                      int is_prefill);
/* io_sched.h:127-140 */
void moe_p1_get_lru_state(moe_p1* p, int layer_idx, int32_t* out_eids, int32_t* out_slots, int* out_count);
void moe_p1_set_lru_state(moe_p1* p, int layer_idx, const int32_t* ordered_eids, const int32_t* ordered_slots,
                          int count, uint64_t add_prefill_requests, uint64_t add_prefill_hits,
                          uint64_t add_prefill_misses);
/* io_sched.h:142-143 */
void moe_p1_get_layer_stats(moe_p1* p, int layer_idx, uint64_t* out16);
void moe_p1_get_total_stats(moe_p1* p, int num_layers, uint64_t* out16);

#ifdef __cplusplus
}
#endif
#endif /* MOE_OFFLOAD_H */
