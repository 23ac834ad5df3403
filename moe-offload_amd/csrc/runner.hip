// Host-driven decode token in native code: the C++ runner's per-layer loop (cpp/src/engine.cpp:
// 572-660, loader.py:920-977's order) over this library's entry points, so the host's part of
// each layer -- reading the router's ids, the slot-table step, queueing the DMA copies, the next
// layer's prefetch -- costs microseconds instead of an interpreter's tens of microseconds.
//
// Per cached layer: router(l) writes its ids and next-layer predictions straight into pinned host
// memory (mapped, so the kernel's stores land there); the host waits for the router's event,
// steps the layer's table (copies of the misses queued to the DMA engines, slot ids written on
// the compute stream), launches the SwitchGLU (it waits on the GPU for this layer's copies), then
// runs the next layer's prefetch (its copies queue behind this layer's demand copies, so the link
// stays busy while the GLU and the next router run).  Layer 0's experts are all resident.
#include <string.h>

#include <chrono>

#include "moe_common.h"
#include "moe_offload.h"

namespace {

hipEvent_t g_router_done = nullptr;

// The router event has fired (the ids and predictions are in host memory).  Spins on the event:
// the wait is a few microseconds and sits on the token's critical path.  A router that has not
// finished after kRouterWaitSec (a stalled device) is reported as an error instead of spinning on.
constexpr double kRouterWaitSec = 10.0;

int wait_router(hipStream_t s) {
    if (!g_router_done) HIP_TRY(hipEventCreateWithFlags(&g_router_done, hipEventDisableTiming));
    HIP_TRY(hipEventRecord(g_router_done, s));
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t n = 0;; ++n) {
        const hipError_t e = hipEventQuery(g_router_done);
        if (e == hipSuccess) return 0;
        if (e != hipErrorNotReady) {
            moe_set_error("runner: router event: %s", hipGetErrorString(e));
            return -1;
        }
        if ((n & 1023u) == 1023u &&
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kRouterWaitSec) {
            moe_set_error("runner: the router has not finished after %.0f s", kRouterWaitSec);
            return -1;
        }
    }
}

bool desc_ok(const moe_stack_desc* d) {
    if (!d) return false;
    if (d->n_layers < 1 || d->layer_base < 0 || d->layer_base + d->n_layers > MOE_MAX_LAYERS) return false;
    if (d->top_k < 1 || d->top_k > MOE_MAX_K || d->top_m < 0 || d->top_m > MOE_MAX_PREFETCH) return false;
    if (!d->xs || !d->hs || !d->router_w || !d->norm_w || !d->scores || !d->ids0 || !d->ids_host ||
        !d->router_ws || !d->pool0 || !d->h_ws)
        return false;
    if (d->prefetch && d->n_layers > 1 && !d->pred_host) return false;
    return true;
}

}  // namespace

extern "C" int moe_stack_token_host(const moe_stack_desc* d, void* stream) {
    if (!desc_ok(d)) {
        moe_set_error("moe_stack_token_host: bad descriptor (layers, k, m or a null buffer)");
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    if (c_set_compute_stream(stream)) return -1;
    const int H = d->hidden, k = d->top_k, m = d->top_m;
    const size_t xb = (size_t)H * sizeof(__half);
    char* xs = (char*)d->xs;
    const char* rw = (const char*)d->router_w;
    const size_t rw_layer = (size_t)d->n_exp * H * sizeof(__half);
    const char* nw = (const char*)d->norm_w;
    char* sc = (char*)d->scores;
    for (int l = 0; l < d->n_layers; ++l) {
        const bool pf = d->prefetch && l + 1 < d->n_layers;
        const float* h_in = l ? d->hs + (size_t)(l - 1) * H : nullptr;
        const void* norm = l ? nw + (size_t)(l - 1) * xb : nullptr;
        const void* x_in = l ? nullptr : xs;
        void* x_out = l ? xs + (size_t)l * xb : nullptr;
        uint32_t* ids = l ? d->ids_host + (size_t)l * k : d->ids0;
        int32_t* pred = pf ? d->pred_host + (size_t)l * m : nullptr;
        void* scores = sc + (size_t)l * k * sizeof(__half);
        if (moe_router(h_in, norm, d->eps, x_in, x_out, rw + (size_t)l * rw_layer, pf ? rw + (size_t)(l + 1) * rw_layer : nullptr,
                       H, d->n_exp, k, pf ? m : 0, (char*)d->router_ws + (size_t)l * d->router_ws_bytes, ids, scores, pred,
                       stream))
            return -1;
        void* x_l = xs + (size_t)l * xb;
        float* y_l = d->hs + (size_t)l * H;
        if (l == 0) {
            if (moe_q2_switch_glu(x_l, d->pool0, d->blob_bytes, d->n_exp, d->ids0, scores, k, H, d->inter, d->group,
                                  x_l, d->h_ws, y_l, 0, stream))
                return -1;
            if (pf) {
                if (wait_router(s)) return -1;
                c_layer_start_prefetch(d->layer_base + 1, pred, m, d->prefetch_cap);
            }
            continue;
        }
        if (wait_router(s)) return -1;
        const int li = d->layer_base + l;
        if (c_layer_step_decode_ex(li, ids, k, 1) < 0) return -1;
        if (c_layer_switch_glu(li, x_l, scores, x_l, d->h_ws, y_l, 0, k, stream)) return -1;
        if (pf) c_layer_start_prefetch(li + 1, pred, m, d->prefetch_cap);
        if (c_last_error()[0]) return -1;
    }
    if (moe_rmsnorm(d->hs + (size_t)(d->n_layers - 1) * H, nw + (size_t)(d->n_layers - 1) * xb, d->eps, H,
                    xs + (size_t)d->n_layers * xb, stream))
        return -1;
    return c_last_error()[0] ? -1 : 0;
}
