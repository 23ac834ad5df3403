"""ctypes binding of libmoe_offload.so (the C-ABI declared in include/moe_offload.h).

Loaded the same way the reference loads its native expert cache
(`mlx-qwen38/loader.py:100-220`): one CDLL with argtypes/restype set per symbol.  There is no
fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libmoe_offload.so"
SRC_DIR = PKG_DIR.parent

_c_int, _c_u32, _c_i32, _c_u64, _c_f, _c_vp = (ctypes.c_int, ctypes.c_uint32, ctypes.c_int32,
                                              ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p)
_u32p, _i32p, _u64p = (ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32),
                       ctypes.POINTER(ctypes.c_uint64))

# name -> (restype, argtypes)
class StackDesc(ctypes.Structure):
    """moe_stack_desc (include/moe_offload.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "layer_base", "hidden", "n_exp", "top_k", "top_m", "inter",
                                            "group", "prefetch", "prefetch_cap")] + [
        ("eps", ctypes.c_float), ("xs", ctypes.c_void_p), ("hs", ctypes.c_void_p), ("router_w", ctypes.c_void_p),
        ("norm_w", ctypes.c_void_p), ("scores", ctypes.c_void_p), ("ids0", ctypes.c_void_p),
        ("ids_host", ctypes.c_void_p), ("pred_host", ctypes.c_void_p), ("router_ws", ctypes.c_void_p),
        ("router_ws_bytes", ctypes.c_uint64), ("pool0", ctypes.c_void_p), ("blob_bytes", ctypes.c_uint64),
        ("h_ws", ctypes.c_void_p)]


SIGNATURES: dict[str, tuple] = {
    # expert_io.c entry points
    "c_io_init": (None, [_c_int]),
    "c_io_shutdown": (None, []),
    "c_io_set_direct": (None, [_c_int]),
    "c_layer_io_direct": (_c_int, [_c_int]),
    "c_io_threads": (_c_int, []),
    "c_io_read_ranges": (_c_int, [_c_int, _u64p, _u64p, _u64p, _c_int]),
    "c_layer_init": (None, [_c_int, _c_int, _c_int, _u64p, _u64p, _u64p, _c_u64]),
    "c_layer_reset_cache": (None, [_c_int]),
    "c_layer_reset_stats": (None, [_c_int]),
    "c_layer_step_decode_ex": (_c_int, [_c_int, _u32p, _c_int, _c_int]),
    "c_layer_step_decode": (_c_int, [_c_int, _u32p, _c_int]),
    "c_layer_step_decode10": (_c_int, [_c_int] + [_c_u32] * 10),
    "c_layer_step_decode10_async": (_c_int, [_c_int] + [_c_u32] * 10),
    "c_layer_start_prefetch": (None, [_c_int, _i32p, _c_int, _c_int]),
    "c_layer_start_prefetch10": (None, [_c_int, _c_int] + [_c_i32] * 10),
    "c_layer_start_prefetch12": (None, [_c_int, _c_int] + [_c_i32] * 12),
    "c_layer_wait_prefetch": (None, [_c_int]),
    "c_layer_load_sync": (None, [_c_int, _i32p, _i32p, _c_int, _c_int]),
    "c_layer_get_lru_state": (None, [_c_int, _i32p, _i32p, ctypes.POINTER(ctypes.c_int)]),
    "c_layer_set_lru_state": (None, [_c_int, _i32p, _i32p, _c_int, _c_u64, _c_u64, _c_u64]),
    "c_layer_get_stats": (None, [_c_int, _u64p]),
    "c_get_decode_totals": (None, [_c_int, _u64p]),
    # superset ABI of the reference's C++ runner (cpp/src/expert_io.h)
    "c_layer_decode_step_sched": (_c_int, [_c_int, _i32p, _c_int, _i32p, _c_int, _c_int, _c_int, _c_int]),
    "c_layer_get_split_inds": (None, [_c_int, _u32p, _u32p, _i32p]),
    "c_layer_wait_demand": (None, [_c_int]),
    "c_set_io_accounting": (None, [_c_int]),
    "c_begin_decode_token": (None, [_c_int]),
    "c_end_decode_token": (None, [_u64p]),
    "c_get_native_buffer_bytes": (_c_u64, []),
    # compute
    "moe_router": (_c_int, [_c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int,
                            _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_router_workspace_bytes": (_c_u64, [_c_int]),
    "moe_router_noalloc": (_c_int, [_c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int,
                                    _c_int, _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_router_logits": (_c_int, [_c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp]),
    "moe_q2_gate_up_routed": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_u64, _c_int, _c_int, _c_int, _c_vp,
                                       _c_vp, _c_vp, _c_vp]),
    "moe_rmsnorm": (_c_int, [_c_vp, _c_vp, _c_f, _c_int, _c_vp, _c_vp]),
    "moe_rmsnorm_bf16": (_c_int, [_c_vp, _c_vp, _c_f, _c_int, _c_vp, _c_vp, _c_vp]),
    "moe_f64_to_f16": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "moe_q2_expert_bytes": (_c_u64, [_c_int, _c_int, _c_int]),
    "moe_q2_gate_up": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp,
                                _c_vp]),
    "moe_q2_down": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                             _c_vp, _c_vp, _c_int, _c_vp]),
    "moe_q2_switch_glu": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                   _c_vp, _c_vp, _c_vp, _c_int, _c_vp]),
    "moe_q2t_gate_up": (_c_int, [_c_vp, _u64p, _u64p, _c_int, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp,
                                 _c_vp]),
    "moe_q2t_gate_up_routed": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _u64p, _u64p, _c_int, _c_int, _c_int, _c_int,
                                        _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_q2t_down": (_c_int, [_c_vp, _u64p, _u64p, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp,
                              _c_vp, _c_int, _c_vp]),
    "moe_q2t_switch_glu": (_c_int, [_c_vp, _u64p, _u64p, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                    _c_vp, _c_vp, _c_vp, _c_int, _c_vp]),
    "moe_q2_grouped_gate_up": (_c_int, [_c_vp, _c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_u64, _c_int,
                                        _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "moe_q2_grouped_down": (_c_int, [_c_vp, _c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_u64, _c_int,
                                     _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "moe_q2_grouped_switch_glu": (_c_int, [_c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_vp,
                                           _c_u64, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "moe_cb_expert_bytes": (_c_u64, [_c_int, _c_int]),
    "moe_cb_up": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "moe_cb_down": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                             _c_int, _c_vp]),
    "moe_cb_moe": (_c_int, [_c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                            _c_vp, _c_int, _c_vp]),
    "moe_cb_moe_norm": (_c_int, [_c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_u64, _c_int, _c_vp, _c_vp, _c_int,
                                 _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_pair_combine": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    # no reference counterpart
    "c_last_error": (ctypes.c_char_p, []),
    "c_clear_error": (None, []),
    "c_set_compute_stream": (_c_int, [_c_vp]),
    "c_host_alloc": (_c_vp, [_c_u64]),
    "c_host_free": (_c_int, [_c_vp]),
    "c_layer_set_format": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "c_layer_set_format9": (_c_int, [_c_int, _c_int, _c_int, _c_int, _i32p, _c_int]),
    "moe_q2t_grouped_switch_glu": (_c_int, [_c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_int, _u64p,
                                            _u64p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "c_layer_switch_glu": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp]),
    "c_layer_mark_read": (_c_int, [_c_int, _c_vp]),
    "c_router_tables_dev": (_c_int, [_c_int, _c_int, _c_int, _c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_vp, _c_vp, _c_int,
                                     _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "c_layer_grouped_switch_glu": (_c_int, [_c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_int, _c_vp,
                                            _c_vp, _c_vp]),
    "c_layer_set_device_mode": (_c_int, [_c_int, _c_int]),
    "c_layer_set_sched": (_c_int, [_c_int, _c_int]),
    "c_layer_switch_glu_split": (_c_int, [_c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "c_layer_step_decode_dev": (_c_int, [_c_int, _c_vp, _c_int, _c_int, _c_vp]),
    "c_layer_start_prefetch_dev": (_c_int, [_c_int, _c_vp, _c_int, _c_int, _c_int, _c_vp]),
    "c_layer_stage_dev": (_c_int, [_c_int, _c_int, _c_int, _c_vp]),
    "c_layer_publish_dev": (_c_int, [_c_int, _c_int, _c_vp]),
    "c_io_set_feed_timeout_us": (None, [_c_u64]),
    "c_layer_device_table": (_c_u64, [_c_int]),
    "c_layer_table_status": (_c_int, [_c_int]),
    "c_io_fault": (_c_int, []),
    "c_io_clear_fault": (None, []),
    "c_sync_copies": (_c_int, []),
    "c_timing_begin": (_c_int, [_c_int]),
    "c_timing_end": (_c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]),
    "moe_calibrate_copy": (_c_int, [_c_vp, _c_vp, _c_u64, _c_vp]),
    "moe_calibrate_stream": (_c_int, [_c_vp, _c_u64, _c_int, _c_vp, _c_vp]),
    "c_abi_version": (_c_int, []),
    "moe_stack_token_host": (_c_int, [_c_vp, _c_vp]),
    "moe_router_q8_workspace_bytes": (_c_u64, [_c_int]),
    "moe_router_q8": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp,
                               _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_router_q8_norm": (_c_int, [_c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int,
                                    _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    # P1 I/O scheduler (cpp/src/io_sched.h)
    "moe_p1_create": (_c_vp, []),
    "moe_p1_destroy": (None, [_c_vp]),
    "moe_p1_init": (None, [_c_vp, _c_int]),
    "moe_p1_shutdown": (None, [_c_vp]),
    "moe_p1_num_threads": (_c_int, [_c_vp]),
    "moe_p1_set_wait_reader_callback": (None, [_c_vp, _c_vp, _c_vp]),
    "moe_p1_set_compute_stream": (None, [_c_vp, _c_vp]),
    "moe_p1_mark_read": (_c_int, [_c_vp, _c_int, _c_vp]),
    "moe_p1_layer_init": (None, [_c_vp, _c_int, _c_int, _c_int, _c_int, _u64p, _u64p, _u64p, _c_u64]),
    "moe_p1_resize_layer": (None, [_c_vp, _c_int, _c_int, _u64p, _c_u64, _i32p, _i32p, _c_int]),
    "moe_p1_reset_cache": (None, [_c_vp, _c_int]),
    "moe_p1_reset_stats": (None, [_c_vp, _c_int]),
    "moe_p1_start_prefetch": (None, [_c_vp, _c_int, _i32p, _c_int, _c_int]),
    "moe_p1_step_decode": (_c_int, [_c_vp, _c_int, _u32p, _c_int, _u32p]),
    "moe_p1_wait_layer_urgent": (None, [_c_vp, _c_int]),
    "moe_p1_wait_layer_all": (None, [_c_vp, _c_int]),
    "moe_p1_wait_all": (None, [_c_vp]),
    "moe_p1_unpin_layer_slots": (None, [_c_vp, _c_int]),
    "moe_p1_pin_slots": (None, [_c_vp, _c_int, _u32p, _c_int]),
    "moe_p1_unpin_slots": (None, [_c_vp, _c_int, _u32p, _c_int]),
    "moe_p1_get_slot_pin_count": (_c_int, [_c_vp, _c_int, _c_int]),
    "moe_p1_force_invalidate": (_c_int, [_c_vp, _c_int, ctypes.c_double, _c_vp, _c_vp]),
    "moe_p1_mt64_create": (_c_vp, [_c_u64]),
    "moe_p1_mt64_destroy": (None, [_c_vp]),
    "moe_p1_mt64_next": (_c_u64, [_c_vp]),
    "moe_p1_mt64_uniform": (ctypes.c_double, [_c_vp]),
    "moe_p1_load_sync": (None, [_c_vp, _c_int, _i32p, _i32p, _c_int, _c_int]),
    "moe_p1_get_lru_state": (None, [_c_vp, _c_int, _i32p, _i32p, ctypes.POINTER(ctypes.c_int)]),
    "moe_p1_set_lru_state": (None, [_c_vp, _c_int, _i32p, _i32p, _c_int, _c_u64, _c_u64, _c_u64]),
    "moe_p1_get_layer_stats": (None, [_c_vp, _c_int, _u64p]),
    "moe_p1_get_total_stats": (None, [_c_vp, _c_int, _u64p]),
}


class NativeError(RuntimeError):
    pass


def build(verbose: bool = False) -> None:
    """Compile libmoe_offload.so for gfx950 in-tree (hipcc via moe-offload_amd/Makefile)."""
    r = subprocess.run(["make", "-C", str(SRC_DIR), "-B"], capture_output=not verbose, text=True)
    if r.returncode != 0:
        raise NativeError(f"libmoe_offload build failed:\n{r.stdout}\n{r.stderr}")


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises NativeError if it is missing (no CPU fallback exists)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise NativeError(f"{LIB_PATH} not found: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def last_error() -> str:
    msg = lib().c_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str = "") -> int:
    """Raise NativeError (with the library's recorded message) when rc < 0 or an error is pending."""
    err = last_error()
    if (rc is not None and rc < 0) or err:
        lib().c_clear_error()
        raise NativeError(f"{what}: {err or 'failed'}")
    return rc


def check_error(what: str = "") -> None:
    """For void entry points: raise if the library recorded a failure."""
    err = last_error()
    if err:
        lib().c_clear_error()
        raise NativeError(f"{what}: {err}")
