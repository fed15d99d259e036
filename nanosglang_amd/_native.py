"""ctypes binding of libnsg_spec.so (declared in include/nsg_spec.h).

The library is the product path: there is no CPU or PyTorch fallback.  If it
is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libnsg_spec.so")

NSG_ATTN_WORK_INTS = 8
ABI_VERSION = 21

i32, i64, u32, u64, f32 = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float
vp = C.c_void_p


class AttnPlan(C.Structure):
    """Mirror of nsg_attn_plan_t."""
    _fields_ = [
        ("num_work", i32), ("num_merge", i32), ("num_groups", i32), ("row_tiles", i32), ("q_tile_tokens", i32),
        ("max_splits", i32), ("head_dim", i32), ("num_qo_heads", i32), ("num_kv_heads", i32),
        ("kv_groups", i32), ("workspace_bytes", i64),
    ]


class StepBufs(C.Structure):
    """Mirror of nsg_spec_step_bufs_t (host staging pointers of one step)."""
    _fields_ = [
        ("token0", vp), ("start", vp), ("draft_pos", vp), ("draft_slot", vp),
        ("verify_pos", vp), ("verify_slot", vp), ("qo_indptr", vp), ("kv_indptr", vp),
        ("kv_last_page_len", vp), ("kv_indices", vp), ("work", vp),
        ("indptr_stride", i32), ("indices_stride", i32), ("work_stride", i32),
    ]


# name -> (restype, argtypes); every symbol include/nsg_spec.h declares.
SIGNATURES = {
    "nsg_last_error": (C.c_char_p, []),
    "nsg_abi_version": (i32, []),
    "nsg_attn_plan": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, i32,
                            C.POINTER(AttnPlan)]),
    "nsg_attn_fixed_capacity": (i32, [i32, i32, i32, i32, i32, i32, C.POINTER(i32),
                                      C.POINTER(i32)]),
    "nsg_attn_plan_fixed": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, i32, i32,
                                  i32, vp, i32, C.POINTER(AttnPlan)]),
    "nsg_attn_workspace_bytes": (i64, [C.POINTER(AttnPlan)]),
    "nsg_linear_max_rows": (i32, []),
    "nsg_linear_preferred": (i32, [i32, i32, i32]),
    "nsg_linear": (i32, [vp, i64, vp, i64, vp, vp, i64, i32, i32, i32, i32, vp]),
    "nsg_linear_fp8": (i32, [vp, i64, vp, i64, vp, vp, vp, i64, i32, i32, i32, i32, vp]),
    "nsg_linear_rope_kv_fp8": (i32, [vp, i64, vp, i64, vp, vp, i32, i32, i32, i32, i32, vp, vp,
                                     vp, i32, vp, vp, vp, vp, i64, vp, vp]),
    "nsg_linear_rope_kv": (i32, [vp, i64, vp, i64, vp, i32, i32, i32, i32, i32, vp, vp, vp,
                                 i32, vp, vp, vp, vp, i64, vp, vp]),
    "nsg_attn_run": (i32, [C.POINTER(AttnPlan), vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32,
                           f32, i32, vp, i64, vp]),
    "nsg_attn_check_flags": (i32, [vp, C.POINTER(i32), vp]),
    "nsg_spec_accept_check_flags": (i32, [vp, i64, C.POINTER(i32), vp]),
    "nsg_spec_accept_greedy_tokens": (i32, [vp, vp, i64, i64, i32, i32, i32, vp, vp, vp, i32,
                                            vp, vp, vp, vp, vp]),
    "nsg_spec_accept_greedy_keys": (i32, [vp, i32, vp, vp, i64, i64, i32, i32, i32, vp, vp, vp,
                                          i32, vp, vp, vp, vp, vp]),
    "nsg_spec_accept_workspace_bytes": (i64, [i32, i32, i32]),
    "nsg_spec_accept": (i32, [vp, i64, i64, vp, i64, i64, i32, vp, vp, vp, i32, i32, i32, f32,
                              vp, vp, vp, i32, vp, vp, vp, vp, i64, vp]),
    "nsg_spec_accept_noalloc_max_bytes": (i64, []),
    "nsg_spec_accept_noalloc_reset": (i32, [vp]),
    "nsg_spec_accept_noalloc": (i32, [vp, i64, i64, vp, i64, i64, i32, vp, vp, vp, i32, i32, i32,
                                      f32, vp, vp, vp, i32, vp, vp, vp, vp, vp]),
    "nsg_sample_workspace_bytes": (i64, [i32, i32]),
    "nsg_dequant_fp8": (i32, [vp, i64, vp, vp, i64, i32, i32, vp]),
    "nsg_sample": (i32, [vp, i64, i32, i32, i32, f32, i32, f32, vp, i64, vp, vp, i64, vp]),
    "nsg_kv_write": (i32, [vp, vp, i64, vp, i32, vp, vp, i32, i32, i64, vp]),
    "nsg_kv_clear_slots": (i32, [vp, i32, vp, vp, i32, i64, i32, i32, i64, vp]),
    "nsg_rope_kv_write": (i32, [vp, i64, vp, vp, vp, i32, vp, i32, i32, i32, i32, vp, vp, vp,
                                i64, vp, vp]),
    "nsg_rmsnorm": (i32, [vp, vp, vp, vp, i32, i32, f32, vp]),
    "nsg_linear_fold": (i32, [vp, i64, vp, i64, vp, vp, i64, i32, i32, i32, i32, vp, i32, i32,
                              f32, vp, i64, vp, vp]),
    "nsg_linear_rope_kv_fold": (i32, [vp, i64, vp, i64, vp, i32, i32, i32, i32, i32, vp, vp, vp,
                                      i32, vp, vp, vp, vp, i64, vp, vp, i32, i32, f32, vp]),
    "nsg_row_sumsq": (i32, [vp, i64, i32, i32, vp, vp]),
    "nsg_linear_argmax_workspace_bytes": (i64, [i32, i32]),
    "nsg_linear_argmax": (i32, [vp, i64, vp, i64, vp, i32, i32, i32, vp, i64, vp, i64, vp]),
    "nsg_lm_head_fold_supported": (i32, [i32, i32, i32, i32]),
    "nsg_lm_head_fold": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, vp, i32, i32, f32, vp]),
    "nsg_lm_head_fold_argmax": (i32, [vp, i64, vp, i64, i32, i32, i32, vp, i32, i32, f32, vp,
                                      i64, vp, i64, vp]),
    "nsg_embed_rows": (i32, [vp, i64, i64, i32, i32, vp, i64, i32, i32, vp, i64, vp, vp]),
    "nsg_lm_head_fold_keys": (i32, [vp, i64, vp, i64, i32, i32, i32, vp, i32, i32, f32, vp, i64,
                                    vp, vp]),
    "nsg_embed_rows_keys": (i32, [vp, i64, i64, i32, i32, i32, vp, i32, vp, i64, i32, i32, vp,
                                  i64, vp, vp]),
    "nsg_silu_mul": (i32, [vp, vp, i64, i32, vp]),
    "nsg_philox_uniform": (i32, [u64, u32, u64, i64, vp, vp]),
    "nsg_export_step": (i32, [vp, vp, i32, i32, vp, vp, vp, vp]),
    "nsg_host_gate_wait_segments": (i32, [vp, i32, vp, i64, vp, vp, i64, vp, vp, i32, vp]),
    "nsg_host_gate_alloc": (i32, [C.POINTER(C.c_void_p)]),
    "nsg_host_gate_free": (i32, [vp]),
    "nsg_host_gate_wait": (i32, [vp, vp, i64, vp, vp, i64, vp]),
    "nsg_spec_step_fill": (i32, [vp, i64, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                 i32, i32, i32, C.POINTER(StepBufs), C.POINTER(AttnPlan)]),
    "nsg_spec_step_fill_next": (i32, [vp, i64, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32,
                                      i32, i32, i32, i32, i32, C.POINTER(StepBufs),
                                      C.POINTER(AttnPlan), C.POINTER(i32)]),
}

_lib = None


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load(path: str | None = None) -> C.CDLL:
    """Load (once) and type the library.  Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"{p} not found: build the HIP library first (python -m nanosglang_amd.build)")
    lib = C.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.nsg_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI {lib.nsg_abi_version()} != expected {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().nsg_last_error().decode(errors="replace")
        raise NativeError(f"{what} failed (status {rc}): {msg}")
