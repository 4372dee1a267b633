"""ctypes binding of libgrws.so (the C ABI declared in include/grws.h).

The library is the only compute path: if it is missing or fails to load,
every op raises (there is no CPU or PyTorch fallback).  torch is imported
first so that libgrws.so binds to the HIP runtime torch already loaded.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading libgrws.so)

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("GRWS_LIB", os.path.join(_PKG, "libgrws.so"))

GRWS_F32, GRWS_F16, GRWS_BF16 = 0, 1, 2
GRWS_OK = 0
GRWS_E_INVALID, GRWS_E_DTYPE, GRWS_E_CAPACITY, GRWS_E_HIP, GRWS_E_RANGE = -1, -2, -3, -4, -5

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p


class BcsrView(ctypes.Structure):
    """grws_bcsr (include/grws.h)."""
    _fields_ = [("window_offset", _vp), ("col_indices", _vp), ("values", _vp),
                ("num_windows", ctypes.c_int64), ("num_tiles", ctypes.c_int64),
                ("tile_rows", ctypes.c_int32), ("tile_cols", ctypes.c_int32),
                ("values_dtype", ctypes.c_int32), ("max_window_slabs", ctypes.c_int32)]


class PackedTilesView(ctypes.Structure):
    """grws_packed_tiles (include/grws.h)."""
    _fields_ = [("header", _vp), ("values", _vp), ("num_values", ctypes.c_int64)]


class GroupedTilesView(ctypes.Structure):
    """grws_grouped_tiles (include/grws.h)."""
    _fields_ = [("group_offset", _vp), ("col_indices", _vp), ("header", _vp), ("values", _vp),
                ("num_groups", ctypes.c_int64), ("num_slabs", ctypes.c_int64), ("num_values", ctypes.c_int64),
                ("max_group_slabs", ctypes.c_int64), ("num_cols", ctypes.c_int64), ("group_size", ctypes.c_int32)]


class SpmmPlanView(ctypes.Structure):
    """grws_spmm_plan (include/grws.h)."""
    _fields_ = [("items", _vp), ("split", _vp), ("num_items", ctypes.c_int64),
                ("num_split", ctypes.c_int64), ("num_slots", ctypes.c_int64),
                ("slabs_per_item", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class HacsView(ctypes.Structure):
    """grws_hacs (include/grws.h)."""
    _fields_ = [("static_scores", _vp), ("window_part_ids", _vp), ("part_starts", _vp),
                ("part_ends", _vp), ("num_static_scores", ctypes.c_int64),
                ("num_window_part_ids", ctypes.c_int64), ("num_parts", ctypes.c_int64),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("delta", ctypes.c_float),
                ("gamma_bonus", ctypes.c_float), ("score_scale", ctypes.c_float),
                ("use_hacs", ctypes.c_int32), ("locality_enabled", ctypes.c_int32)]


# name -> (restype, argtypes)
_PROTOS = {
    "grws_last_error": (ctypes.c_char_p, []),
    "grws_abi_version": (ctypes.c_int, []),
    "grws_spmm_plan_capacity": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                               ctypes.c_int32, _c_i64p, _c_i64p]),
    "grws_spmm_default_slabs": (ctypes.c_int32, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                                 ctypes.c_int64]),
    "grws_spmm_plan_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_spmm_plan_order_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_spmm_plan_order": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_size_t, _vp]),
    "grws_spmm_plan_build": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                            ctypes.c_int32, _vp, ctypes.c_int64, _vp,
                                            ctypes.c_int64, _vp, ctypes.c_size_t, _c_i64p, _vp]),
    "grws_spmm_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SpmmPlanView), ctypes.c_int64]),
    "grws_spmm": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.POINTER(SpmmPlanView), _vp,
                                 ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                 _vp, ctypes.c_int32, ctypes.c_int64, _vp, ctypes.c_size_t, _vp]),
    "grws_spmm_packed": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.POINTER(PackedTilesView),
                                        ctypes.POINTER(SpmmPlanView), _vp, ctypes.c_int32, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int32, ctypes.c_int64,
                                        _vp, ctypes.c_size_t, _vp]),
    "grws_spmm_residual": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.POINTER(PackedTilesView),
                                          ctypes.POINTER(SpmmPlanView), _vp, ctypes.c_int32, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int64,
                                          _vp, ctypes.c_int32, ctypes.c_int64, _vp, ctypes.c_size_t, _vp]),
    "grws_spmm_noalloc": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.POINTER(PackedTilesView),
                                         ctypes.POINTER(SpmmPlanView), _vp, ctypes.c_int32, ctypes.c_int64,
                                         ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int64,
                                         _vp, ctypes.c_int32, ctypes.c_int64, _vp]),
    "grws_spmm_set_tuning": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int32]),
    "grws_spmm_get_tuning": (ctypes.c_int32, [ctypes.c_char_p]),
    "grws_pack_tiles_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_pack_tiles_count": (ctypes.c_int, [ctypes.POINTER(BcsrView), _vp, ctypes.c_size_t,
                                             ctypes.POINTER(ctypes.c_int64), _vp]),
    "grws_pack_tiles_fill": (ctypes.c_int, [ctypes.POINTER(BcsrView), _vp, _vp, ctypes.c_int64, _vp,
                                            ctypes.c_size_t, _vp]),
    "grws_group_tiles_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(BcsrView), ctypes.c_int64,
                                                           ctypes.c_int32]),
    "grws_group_tiles_count": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, ctypes.c_int32, _vp,
                                              ctypes.c_size_t, _c_i64p, _c_i64p, _c_i64p, _vp]),
    "grws_group_tiles_fill": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, ctypes.c_int32,
                                             ctypes.c_int64, _vp, _vp, _vp, _vp, ctypes.c_int64, _vp,
                                             ctypes.c_size_t, _vp]),
    "grws_spmm_grouped": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.POINTER(GroupedTilesView), _vp,
                                         ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp,
                                         ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int32, ctypes.c_int64,
                                         _vp]),
    "grws_csr_to_bcsr_host_count": (ctypes.c_int, [ctypes.c_int64, _vp, _vp, ctypes.c_int32,
                                                   ctypes.c_int32, _vp, _c_i64p, ctypes.c_int32]),
    "grws_csr_to_bcsr_host_fill": (ctypes.c_int, [ctypes.c_int64, _vp, _vp, _vp, ctypes.c_int32,
                                                  ctypes.c_int32, _vp, _vp, _vp, ctypes.c_int32]),
    "grws_bcsr_build_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64,
                                                          ctypes.c_int64, ctypes.c_int32]),
    "grws_bcsr_build_count": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _vp,
                                             _vp, ctypes.c_size_t, _c_i64p, _vp]),
    "grws_bcsr_build_fill": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_int32, ctypes.c_int32, _vp, ctypes.c_int64,
                                            _vp, _vp, ctypes.c_int32, _vp, ctypes.c_size_t, _vp]),
    "grws_bcsr_to_coo_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_bcsr_to_coo_count": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp,
                                              ctypes.c_size_t, _c_i64p, _vp]),
    "grws_bcsr_to_coo_fill": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp, _vp,
                                             _vp, _vp, ctypes.c_size_t, _vp]),
    "grws_coo_to_csr_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64,
                                                          ctypes.c_int64]),
    "grws_coo_to_csr": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int64, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "grws_reindex_prune": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_int32, _vp,
                                          ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _vp, _vp]),
    "grws_sample_hop_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_sample_hop": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp,
                                       ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64, _vp, _vp,
                                       _vp, ctypes.c_int64, _vp, ctypes.c_size_t, _c_i64p, _vp]),
    "grws_window_sample_num": (ctypes.c_int32, [ctypes.c_int32]),
    "grws_window_seeds_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_window_seeds": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                         ctypes.c_int32, _vp, _vp, _vp, ctypes.c_size_t, _c_i64p,
                                         _vp]),
    "grws_window_topk_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_window_topk_key_scratch_bytes": (ctypes.c_size_t, [ctypes.POINTER(BcsrView)]),
    "grws_window_topk": (ctypes.c_int, [ctypes.POINTER(BcsrView), _vp, ctypes.c_int64,
                                        ctypes.c_int32, ctypes.POINTER(HacsView), _vp, _vp, _vp,
                                        _vp, ctypes.c_size_t, _c_i64p, _vp]),
    "grws_window_recompress": (ctypes.c_int, [ctypes.POINTER(BcsrView), _vp, ctypes.c_int64,
                                              ctypes.c_int32, _vp, _vp, _vp, ctypes.c_int64, _vp,
                                              _vp, _vp]),
    "grws_window_sample_layers_bounds": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64,
                                                        ctypes.c_int64, _vp, ctypes.c_int32, _vp, _vp]),
    "grws_window_sample_layers_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(BcsrView), ctypes.c_int64,
                                                                     ctypes.c_int64, _vp, ctypes.c_int32]),
    "grws_window_sample_layers": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp, ctypes.c_int64,
                                                 _vp, ctypes.c_int32, ctypes.POINTER(HacsView), _vp, _vp, _vp,
                                                 _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "grws_window_sample_layers_enqueue": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp,
                                                         ctypes.c_int64, _vp, _vp, ctypes.c_int32,
                                                         ctypes.POINTER(HacsView), _vp, _vp, _vp, _vp, _vp, _vp,
                                                         ctypes.c_size_t, _vp, _vp, _vp]),
    "grws_window_sample_layers_status": (ctypes.c_int, [ctypes.c_int64]),
    "grws_sample_state_init": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, _vp]),
    "grws_sample_block_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int32,
                                                            ctypes.c_int64]),
    "grws_sample_block_capacity": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                                  _c_i64p, _c_i64p]),
    "grws_sample_block": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp,
                                         ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64, _vp, _vp,
                                         ctypes.c_int32, ctypes.c_int32, _vp, ctypes.c_int64, _vp,
                                         _vp, _vp, ctypes.c_int64, _vp, ctypes.c_size_t, _c_i64p,
                                         _vp]),
    "grws_sample_blocks_state_words": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_sample_blocks_state_init": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, _vp]),
    "grws_sample_blocks_capacity": (ctypes.c_int, [ctypes.c_int64, _vp, ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.c_int64, _c_i64p, _c_i64p]),
    "grws_sample_blocks_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, _vp, ctypes.c_int32,
                                                             ctypes.c_int32, ctypes.c_int64]),
    "grws_sample_blocks": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64,
                                          _vp, ctypes.c_int32, ctypes.c_uint64, _vp, _vp, ctypes.c_int32,
                                          ctypes.c_int32, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_i64p,
                                          _vp]),
    "grws_sample_blocks_transposed_capacity": (ctypes.c_int, [ctypes.c_int64, _vp, ctypes.c_int32,
                                                              ctypes.c_int32, ctypes.c_int64, _c_i64p, _c_i64p]),
    "grws_sample_blocks_transposed_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, _vp, ctypes.c_int32,
                                                                        ctypes.c_int32, ctypes.c_int64, _vp]),
    "grws_sample_blocks_transposed": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp,
                                                     ctypes.c_int64, _vp, ctypes.c_int32, ctypes.c_uint64, _vp,
                                                     _vp, ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp,
                                                     _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_i64p, _vp]),
    "grws_sample_blocks_enqueue": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64,
                                                  _vp, _vp, ctypes.c_int32, ctypes.c_uint64, _vp, _vp,
                                                  ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp, _vp, _vp,
                                                  _vp, _vp, _vp, ctypes.c_size_t, _vp, _vp]),
    "grws_sample_blocks_error": (ctypes.c_int, [ctypes.c_int64]),
    "grws_copy_ranges": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int32, _vp]),
    "grws_fill_ranges_i64": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int32, _vp]),
    "grws_probe_row_gather": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, _vp,
                                             ctypes.c_int64, _vp, ctypes.c_int32, _vp]),
    "grws_gather_rows": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int32,
                                        ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64, _vp, _vp]),
    "grws_gemm_tn_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64,
                                                       ctypes.c_int64]),
    "grws_gemm_tn": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int32,
                                    ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp,
                                    ctypes.c_int64, ctypes.c_int32, _vp, ctypes.c_size_t, _vp]),
    "grws_repack_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "grws_repack_prepare": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp, ctypes.c_int64,
                                           _vp, _vp, ctypes.POINTER(ctypes.c_int64), _vp,
                                           ctypes.c_size_t, _vp]),
    "grws_repack_externals": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, _vp, ctypes.c_size_t, _vp]),
    "grws_repack_finish": (ctypes.c_int, [ctypes.POINTER(BcsrView), ctypes.c_int64, _vp, ctypes.c_int64,
                                          _vp, ctypes.c_int64, _vp, ctypes.c_int64, _vp, _vp, _vp, _vp,
                                          _vp, _vp, _vp, ctypes.POINTER(ctypes.c_int32), _vp,
                                          ctypes.c_size_t, _vp]),
    "grws_act_norm_dropout_fwd": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                                 ctypes.c_int64, ctypes.c_int32, _vp, _vp, ctypes.c_float,
                                                 ctypes.c_float, ctypes.c_uint64, _vp, _vp, ctypes.c_int32,
                                                 ctypes.c_int64, _vp, _vp, _vp]),
    "grws_act_norm_dropout_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "grws_act_norm_dropout_bwd": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int64, _vp, ctypes.c_int32,
                                                 ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                                 _vp, _vp, _vp, ctypes.c_float, ctypes.c_uint64, _vp, _vp,
                                                 ctypes.c_int64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "grws_cross_entropy_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "grws_cross_entropy_fwd": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int64, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp, _vp,
                                              ctypes.c_size_t, _vp]),
    "grws_cross_entropy_bwd": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int64, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp, _vp,
                                              ctypes.c_int32, ctypes.c_int64, _vp]),
    "grws_relabel_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "grws_relabel": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int64,
                                    _vp, _vp, ctypes.c_int64, _vp, ctypes.c_size_t, _c_i64p,
                                    _vp]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Loads libgrws.so and declares every prototype; raises if missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libgrws.so not found at {LIB_PATH}; build it with "
                "`python -m graph_rws_amd.csrc.build` (there is no fallback path)")
        L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_PROTOS)


class GrwsError(RuntimeError):
    """A libgrws call returned a non-zero status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed ({status}): {msg}")
        self.status = status


def check(fn: str, status: int) -> None:
    if status != GRWS_OK:
        msg = load().grws_last_error()
        raise GrwsError(fn, int(status), msg.decode() if msg else "")


def call(fn: str, *args):
    st = getattr(load(), fn)(*args)
    check(fn, st)
    return st


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return GRWS_F32
    if dt == torch.float16:
        return GRWS_F16
    if dt == torch.bfloat16:
        return GRWS_BF16
    raise TypeError(f"unsupported dtype {dt} (float32, float16, bfloat16)")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def require_device(who: str, dev: torch.device, *tensors) -> None:
    """Raises unless `dev` is a GPU and every tensor given (None skipped)
    lives on it: the library reads them through raw device pointers, and a
    host or other-device pointer would reach a kernel."""
    if dev.type != "cuda":
        raise RuntimeError(f"{who}: tensors must be CUDA tensors (got {dev})")
    for t in tensors:
        if t is not None and t.device != dev:
            raise RuntimeError(f"{who}: every tensor must be on {dev} (got one on {t.device})")


def stream_of(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
