"""ctypes binding of libamass_hip.so (the C-ABI declared in include/amass_hip.h).

The structs below mirror the header field for field; a CPU test parses the header and
checks names, order, types and ``sizeof`` against ``amass_abi_struct_size``.  All kernels
launch on the caller's current torch stream.  There is no fallback: if the library is
missing or a call returns a non-zero status, an :class:`AmassError` is raised.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_F32 = C.c_float
_F64 = C.c_double

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libamass_hip.so")
ABI_VERSION = 11    # AMASS_ABI_VERSION of include/amass_hip.h these mirrors follow


class AmassError(RuntimeError):
    """A libamass_hip entry point returned a non-zero status."""


def _fields(spec: str):
    """'q:p q_st:i64 ...' -> ctypes _fields_."""
    kinds = {"p": _P, "i64": _I64, "i32": _I32, "f32": _F32, "f64": _F64}
    out = []
    for tok in spec.split():
        name, k = tok.split(":")
        out.append((name, kinds[k]))
    return out


class QuadScoreArgs(C.Structure):
    _fields_ = _fields(
        "q:p q_st:i64 q_hs:i64 rec:p rec_sb:i64 block_table:p bt_st:i64 n_sel_hi:p "
        "score:p sc_sr:i64 sc_sh:i64 score_h:p sh_sr:i64 sh_sh:i64 sh_sg:i64 "
        "tile_max:p tm_sr:i64 tm_sh:i64 tm_sg:i64 comb_out:p "
        "scale:f32 n_req:i32 n_kv:i32 G:i32 d:i32 page:i32 rank:i32 v_bits:i32 "
        "max_pages:i32 combine:i32")


class R8ScoreArgs(C.Structure):
    _fields_ = _fields(
        "q:p q_st:i64 q_hs:i64 rec:p rec_sb:i64 block_table:p bt_st:i64 seq_lens:p "
        "n_sel_hi:p score:p sc_sr:i64 sc_sh:i64 comb_out:p scale:f32 n_req:i32 n_kv:i32 "
        "G:i32 d:i32 page:i32 rank:i32 vk_bits:i32 c_bits:i32 max_pages:i32 c_fp32:i32")


class ClseScoreArgs(C.Structure):
    _fields_ = _fields(
        "q:p q_st:i64 q_hs:i64 rec:p rec_sb:i64 block_table:p bt_st:i64 seq_lens:p "
        "n_sel_hi:p score:p sc_sr:i64 sc_sh:i64 score_h:p sh_sr:i64 sh_sh:i64 sh_sg:i64 "
        "tile_max:p tm_sr:i64 tm_sh:i64 tm_sg:i64 comb_out:p scale:f32 n_req:i32 n_kv:i32 "
        "G:i32 d:i32 page:i32 rank:i32 v_bits:i32 "
        "c_bits:i32 max_pages:i32 combine:i32")


class DeriveArgs(C.Structure):
    _fields_ = _fields(
        "seq_lens:p n_pages:p n_sel_hi:p b_fix:p budget:f64 n_req:i32 page:i32 "
        "window_pages:i32 sink_pages:i32")


class NrmArgs(C.Structure):
    _fields_ = _fields(
        "score_h:p sh_sr:i64 sh_sh:i64 sh_sg:i64 score:p sc_sr:i64 sc_sh:i64 n_sel_hi:p "
        "n_req:i32 n_kv:i32 G:i32 max_pages:i32")


class SelectArgs(C.Structure):
    _fields_ = _fields(
        "score:p sc_sr:i64 sc_sh:i64 score_h:p sh_sr:i64 sh_sh:i64 sh_sg:i64 "
        "tile_max:p tm_sr:i64 tm_sh:i64 tm_sg:i64 n_pages:p n_sel_hi:p b_fix:p "
        "page_table:p pt_sr:i64 pt_sh:i64 page_cnt:p pc_sr:i64 "
        "n_sel_out:p coverage:f64 n_req:i32 n_kv:i32 G:i32 max_pages:i32 sink_pages:i32 "
        "mode:i32 tie_mode:i32 score_kind:i32")


class DecodeArgs(C.Structure):
    _fields_ = _fields(
        "q:p q_st:i64 q_hs:i64 k:p k_sb:i64 k_st:i64 k_sh:i64 v:p v_sb:i64 v_st:i64 "
        "v_sh:i64 block_table:p bt_st:i64 seq_lens:p page_table:p pt_sr:i64 pt_sh:i64 "
        "page_cnt:p pc_sr:i64 m_part:p l_part:p acc_part:p out:p o_st:i64 o_hs:i64 hot:p "
        "page2slot:p vbo:p pool:p t_layer:i32 t_nb:i32 t_slots:i32 scale:f32 n_req:i32 "
        "n_kv:i32 G:i32 d:i32 page:i32 split:i32 pps_min:i32 path:i32 dense:i32 v_src:i32")


class TierPlanArgs(C.Structure):
    _fields_ = _fields(
        "page_table:p pt_sr:i64 pt_sh:i64 page_cnt:p pc_sr:i64 block_table:p bt_st:i64 "
        "seq_lens:p page2slot:p slot2page:p lru_clock:p clock:p miss_pages:p miss_cnt:p "
        "victim_slots:p overflow:p fetch_list:p fetch_cnt:p first_pos:p n_req:i32 n_kv:i32 "
        "nb:i32 slots:i32 max_pages:i32 page:i32 fcap:i32")


class TierFetchArgs(C.Structure):
    _fields_ = _fields(
        "fetch_list:p fetch_cnt:p hot:p pool:p vpool:p v_sb:i64 v_st:i64 v_sh:i64 vbo:p "
        "pool_valid:p t_layer:i32 nb:i32 n_kv:i32 slots:i32 page:i32 d:i32 fcap:i32 grid:i32")


class BuildArgs(C.Structure):
    _fields_ = _fields(
        "k:p k_sb:i64 k_st:i64 k_sh:i64 k_layers:p blocks:p rec:p rec_sb:i64 rec_lsb:i64 "
        "tag:p tag_sb:i64 tag_sh:i64 tag_lsb:i64 n:i32 n_layers:i32 n_kv:i32 d:i32 page:i32 "
        "kind:i32 rank:i32 v_bits:i32 c_bits:i32 v_grain:i32 c_grain:i32 tagw:i32")


class CopyRun(C.Structure):
    _fields_ = _fields("dst:p src:p dpitch:i64 spitch:i64 width:i64 height:i64")


class InvalidateArgs(C.Structure):
    _fields_ = _fields(
        "block_table:p bt_st:i64 seq_lens:p query_start_loc:p page2slot:p slot2page:p "
        "pool_valid:p n_req:i32 n_layers:i32 nb:i32 n_kv:i32 slots:i32 page:i32 "
        "max_pages:i32")


class StageArgs(C.Structure):
    _fields_ = _fields(
        "block_table:p bt_st:i64 seq_lens:p query_start_loc:p vbo:p v_flushed:p "
        "free_stack:p free_top:p v_slot:p flush_list:p flush_cnt:p overflow:p mark:p first:p "
        "v_pool:p vp_sl:i64 vp_sb:i64 vp_st:i64 vp_sh:i64 pool:p pool_valid:p "
        "n_req:i32 n_tokens:i32 max_pages:i32 n_layers:i32 nb:i32 nv:i32 n_kv:i32 page:i32 "
        "d:i32 maxf:i32")


class ScatterArgs(C.Structure):
    _fields_ = _fields(
        "value:p v_st:i64 v_sh:i64 v_slot:p v_pool:p vp_sb:i64 vp_st:i64 vp_sh:i64 "
        "n_tokens:i32 n_kv:i32 d:i32 page:i32 nv:i32")


STRUCTS = {
    "amass_quad_score_args": (0, QuadScoreArgs),
    "amass_r8_score_args": (1, R8ScoreArgs),
    "amass_derive_args": (2, DeriveArgs),
    "amass_nrm_args": (3, NrmArgs),
    "amass_select_args": (4, SelectArgs),
    "amass_decode_args": (5, DecodeArgs),
    "amass_tier_plan_args": (6, TierPlanArgs),
    "amass_tier_fetch_args": (7, TierFetchArgs),
    "amass_copy_run": (8, CopyRun),
    "amass_build_args": (9, BuildArgs),
    "amass_clse_score_args": (10, ClseScoreArgs),
    "amass_invalidate_args": (11, InvalidateArgs),
    "amass_stage_args": (12, StageArgs),
    "amass_scatter_args": (13, ScatterArgs),
}

# entry point -> argument struct (None = custom signature)
ENTRY_POINTS = {
    "amass_quad_score": QuadScoreArgs,
    "amass_r8_score": R8ScoreArgs,
    "amass_derive_params": DeriveArgs,
    "amass_nrm_combine": NrmArgs,
    "amass_topb_select": SelectArgs,
    "amass_coverage_select": SelectArgs,
    "amass_sparse_decode": DecodeArgs,
    "amass_sparse_decode_noalloc": DecodeArgs,
    "amass_dense_paged_decode": DecodeArgs,
    "amass_tier_decode": DecodeArgs,
    "amass_tier_gather_plan": TierPlanArgs,
    "amass_tier_fetch": TierFetchArgs,
    "amass_summary_build": BuildArgs,
    "amass_clse_score": ClseScoreArgs,
    "amass_tier_invalidate": InvalidateArgs,
    "amass_stage_begin_step": StageArgs,
    "amass_stage_scatter": ScatterArgs,
}

_LIB: Optional[C.CDLL] = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load libamass_hip.so (host-only introspection works without a GPU)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise AmassError(
            f"{path} is missing: build it with `python amass-kv_amd/build_hip.py` "
            "(there is no CPU fallback for the AMASS hot path)")
    try:
        import torch  # noqa: F401  (bind to torch's already-loaded HIP runtime)
    except Exception:  # noqa: BLE001
        pass
    lib = C.CDLL(path)
    for name, st in ENTRY_POINTS.items():
        fn = getattr(lib, name)
        fn.argtypes = [C.POINTER(st), _P]
        fn.restype = C.c_int
    lib.amass_tier_dma.argtypes = [C.POINTER(CopyRun), C.c_int32, _P]
    lib.amass_tier_dma.restype = C.c_int
    lib.amass_quad_select_attend.argtypes = [C.POINTER(QuadScoreArgs), C.POINTER(SelectArgs),
                                             C.POINTER(DecodeArgs), C.c_int, _P, C.c_int, _P]
    lib.amass_quad_select_attend.restype = C.c_int
    lib.amass_host_pool_alloc.argtypes = [C.c_size_t, C.POINTER(_P), C.POINTER(_P)]
    lib.amass_host_pool_alloc.restype = C.c_int
    lib.amass_host_pool_free.argtypes = [_P]
    lib.amass_host_pool_free.restype = C.c_int
    lib.amass_abi_version.restype = C.c_int
    lib.amass_abi_struct_size.argtypes = [C.c_int]
    lib.amass_abi_struct_size.restype = C.c_size_t
    lib.amass_status_string.argtypes = [C.c_int]
    lib.amass_status_string.restype = C.c_char_p
    lib.amass_last_hip_error.restype = C.c_int
    if lib.amass_abi_version() != ABI_VERSION:
        raise AmassError(f"{path} has ABI version {lib.amass_abi_version()}, these bindings "
                         f"expect {ABI_VERSION}: rebuild it")
    _LIB = lib
    return lib


def status_string(rc: int) -> str:
    return load_library().amass_status_string(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        lib = load_library()
        raise AmassError(f"{what} failed: {status_string(rc)} (status {rc}, "
                         f"hipError {lib.amass_last_hip_error()})")


def call(name: str, args, stream: int) -> None:
    """Invoke entry point `name` with struct `args` on `stream` (a hipStream_t int)."""
    lib = load_library()
    check(getattr(lib, name)(C.byref(args), _P(stream)), name)


def call_select_attend(score, select, decode, mode: int, tickets, wgs_per_unit: int,
                       stream: int) -> None:
    """amass_quad_select_attend (decode None: score + select only; tickets: the device
    address of the zeroed per-unit int32 tickets, or None with wgs_per_unit 1)."""
    lib = load_library()
    check(lib.amass_quad_select_attend(C.byref(score), C.byref(select),
                                       C.byref(decode) if decode is not None else None,
                                       mode, _P(tickets) if tickets else None, wgs_per_unit,
                                       _P(stream)), "amass_quad_select_attend")


def ptr(t) -> Optional[int]:
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def current_stream(device=None) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors) -> None:
    """The hot path runs only on the GPU; CPU tensors are rejected (no CPU fallback)."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise AmassError("AMASS HIP kernels need device tensors; got a CPU tensor "
                             "(there is no CPU fallback on the product path)")
