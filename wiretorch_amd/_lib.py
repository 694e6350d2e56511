"""ctypes binding of ``libwiretorch_amd.so`` (declarations: ``include/wiretorch_amd.h``).

The library is built in-tree by ``python -m wiretorch_amd.build``. There is no
fallback: calling into the engine without the library raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libwiretorch_amd.so"

P = ctypes.c_void_p
I64 = ctypes.c_int64
#: Size of wt_cond_run_noalloc's device workspace (WT_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


class Tables(ctypes.Structure):
    _fields_ = [
        ("theta", P), ("U_reset", P), ("E_L", P), ("C_m", P), ("beta", P), ("n_ref", P),
        ("E_syn", P), ("g_clip", P), ("decay", P), ("jump", P), ("made", P), ("scale", P),
        ("dt", P), ("surr", P), ("types", P), ("type_of", P), ("n_types", I64),
        ("range_rows", P), ("mg_a", P), ("mg_lc", P), ("adapt", P), ("adapt_decay", P),
        ("E_adapt", P), ("N", I64), ("S", I64), ("K", I64),
        ("K_rec", I64),
    ]  # fmt: skip


class Side(ctypes.Structure):
    _fields_ = [
        ("indptr", P), ("split", P), ("targets", P), ("weights", P), ("pathway", P),
        ("n_src", I64),
    ]  # fmt: skip


class Geometry(ctypes.Structure):
    _fields_ = [("groups", I64), ("R", I64), ("range_n", I64), ("frac_bits", I64),
                ("max_list", I64), ("bound", P)]


class RunIO(ctypes.Structure):
    _fields_ = [
        ("x", P), ("B", I64), ("T", I64), ("n_in", I64), ("v", P), ("g", P), ("counter", P),
        ("spikes", P), ("prob", P), ("v_saved", P), ("G_saved", P), ("held", P),
        ("A_saved", P), ("track_v", P), ("track_I", P), ("track_g", P), ("track_b", I64),
        ("in_prob", P), ("in_seed", ctypes.c_uint64), ("in_t0", I64), ("adaptation", P),
        ("a_saved", P), ("track_a", P),
    ]  # fmt: skip


class BackwardIO(ctypes.Structure):
    _fields_ = [
        ("grad_spikes", P), ("grad_prob", P), ("spikes", P), ("v_saved", P),
        ("G_saved", P), ("held", P), ("A", P), ("g_init", P), ("B", I64), ("T", I64),
        ("grad_A", P), ("grad_scale", P), ("grad_theta", P), ("grad_reset", P),
        ("grad_E_L", P), ("grad_C_m", P), ("grad_beta", P), ("grad_E_syn", P),
        ("grad_decay", P), ("grad_jump", P), ("a_saved", P), ("grad_adapt", P),
        ("grad_adapt_decay", P), ("grad_E_adapt", P), ("grad_A_rows", P), ("T_pad", I64),
    ]  # fmt: skip


class RateTables(ctypes.Structure):
    _fields_ = [
        ("theta", P), ("gain", P), ("beta", P), ("nonlinearity", P), ("sign", P),
        ("decay", P), ("jump", P), ("made", P), ("N", I64), ("S", I64), ("K", I64),
        ("K_rec", I64),
    ]  # fmt: skip


class RateOperand(ctypes.Structure):
    _fields_ = [
        ("W", P), ("Wt", P), ("rin", P), ("rpos", P), ("src_of", P),
        ("seg", (ctypes.c_int32 * 4) * 16), ("n_seg", I64), ("B_pad", I64), ("N_pad", I64),
        ("K_rec_pad", I64), ("dtype", I64),
    ]  # fmt: skip


class RateIO(ctypes.Structure):
    _fields_ = [
        ("B", I64), ("T", I64), ("v", P), ("I", P), ("out", P), ("track_v", P),
        ("track_I", P), ("track_b", I64), ("v_saved", P), ("I_saved", P),
        ("target_saved", P), ("A_saved", P), ("A_ff", P), ("split", P),
    ]  # fmt: skip


class RateBackIO(ctypes.Structure):
    _fields_ = [
        ("B", I64), ("T", I64), ("grad_out", P), ("v_saved", P), ("I_saved", P),
        ("target_saved", P), ("A_saved", P), ("I_final", P), ("lam_v", P), ("lam_I", P),
        ("d_rate", P), ("gA_op", P), ("grad_A", P), ("acc_theta", P), ("acc_gain", P),
        ("acc_beta", P), ("acc_decay", P), ("acc_scale", P),
    ]  # fmt: skip


#: Every entry point the header declares, with its ctypes signature.
SIGNATURES = {
    "wt_split_ranges": (ctypes.c_int, [P, P, I64, I64, I64, P, P]),
    "wt_cond_run_scratch_bytes": (I64, [ctypes.POINTER(Geometry), I64, I64]),
    "wt_cond_run_scratch_zeroed": (I64, [ctypes.POINTER(Geometry)]),
    "wt_cond_run": (ctypes.c_int, [ctypes.POINTER(Tables), ctypes.POINTER(Side),
                                   ctypes.POINTER(Side), ctypes.POINTER(Geometry),
                                   ctypes.POINTER(RunIO), P, P]),
    "wt_cond_run_noalloc": (ctypes.c_int, [ctypes.POINTER(Tables), ctypes.POINTER(Side),
                                           ctypes.POINTER(Side), ctypes.POINTER(Geometry),
                                           ctypes.POINTER(RunIO), P, P]),
    "wt_cond_run_timed": (ctypes.c_int, [ctypes.POINTER(Tables), ctypes.POINTER(Side),
                                         ctypes.POINTER(Side), ctypes.POINTER(Geometry),
                                         ctypes.POINTER(RunIO), P, P, P]),
    "wt_cond_scan_backward": (ctypes.c_int, [ctypes.POINTER(Tables),
                                             ctypes.POINTER(BackwardIO), P]),
    "wt_cond_recurrent_backward_scratch_bytes": (I64, [I64, I64, I64, I64]),
    "wt_cond_recurrent_backward": (ctypes.c_int, [ctypes.POINTER(Tables), ctypes.POINTER(Side),
                                                  ctypes.POINTER(BackwardIO), P, P]),
    "wt_rate_split_bytes": (I64, [ctypes.POINTER(RateTables), ctypes.POINTER(RateOperand),
                                  I64]),
    "wt_rate_forward": (ctypes.c_int, [ctypes.POINTER(RateTables), ctypes.POINTER(RateOperand),
                                       ctypes.POINTER(RateIO), P]),
    "wt_rate_backward": (ctypes.c_int, [ctypes.POINTER(RateTables),
                                        ctypes.POINTER(RateOperand),
                                        ctypes.POINTER(RateBackIO), P]),
    "wt_edge_sources": (ctypes.c_int, [P, I64, P, P]),
    "wt_poisson_fill": (ctypes.c_int, [P, I64, ctypes.c_uint64, I64, I64, I64, P, P]),
    "wt_gemm_tn_split": (ctypes.c_int, [P, I64, P, I64, P, I64, I64, I64, I64, ctypes.c_int32,
                                        P]),
    "wt_split_bf16": (ctypes.c_int, [P, I64, P, P, P]),
    "wt_events_scratch_bytes": (I64, [I64, I64]),
    "wt_events_count": (ctypes.c_int, [P, I64, I64, P, P, P]),
    "wt_events_fill": (ctypes.c_int, [P, I64, I64, P, P, P, P, I64, I64, P]),
    "wt_gate_scan": (ctypes.c_int, [P, I64, I64, I64, P, I64, P, P, I64, I64, I64, P, P]),
    "wt_weight_gradient": (ctypes.c_int, [ctypes.POINTER(Side), P, I64, P, P, P, P, I64,
                                          I64, I64, I64, P, P]),
    "wt_weight_gradient_by_target": (ctypes.c_int, [P, I64, P, P, I64, I64, P, P, P, P, I64,
                                                    P, P, P]),
    "wt_filter_forward": (ctypes.c_int, [P, P, P, P, P, ctypes.c_float, ctypes.c_float, I64,
                                         I64, I64, P]),
    "wt_filter_backward": (ctypes.c_int, [P, P, ctypes.c_float, ctypes.c_float, I64, I64, I64,
                                          P]),
    "wt_device_info": (ctypes.c_int, [ctypes.POINTER(I64), ctypes.POINTER(I64)]),
}  # fmt: skip

_lib = None


def load(path: Path = LIBRARY) -> ctypes.CDLL:
    """The library, loaded once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build the HIP extension with "
                "`python -m wiretorch_amd.build` (there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with HIP error {status}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()
