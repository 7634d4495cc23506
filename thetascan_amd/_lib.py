"""ctypes binding of ``libthetascan_hip.so`` (C ABI in ``include/thetascan_hip.h``).

The library is loaded after torch so that it binds to the HIP runtime torch
already mapped (both carry the ``libamdhip64.so.7`` soname).  Nothing here
falls back to a CPU path: a missing library or a non-GPU tensor raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

import torch

from ._build import LIB_PATH

TS_OK = 0
TS_ERR_VALUE = 1
TS_ERR_NOT_IMPLEMENTED = 2
TS_ERR_RUNTIME = 3

TS_BF16 = 0
TS_F32 = 1

RET_NONE = 0
RET_STATIC = 1
RET_STREAM = 2

EXT_NONE = 0
EXT_ONES = 1
EXT_ARRAY = 2

GN_RELU2 = 0
GN_TANH = 1
GN_SILU = 2
GN_SWIGLU = 3

OUT_STORE = 0
OUT_STORE_F32 = 1
OUT_ACCUM_F32 = 2


class Strided(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("sb", ctypes.c_int64),
        ("sh", ctypes.c_int64),
        ("st", ctypes.c_int64),
    ]


class ScanDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("dk", ctypes.c_int32),
        ("dv", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("retention", ctypes.c_int32),
        ("reverse", ctypes.c_int32),
        ("q_ext", ctypes.c_int32),
        ("k_ext", ctypes.c_int32),
        ("v_ext", ctypes.c_int32),
        ("out_mode", ctypes.c_int32),
        ("out_scale", ctypes.c_float),
        ("seg_chunks", ctypes.c_int32),
        ("want_final", ctypes.c_int32),
        ("value_split", ctypes.c_int32),
        ("states_in", ctypes.c_int32),
        ("init_state", ctypes.c_int32),
    ]


class ScanPairIO(ctypes.Structure):
    _fields_ = [(n, Strided) for n in ("qa", "k", "v", "qb", "out_a", "out_b", "k_ext")] + [
        ("log_alpha", ctypes.c_void_p)]


MAX_VIEWS = 3


class ScanViewsDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("dk", ctypes.c_int32),
        ("dv", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("n_views", ctypes.c_int32),
        ("mass", ctypes.c_int32),
        ("seg_chunks", ctypes.c_int32),
    ]


class ScanViewsIO(ctypes.Structure):
    _fields_ = [
        ("q", Strided),
        ("k", Strided),
        ("v", Strided),
        ("log_alpha", ctypes.c_void_p * MAX_VIEWS),
        ("out", Strided * MAX_VIEWS),
        ("out_ext", Strided * MAX_VIEWS),
    ]


class ScanIO(ctypes.Structure):
    _fields_ = [
        ("q", Strided),
        ("k", Strided),
        ("v", Strided),
        ("q_ext", Strided),
        ("k_ext", Strided),
        ("v_ext", Strided),
        ("log_alpha", ctypes.c_void_p),
        ("decay", Strided),
        ("out", Strided),
        ("out_ext", Strided),
        ("final_state", ctypes.c_void_p),
        ("init_state", ctypes.c_void_p),
    ]


class FeatureDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("m", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("kind", ctypes.c_int32),
        ("in_rot", ctypes.c_int32),
        ("feat_rot", ctypes.c_int32),
        ("has_tau", ctypes.c_int32),
        ("gain", ctypes.c_float),
        ("resid_scale", ctypes.c_float),
        ("eps", ctypes.c_float),
    ]


class FeatureIO(ctypes.Structure):
    _fields_ = [
        ("x", Strided),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("in_cos", ctypes.c_void_p),
        ("in_sin", ctypes.c_void_p),
        ("f_cos", ctypes.c_void_p),
        ("f_sin", ctypes.c_void_p),
        ("phi", Strided),
        ("resid", Strided),
    ]


class FeatureBwdIO(ctypes.Structure):
    _fields_ = [
        ("x", Strided),
        ("w1", ctypes.c_void_p),
        ("w1t", ctypes.c_void_p),
        ("w2t", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("in_cos", ctypes.c_void_p),
        ("in_sin", ctypes.c_void_p),
        ("f_cos", ctypes.c_void_p),
        ("f_sin", ctypes.c_void_p),
        ("dphi", Strided),
        ("dresid", Strided),
        ("dx", Strided),
        ("da", Strided),
        ("xn", Strided),
        ("h", Strided),
        ("dtau", Strided),
        ("dw1_part", ctypes.c_void_p),
        ("dw2_part", ctypes.c_void_p),
        ("dtau_part", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
    ]


class ReadDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("normalize", ctypes.c_int32),
        ("gate", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("eps", ctypes.c_float),
    ]


class ReadIO(ctypes.Structure):
    _fields_ = [("num", Strided), ("mass", Strided), ("resid", Strided), ("g", Strided), ("y", Strided),
                ("g_bias", ctypes.c_void_p)]


class QkNormDesc(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32), ("d", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("rot", ctypes.c_int32), ("eps", ctypes.c_float)]


class ContractDesc(ctypes.Structure):
    _fields_ = [("G", ctypes.c_int32), ("N", ctypes.c_int32), ("p", ctypes.c_int32), ("q", ctypes.c_int32),
                ("dtype", ctypes.c_int32)]


class ReadBwdIO(ctypes.Structure):
    _fields_ = [
        ("num", Strided),
        ("mass", Strided),
        ("resid", Strided),
        ("g", Strided),
        ("dy", Strided),
        ("dnum", Strided),
        ("dmass", Strided),
        ("dresid", Strided),
        ("dg", Strided),
        ("g_bias", ctypes.c_void_p),
        ("dg_bias_part", ctypes.c_void_p),
    ]


class KmapDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "m", "dtype", "kind", "rms", "gain_mode", "sparsity")] + \
        [("gain", ctypes.c_float), ("temperature", ctypes.c_float), ("eps", ctypes.c_float)]


class KmapParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("shift", "gain", "rho", "alpha")]


class KmapGrads(ctypes.Structure):
    _fields_ = [("da", Strided)] + [(n, ctypes.c_void_p) for n in ("dshift_part", "dgain_part", "drho_part",
                                                                    "dalpha_part")]


class AnchorDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "d", "V", "c_heads", "dtype")] + \
        [("gain", ctypes.c_float), ("eps", ctypes.c_float)]


class ReadOutDesc(ctypes.Structure):
    _fields_ = [("read", ReadDesc), ("n", ctypes.c_int32)]


class ReadOutIO(ctypes.Structure):
    _fields_ = [("num", Strided), ("mass", Strided), ("resid", Strided), ("g", Strided),
                ("g_bias", ctypes.c_void_p), ("w", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("out_ld", ctypes.c_int64), ("y", ctypes.c_void_p), ("y_ld", ctypes.c_int64)]


class ReadOutBwdIO(ctypes.Structure):
    _fields_ = [("num", Strided), ("mass", Strided), ("resid", Strided), ("g", Strided),
                ("g_bias", ctypes.c_void_p), ("w_t", ctypes.c_void_p), ("dout", ctypes.c_void_p),
                ("dout_ld", ctypes.c_int64), ("dnum", Strided), ("dmass", Strided), ("dresid", Strided),
                ("dg", Strided), ("dg_bias_part", ctypes.c_void_p)]


class WcumsumDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("F", ctypes.c_int32),
        ("retention", ctypes.c_int32),
        ("reverse", ctypes.c_int32),
    ]


class BsplineDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("P", ctypes.c_int32),
        ("n_basis", ctypes.c_int32),
        ("degree", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("bound", ctypes.c_float),
        ("scale", ctypes.c_float),
    ]


class AbsMassDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "F", "dtype", "retention")]


class RowNormDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "W", "dtype", "rope")] + [("eps", ctypes.c_float)]


class StackDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "d", "n", "dtype")]


class RowsDesc(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int64), ("W", ctypes.c_int32), ("dtype", ctypes.c_int32)]


class GnActDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "m", "dtype", "act", "has_tau")] + [
        ("eps", ctypes.c_float)]


class GnDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("m", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("has_tau", ctypes.c_int32),
        ("s", ctypes.c_float),
        ("inv_depth", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("act", ctypes.c_int32),
        ("damping", ctypes.c_float),
    ]


class GnIO(ctypes.Structure):
    _fields_ = [
        ("x", Strided),
        ("v", Strided),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("w2t", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("h", Strided),
        ("lam", Strided),
        ("g", Strided),
    ]


class GnBwdIO(ctypes.Structure):
    _fields_ = [
        ("x", Strided),
        ("v", Strided),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("w1t", ctypes.c_void_p),
        ("w2t", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("dh", Strided),
        ("dlam", Strided),
        ("dg", Strided),
        ("dx_in", Strided),
        ("dx", Strided),
        ("dv", Strided),
        ("tiles_m", ctypes.c_void_p),
        ("tiles_d", ctypes.c_void_p),
    ]


class GnReadDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("m", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("has_tau", ctypes.c_int32),
        ("corr", ctypes.c_int32),
        ("want_resid", ctypes.c_int32),
        ("s", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("act", ctypes.c_int32),
    ]


class GnReadIO(ctypes.Structure):
    _fields_ = [
        ("q", Strided),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("num", Strided),
        ("mass", Strided),
        ("h", Strided),
        ("resid", Strided),
    ]


class GnReadBwdIO(ctypes.Structure):
    _fields_ = [
        ("q", Strided),
        ("w1", ctypes.c_void_p),
        ("w1t", ctypes.c_void_p),
        ("w2t", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("num", Strided),
        ("mass", Strided),
        ("dh", Strided),
        ("dresid", Strided),
        ("dq", Strided),
        ("dnum", Strided),
        ("dmass", ctypes.c_void_p),
        ("tiles_m", ctypes.c_void_p),
        ("tiles_d", ctypes.c_void_p),
    ]


class BlendDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("n_in", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class MemoryDesc(ctypes.Structure):
    _fields_ = [
        ("feat", FeatureDesc),
        ("normalize", ctypes.c_int32),
        ("gate", ctypes.c_int32),
        ("has_g_bias", ctypes.c_int32),
        ("seg_chunks", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
    ]


class MemoryIO(ctypes.Structure):
    _fields_ = [
        ("q", Strided),
        ("k", Strided),
        ("v", Strided),
        ("g", Strided),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("g_bias", ctypes.c_void_p),
        ("in_cos", ctypes.c_void_p),
        ("in_sin", ctypes.c_void_p),
        ("f_cos", ctypes.c_void_p),
        ("f_sin", ctypes.c_void_p),
    ]


class MemoryGrads(ctypes.Structure):
    _fields_ = [
        ("dy", Strided),
        ("dq", Strided),
        ("dk", Strided),
        ("dv", Strided),
        ("dg", Strided),
        ("dw1", ctypes.c_void_p),
        ("dw2", ctypes.c_void_p),
        ("dtau", ctypes.c_void_p),
        ("dg_bias", ctypes.c_void_p),
    ]


class RetentionDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("B", "H", "T", "dk", "dv", "dtype", "has_mass", "seg_tiles")]


class RetentionIO(ctypes.Structure):
    _fields_ = [(n, Strided) for n in ("q", "k", "v", "dout", "dmass")] + [("log_alpha", ctypes.c_void_p)]


FEAT_RELU2 = 0
FEAT_SOFTMAX = 1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None



def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m thetascan_amd._build` "
                "(or __graft_entry__.build()); the hip backend has no fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        lib.ts_abi_version.restype = ctypes.c_int
        lib.ts_last_error.restype = ctypes.c_char_p
        lib.ts_scan_layout.argtypes = [
            ctypes.POINTER(ScanDesc),
            ctypes.POINTER(ctypes.c_int32),
            ctypes.POINTER(ctypes.c_int32),
            ctypes.POINTER(ctypes.c_int32),
        ]
        lib.ts_scan_workspace_bytes.argtypes = [ctypes.POINTER(ScanDesc), ctypes.POINTER(ctypes.c_size_t)]
        lib.ts_scan_fwd.argtypes = [
            ctypes.POINTER(ScanDesc),
            ctypes.POINTER(ScanIO),
            ctypes.c_void_p,
            ctypes.c_size_t,
            ctypes.c_void_p,
        ]
        P = ctypes.POINTER
        lib.ts_scan_pair_fwd.argtypes = [P(ScanDesc), P(ScanPairIO), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_scan_fwd_noalloc.argtypes = [P(ScanDesc), P(ScanIO), ctypes.c_void_p]
        lib.ts_scan_views_workspace_bytes.argtypes = [P(ScanViewsDesc), P(ctypes.c_size_t)]
        lib.ts_scan_views_fwd.argtypes = [P(ScanViewsDesc), P(ScanViewsIO), ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p]
        lib.ts_feature_fwd.argtypes = [P(FeatureDesc), P(FeatureIO), ctypes.c_void_p]
        lib.ts_feature_fwd_summary.argtypes = [P(FeatureDesc), P(FeatureIO), Strided, P(ScanDesc), ctypes.c_void_p,
                                               ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_feature_bwd.argtypes = [P(FeatureDesc), P(FeatureBwdIO), ctypes.c_void_p]
        lib.ts_feature_bwd_parts.argtypes = [P(FeatureDesc), ctypes.c_int32, P(ctypes.c_int32)]
        lib.ts_feature_bwd_transposed.argtypes = [P(FeatureDesc), ctypes.c_int32, ctypes.c_int32, P(ctypes.c_int32)]
        lib.ts_read_fwd.argtypes = [P(ReadDesc), P(ReadIO), ctypes.c_void_p]
        lib.ts_read_bwd.argtypes = [P(ReadDesc), P(ReadBwdIO), ctypes.c_void_p]
        lib.ts_read_bwd_parts.argtypes = [P(ReadDesc), P(ctypes.c_int32)]
        lib.ts_kmap_parts.argtypes = [P(KmapDesc), P(KmapParams), P(ctypes.c_int32)]
        lib.ts_kmap_fwd.argtypes = [P(KmapDesc), P(KmapParams), Strided, Strided, ctypes.c_void_p]
        lib.ts_kmap_bwd.argtypes = [P(KmapDesc), P(KmapParams), Strided, Strided, P(KmapGrads), ctypes.c_void_p]
        lib.ts_anchor_width.argtypes = [P(AnchorDesc), P(ctypes.c_int32)]
        lib.ts_anchor_fwd.argtypes = [P(AnchorDesc), Strided, ctypes.c_void_p, Strided, ctypes.c_void_p]
        lib.ts_anchor_bwd.argtypes = [P(AnchorDesc), Strided, ctypes.c_void_p, Strided, Strided, ctypes.c_void_p,
                                      ctypes.c_void_p]
        lib.ts_read_out_fwd.argtypes = [P(ReadOutDesc), P(ReadOutIO), ctypes.c_void_p]
        lib.ts_read_out_bwd.argtypes = [P(ReadOutDesc), P(ReadOutBwdIO), ctypes.c_void_p]
        lib.ts_read_out_bwd_parts.argtypes = [P(ReadOutDesc), P(ctypes.c_int32)]
        lib.ts_contract_workspace_bytes.argtypes = [P(ContractDesc), P(ctypes.c_size_t)]
        lib.ts_contract_tokens.argtypes = [P(ContractDesc), ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_qknorm_fwd.argtypes = [P(QkNormDesc), Strided, Strided, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p]
        lib.ts_qknorm_bwd.argtypes = [P(QkNormDesc), Strided, Strided, Strided, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p]
        lib.ts_wcumsum_workspace_bytes.argtypes = [P(WcumsumDesc), P(ctypes.c_size_t)]
        lib.ts_wcumsum.argtypes = [P(WcumsumDesc), Strided, Strided, ctypes.c_void_p, Strided, ctypes.c_void_p,
                                   ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_col_sums.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
        lib.ts_sum_slots.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                     ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32, ctypes.c_float,
                                     ctypes.c_void_p]
        lib.ts_bspline_fwd.argtypes = [P(BsplineDesc), Strided, ctypes.c_void_p, Strided, ctypes.c_void_p]
        lib.ts_bspline_parts.argtypes = [P(BsplineDesc), P(ctypes.c_int32)]
        lib.ts_bspline_bwd.argtypes = [P(BsplineDesc), Strided, ctypes.c_void_p, Strided, Strided, ctypes.c_void_p,
                                       ctypes.c_void_p]
        lib.ts_bspline_norm_fwd.argtypes = [P(BsplineDesc), Strided, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                             Strided, ctypes.c_void_p]
        lib.ts_bspline_norm_bwd.argtypes = [P(BsplineDesc), Strided, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                             Strided, Strided, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_blend_fwd.argtypes = [P(BlendDesc), P(Strided), ctypes.c_void_p, Strided, ctypes.c_void_p]
        lib.ts_blend_gated_fwd.argtypes = [P(BlendDesc), P(Strided), ctypes.c_void_p, Strided, ctypes.c_void_p, Strided,
                                           ctypes.c_void_p]
        lib.ts_blend_parts.argtypes = [P(BlendDesc), P(ctypes.c_int32)]
        lib.ts_blend_bwd.argtypes = [P(BlendDesc), P(Strided), ctypes.c_void_p, Strided, P(Strided),
                                     ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_gn_write_fwd.argtypes = [P(GnDesc), P(GnIO), ctypes.c_void_p]
        lib.ts_gn_write_bwd.argtypes = [P(GnDesc), P(GnBwdIO), ctypes.c_void_p]
        lib.ts_gn_read_fwd.argtypes = [P(GnReadDesc), P(GnReadIO), ctypes.c_void_p]
        lib.ts_gn_read_bwd.argtypes = [P(GnReadDesc), P(GnReadBwdIO), ctypes.c_void_p]
        lib.ts_abs_mass_workspace_bytes.argtypes = [P(AbsMassDesc), P(ctypes.c_size_t)]
        lib.ts_abs_mass_fwd.argtypes = [P(AbsMassDesc), Strided, Strided, ctypes.c_void_p, Strided, Strided,
                                        ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_abs_mass_bwd.argtypes = [P(AbsMassDesc), Strided, Strided, Strided, ctypes.c_void_p, Strided, Strided,
                                        Strided, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_rownorm_fwd.argtypes = [P(RowNormDesc), Strided, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_rownorm_bwd.argtypes = [P(RowNormDesc), Strided, Strided, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p]
        lib.ts_gn_act_fwd.argtypes = [P(GnActDesc), Strided, Strided, ctypes.c_void_p, Strided, Strided, Strided,
                                      ctypes.c_void_p]
        lib.ts_gn_act_bwd.argtypes = [P(GnActDesc), Strided, Strided, ctypes.c_void_p] + [Strided] * 6 + [
            ctypes.c_void_p]
        lib.ts_memory_bytes.argtypes = [P(MemoryDesc), P(ctypes.c_size_t), P(ctypes.c_size_t)]
        lib.ts_memory_fwd.argtypes = [P(MemoryDesc), P(MemoryIO), Strided, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p]
        lib.ts_memory_bwd.argtypes = [P(MemoryDesc), P(MemoryIO), P(MemoryGrads), ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_retention_workspace_bytes.argtypes = [P(RetentionDesc), P(ctypes.c_size_t)]
        lib.ts_retention_grad.argtypes = [P(RetentionDesc), P(RetentionIO), ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_void_p]
        lib.ts_stack_heads.argtypes = [P(StackDesc), P(Strided), ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_scale_add_fwd.argtypes = [P(RowsDesc)] + [ctypes.c_void_p] * 6
        lib.ts_scale_add_parts.argtypes = [P(RowsDesc), P(ctypes.c_int32)]
        lib.ts_scale_add_bwd.argtypes = [P(RowsDesc)] + [ctypes.c_void_p] * 10
        lib.ts_relu2_fwd.argtypes = [P(RowsDesc)] + [ctypes.c_void_p] * 3
        lib.ts_relu2_bwd.argtypes = [P(RowsDesc)] + [ctypes.c_void_p] * 4
        lib.ts_softcap_xent_fwd.argtypes = [P(RowsDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_softcap_xent_bwd.argtypes = [P(RowsDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                            ctypes.c_void_p]
        if lib.ts_abi_version() != 17:
            raise RuntimeError("libthetascan_hip.so ABI version mismatch")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status == TS_OK:
        return
    message = (load().ts_last_error() or b"").decode(errors="replace") or what
    if status == TS_ERR_VALUE:
        raise ValueError(message)
    if status == TS_ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(message)
    raise RuntimeError(message)


def strided(t: torch.Tensor | None) -> Strided:
    """Describe a [B,H,T,(F)] tensor (or None) for the C ABI."""
    if t is None:
        return Strided(None, 0, 0, 0)
    s = t.stride()
    return Strided(t.data_ptr(), s[0], s[1], s[2])


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The caller's current HIP stream on ``device`` (kernels launch on it)."""
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


# ------------------------------------------------------------ launch timing

_RECORDS: list | None = None


@contextlib.contextmanager
def record_launches():
    """Collect ``(name, start_event, end_event, bytes)`` for every entry-point
    call made inside the block.  The events bracket the C call on the stream
    it launches on; ``bytes`` is the call's algorithmic traffic (every input
    element read once, every output element written once)."""
    global _RECORDS
    previous, _RECORDS = _RECORDS, []
    try:
        yield _RECORDS
    finally:
        _RECORDS = previous


def recording() -> bool:
    """Whether entry-point launches are being recorded."""
    return _RECORDS is not None


class _Untimed:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_UNTIMED = _Untimed()


class _Timed:
    __slots__ = ("name", "nbytes", "start", "end")

    def __init__(self, name, nbytes):
        self.name, self.nbytes = name, nbytes

    def __enter__(self):
        self.start, self.end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        self.start.record()

    def __exit__(self, *exc):
        self.end.record()
        nb = self.nbytes() if callable(self.nbytes) else self.nbytes
        _RECORDS.append((self.name, self.start, self.end, int(nb)))
        return False


def timed(name: str, nbytes):
    """Bracket one entry-point call with events when launches are recorded.
    ``nbytes`` (an int or a callable returning one) is evaluated only then."""
    if _RECORDS is None:
        return _UNTIMED
    return _Timed(name, nbytes)


def nbytes(*tensors) -> int:
    """Bytes of the given tensors (None entries count zero)."""
    return sum(t.numel() * t.element_size() for t in tensors if t is not None)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return TS_BF16
    if dtype == torch.float32:
        return TS_F32
    raise NotImplementedError(f"hip backend computes in bfloat16 or float32, got {dtype}")
