"""ctypes front-end of ``oracle/sas_golden.c`` -- TEST INFRASTRUCTURE ONLY.

Same semantics as :func:`oracle.golden_ref.golden_attention` (reference
``golden.py:69-204``) but in C with OpenMP over tokens, so parity cases and the
CPU baseline can run at sizes the numpy restatement cannot.  Arrays are numpy:
bf16/fp16 payloads are passed as ``uint16`` bit patterns, fp8 e4m3 as ``uint8``
codes with a float32 per-row scale.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libsas_golden.so")

DT_CODES = {"fp32": 0, "bf16": 1, "fp16": 2, "fp8e4m3": 3}


class SasgParams(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_int32), ("H", ctypes.c_int32), ("D", ctypes.c_int32),
        ("Dv", ctypes.c_int32), ("B", ctypes.c_int32),
        ("scenario", ctypes.c_int32), ("win_left", ctypes.c_int32),
        ("cmp_ratio", ctypes.c_int32), ("K", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32), ("kv_dtype", ctypes.c_int32),
        ("ori_block_size", ctypes.c_int32), ("ori_table_len", ctypes.c_int32),
        ("ori_block_num", ctypes.c_int32),
        ("cmp_block_size", ctypes.c_int32), ("cmp_table_len", ctypes.c_int32),
        ("cmp_block_num", ctypes.c_int32),
        ("ori_block_stride", ctypes.c_int64), ("ori_row_stride", ctypes.c_int64),
        ("cmp_block_stride", ctypes.c_int64), ("cmp_row_stride", ctypes.c_int64),
        ("softmax_scale", ctypes.c_float), ("nthreads", ctypes.c_int32),
    ]


_lib = None


def load():
    """Load the oracle library, building it with ``make`` if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    lib = ctypes.CDLL(_SO)
    P = ctypes.c_void_p
    lib.sasg_attention.argtypes = [ctypes.POINTER(SasgParams), P, P, P, P, P, P, P, P, P, P,
                                   P, P, P, ctypes.c_int32, P, P]
    lib.sasg_attention.restype = ctypes.c_int
    lib.sasg_attention_exact.argtypes = lib.sasg_attention.argtypes
    lib.sasg_attention_exact.restype = ctypes.c_int
    lib.sasg_resolve.argtypes = [ctypes.POINTER(SasgParams), P, P, P, P, P, P, ctypes.c_int32,
                                 P, P, P]
    lib.sasg_resolve.restype = ctypes.c_int
    lib.sasg_attention_bwd_exact.argtypes = [ctypes.POINTER(SasgParams), P, P, P, P, P, P, P, P,
                                             P, P, P, P, P, P, ctypes.c_int32, P, P, P, P]
    lib.sasg_attention_bwd_exact.restype = ctypes.c_int
    lib.sasg_round.argtypes = [ctypes.c_int, P, P, ctypes.c_int64]
    lib.sasg_round.restype = ctypes.c_int
    _lib = lib
    return lib


def round_array(x: np.ndarray, dtype: str) -> np.ndarray:
    """The C oracle's rounding of float32 values to ``dtype`` ("bf16" or "fp16"),
    returned as float32 (the step it applies to P before PV and to the output)."""
    src = np.ascontiguousarray(x, dtype=np.float32)
    dst = np.empty_like(src)
    rc = load().sasg_round(DT_CODES[dtype], _ptr(src), _ptr(dst), src.size)
    if rc != 0:
        raise RuntimeError(f"sasg_round: {rc}")
    return dst


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def _params(*, T, H, D, Dv, B, scenario, win_left, cmp_ratio, K, q_dtype, kv_dtype,
            ori_shape, ori_table_len, cmp_shape, cmp_table_len, softmax_scale, nthreads):
    p = SasgParams()
    p.T, p.H, p.D, p.Dv, p.B = T, H, D, Dv, B
    p.scenario, p.win_left, p.cmp_ratio, p.K = scenario, win_left, cmp_ratio, K
    p.q_dtype, p.kv_dtype = DT_CODES[q_dtype], DT_CODES[kv_dtype]
    p.ori_block_num, p.ori_block_size = ori_shape[0], ori_shape[1]
    p.ori_table_len = ori_table_len
    p.ori_block_stride, p.ori_row_stride = ori_shape[1] * D, D
    if cmp_shape is not None:
        p.cmp_block_num, p.cmp_block_size = cmp_shape[0], cmp_shape[1]
        p.cmp_block_stride, p.cmp_row_stride = cmp_shape[1] * D, D
    else:
        p.cmp_block_num, p.cmp_block_size, p.cmp_block_stride, p.cmp_row_stride = 1, 1, D, D
    p.cmp_table_len = cmp_table_len
    p.softmax_scale = float(softmax_scale)
    p.nthreads = nthreads
    return p


def attention(
    *,
    q: np.ndarray,  # [T, H, D]: float32, or uint16 bits when q_dtype is bf16/fp16
    ori_kv: np.ndarray,  # [NB1, BS1, D] (N2 = 1 squeezed), payload per kv_dtype
    ori_block_table: np.ndarray,
    q_prefix: Sequence[int],
    act_q: Sequence[int],
    seqused_kv: Sequence[int],
    sinks: np.ndarray,
    softmax_scale: float,
    scenario: int,
    cmp_kv: Optional[np.ndarray] = None,
    cmp_block_table: Optional[np.ndarray] = None,
    cmp_sparse_indices: Optional[np.ndarray] = None,  # [T, K]
    cmp_ratio: int = 4,
    win_left: int = 127,
    d_v: Optional[int] = None,
    q_dtype: str = "bf16",
    kv_dtype: str = "bf16",
    ori_scale: Optional[np.ndarray] = None,  # [NB1, BS1] float32 (fp8 only)
    cmp_scale: Optional[np.ndarray] = None,
    tokens: Optional[Sequence[int]] = None,
    nthreads: int = 0,
    exact: bool = False,
):
    """Returns ``(out [T, H, d_v] float32, lse [T, H] float32)``.

    ``exact=True`` evaluates the one-shot sink softmax over the same resolved
    rows in float64 with no intermediate or output rounding: the mathematical
    value both the reference golden model and the device kernel approximate."""
    lib = load()
    T, H, D = q.shape
    d_v = D if d_v is None else d_v
    B = len(act_q)
    K = 0 if cmp_sparse_indices is None else cmp_sparse_indices.shape[-1]
    qdt = np.float32 if q_dtype == "fp32" else np.uint16
    kdt = {"fp32": np.float32, "bf16": np.uint16, "fp16": np.uint16, "fp8e4m3": np.uint8}[kv_dtype]
    q_a = _c(q, qdt)
    ori_a = _c(ori_kv, kdt)
    cmp_a = _c(cmp_kv, kdt)
    obt = _c(ori_block_table, np.int32)
    cbt = _c(cmp_block_table, np.int32)
    idx = _c(cmp_sparse_indices.reshape(T, -1) if cmp_sparse_indices is not None else None, np.int32)
    qp = _c(np.asarray(q_prefix), np.int32)
    aq = _c(np.asarray(act_q), np.int32)
    skv = _c(np.asarray(seqused_kv), np.int32)
    snk = _c(sinks, np.float32)
    osc = _c(ori_scale, np.float32)
    csc = _c(cmp_scale, np.float32)
    tok = _c(np.asarray(tokens), np.int32) if tokens is not None else None
    out = np.zeros((T, H, d_v), dtype=np.float32)
    lse = np.zeros((T, H), dtype=np.float32)
    p = _params(T=T, H=H, D=D, Dv=d_v, B=B, scenario=scenario, win_left=win_left,
                cmp_ratio=cmp_ratio, K=K, q_dtype=q_dtype, kv_dtype=kv_dtype,
                ori_shape=ori_a.shape, ori_table_len=obt.shape[1],
                cmp_shape=None if cmp_a is None else cmp_a.shape,
                cmp_table_len=1 if cbt is None else cbt.shape[1],
                softmax_scale=softmax_scale, nthreads=nthreads)
    fn = lib.sasg_attention_exact if exact else lib.sasg_attention
    rc = fn(ctypes.byref(p), _ptr(q_a), _ptr(ori_a), _ptr(osc), _ptr(obt),
                            _ptr(cmp_a), _ptr(csc), _ptr(cbt), _ptr(idx), _ptr(qp), _ptr(aq),
                            _ptr(skv), _ptr(snk), _ptr(tok),
                            0 if tok is None else len(tok), _ptr(out), _ptr(lse))
    if rc != 0:
        raise ValueError(f"oracle rejected the inputs (code {rc})")
    return out, lse


def resolve(
    *,
    T: int,
    ori_block_table: np.ndarray,
    ori_block_size: int,
    q_prefix: Sequence[int],
    act_q: Sequence[int],
    seqused_kv: Sequence[int],
    scenario: int,
    cmp_block_table: Optional[np.ndarray] = None,
    cmp_block_size: int = 1,
    cmp_sparse_indices: Optional[np.ndarray] = None,
    cmp_ratio: int = 4,
    win_left: int = 127,
    max_rows: Optional[int] = None,
):
    """Rows every token attends, golden walk order.  Returns ``(rows [T, max_rows]
    int64 pool rows (-1 = unpaged), n_ori [T], n_cmp [T])``."""
    lib = load()
    B = len(act_q)
    K = 0 if cmp_sparse_indices is None else cmp_sparse_indices.reshape(T, -1).shape[1]
    if max_rows is None:
        max_rows = win_left + 1 + (K if scenario == 3 else 0)
        if scenario == 2:
            max_rows += max(int(x) for x in seqused_kv) // cmp_ratio + 1
    obt = _c(ori_block_table, np.int32)
    cbt = _c(cmp_block_table, np.int32)
    idx = _c(cmp_sparse_indices.reshape(T, -1) if cmp_sparse_indices is not None else None, np.int32)
    p = _params(T=T, H=1, D=1, Dv=1, B=B, scenario=scenario, win_left=win_left,
                cmp_ratio=cmp_ratio, K=K, q_dtype="fp32", kv_dtype="fp32",
                ori_shape=(1, ori_block_size), ori_table_len=obt.shape[1],
                cmp_shape=None if cbt is None else (1, cmp_block_size),
                cmp_table_len=1 if cbt is None else cbt.shape[1], softmax_scale=1.0, nthreads=1)
    rows = np.full((T, max_rows), -1, dtype=np.int64)
    n_ori = np.zeros(T, np.int32)
    n_cmp = np.zeros(T, np.int32)
    rc = lib.sasg_resolve(ctypes.byref(p), _ptr(obt), _ptr(cbt), _ptr(idx),
                          _ptr(_c(np.asarray(q_prefix), np.int32)),
                          _ptr(_c(np.asarray(act_q), np.int32)),
                          _ptr(_c(np.asarray(seqused_kv), np.int32)), max_rows, _ptr(rows),
                          _ptr(n_ori), _ptr(n_cmp))
    if rc != 0:
        raise ValueError(f"oracle resolve failed (code {rc})")
    return rows, n_ori, n_cmp


def backward_exact(
    *,
    q: np.ndarray,
    ori_kv: np.ndarray,
    ori_block_table: np.ndarray,
    q_prefix: Sequence[int],
    act_q: Sequence[int],
    seqused_kv: Sequence[int],
    sinks: np.ndarray,
    softmax_scale: float,
    scenario: int,
    dout: np.ndarray,  # [T, H, d_v] float32 values
    cmp_kv: Optional[np.ndarray] = None,
    cmp_block_table: Optional[np.ndarray] = None,
    cmp_sparse_indices: Optional[np.ndarray] = None,
    cmp_ratio: int = 4,
    win_left: int = 127,
    d_v: Optional[int] = None,
    q_dtype: str = "bf16",
    kv_dtype: str = "bf16",
    ori_scale: Optional[np.ndarray] = None,
    cmp_scale: Optional[np.ndarray] = None,
    tokens: Optional[Sequence[int]] = None,
    nthreads: int = 0,
    kv_grad: bool = False,
):
    """The float64 backward of the exact forward over the same resolved rows:
    ``(dq [T, H, D], dsinks [H], dori, dcmp)`` as float32 (the pool gradients in
    the pools' [NB, BS, D] shape when ``kv_grad``, else None)."""
    lib = load()
    T, H, D = q.shape
    d_v = D if d_v is None else d_v
    B = len(act_q)
    K = 0 if cmp_sparse_indices is None else cmp_sparse_indices.reshape(T, -1).shape[1]
    qdt = np.float32 if q_dtype == "fp32" else np.uint16
    kdt = {"fp32": np.float32, "bf16": np.uint16, "fp16": np.uint16, "fp8e4m3": np.uint8}[kv_dtype]
    q_a = _c(q, qdt)
    ori_a = _c(ori_kv, kdt)
    cmp_a = _c(cmp_kv, kdt)
    obt = _c(ori_block_table, np.int32)
    cbt = _c(cmp_block_table, np.int32)
    idx = _c(cmp_sparse_indices.reshape(T, -1) if cmp_sparse_indices is not None else None, np.int32)
    tok = _c(np.asarray(tokens), np.int32) if tokens is not None else None
    dq = np.zeros((T, H, D), np.float32)
    ds = np.zeros(H, np.float32)
    dori = np.zeros(ori_a.shape[:2] + (D,), np.float32) if kv_grad else None
    dcmp = np.zeros(cmp_a.shape[:2] + (D,), np.float32) if (kv_grad and cmp_a is not None) else None
    p = _params(T=T, H=H, D=D, Dv=d_v, B=B, scenario=scenario, win_left=win_left,
                cmp_ratio=cmp_ratio, K=K, q_dtype=q_dtype, kv_dtype=kv_dtype,
                ori_shape=ori_a.shape, ori_table_len=obt.shape[1],
                cmp_shape=None if cmp_a is None else cmp_a.shape,
                cmp_table_len=1 if cbt is None else cbt.shape[1],
                softmax_scale=softmax_scale, nthreads=nthreads)
    rc = lib.sasg_attention_bwd_exact(
        ctypes.byref(p), _ptr(q_a), _ptr(ori_a), _ptr(_c(ori_scale, np.float32)), _ptr(obt),
        _ptr(cmp_a), _ptr(_c(cmp_scale, np.float32)), _ptr(cbt), _ptr(idx),
        _ptr(_c(np.asarray(q_prefix), np.int32)), _ptr(_c(np.asarray(act_q), np.int32)),
        _ptr(_c(np.asarray(seqused_kv), np.int32)), _ptr(_c(sinks, np.float32)),
        _ptr(_c(dout, np.float32)), _ptr(tok), 0 if tok is None else len(tok), _ptr(dq), _ptr(ds),
        _ptr(dori), _ptr(dcmp))
    if rc != 0:
        raise ValueError(f"oracle rejected the inputs (code {rc})")
    return dq, ds, dori, dcmp
