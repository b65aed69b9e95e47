"""numpy restatement of the reference golden model -- TEST INFRASTRUCTURE ONLY.

Follows ``sparse_attn_sharedkv_tilelang/golden.py`` of the reference (cited per
function).  It works on the paged inputs directly: a logical position ``p`` of
batch ``b`` lives at row ``p % BS`` of page ``block_table[b, p // BS]``, which is
exactly what ``golden.unpack_paged_kv`` (golden.py:247-268) materialises before
the reference math runs; a ``-1`` page reads as a zero row there and here.

Conventions shared with the product's C ABI: queries are a flat ``[T, H, D]``
array; batch ``b`` owns tokens ``q_prefix[b] .. q_prefix[b] + act_q[b] - 1``
(TND: ``q_prefix = cu_seqlens_q[:-1]``; BSND: ``q_prefix[b] = b * S``).  Tokens
that no batch owns keep zero output and zero LSE, as the reference's padded
BNSD slots do (golden.py:106-111, 286-312).
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np

GOLDEN_S2_TILE = 512  # golden.py:25 -- the reference's S2 tile for the online softmax

SRC_ORI = 0
SRC_CMP = 1


# --------------------------------------------------------------------------
# Rounding helpers (the reference casts P and the output to q's dtype).
# --------------------------------------------------------------------------
def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even); returns float32.

    Adding 0x7FFF plus the lowest kept bit to the bit pattern and clearing the
    low 16 bits rounds to nearest even on the magnitude, for either sign.  For
    every non-NaN input the sum stays below 2^32 (the largest finite pattern is
    0xFF7FFFFF), so it runs in uint32; NaNs are restored afterwards."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(x.shape)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def _fp8e4m3_table() -> np.ndarray:
    """OCP FP8 E4M3FN decode table: bias 7, no infinities, S.1111.111 is NaN."""
    t = np.zeros(256, dtype=np.float32)
    for v in range(256):
        s = -1.0 if v & 0x80 else 1.0
        e = (v >> 3) & 0xF
        m = v & 0x7
        if e == 0xF and m == 0x7:
            t[v] = np.nan
        elif e == 0:
            t[v] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[v] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


FP8E4M3_TABLE = _fp8e4m3_table()


def fp8e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    return FP8E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


# --------------------------------------------------------------------------
# Row resolution: window, compressed indices, paging.
# --------------------------------------------------------------------------
def causal_position(act_kv: int, act_q: int, s_local: int) -> int:
    """golden.py:125 -- ``s_global = act_kv - act_q + s``."""
    return act_kv - act_q + s_local


def window_positions(s_global: int, win_left: int = 127, win_right: int = 0) -> range:
    """golden.py:129-131 -- ``[max(s_global - win_left, 0), s_global + win_right + 1)``."""
    right = s_global + win_right + 1
    left = max(s_global - win_left, 0)
    return range(left, max(right, left))


def cmp_threshold(act_kv: int, act_q: int, s_local: int, cmp_ratio: int) -> int:
    """golden.py:44 (and :147) -- ``floor((act_kv - act_q + s + 1) / cmp_ratio)``."""
    return math.floor((act_kv - act_q + s_local + 1) / cmp_ratio)


def resolve_cmp_ids(
    idx_row: Sequence[int], *, act_kv: int, act_q: int, s_local: int, cmp_ratio: int
) -> List[int]:
    """golden.py:28-66 (``_gather_cmp_kv_tokens``, sparse_block_size=1).

    Examines the first ``min(K, thr)`` slots only; ``-1`` terminates; an id at
    or beyond the threshold is skipped; the survivors keep their slot order and
    duplicates are kept.  Negative ids other than ``-1`` are outside the
    reference contract (Python indexing would wrap them); they are rejected
    here so a test can never silently depend on that wrap.
    """
    K = len(idx_row)
    cmp_act_kv = math.floor(act_kv / cmp_ratio)
    thr = cmp_threshold(act_kv, act_q, s_local, cmp_ratio)
    valid_count = min(K, thr)  # ceil(thr / sparse_block_size) with block size 1
    out: List[int] = []
    for i in range(max(valid_count, 0)):
        tid = int(idx_row[i])
        if tid == -1:
            break
        if tid < -1:
            raise ValueError(f"cmp index {tid} < -1 is outside the operator contract")
        begin, end = tid, tid + 1
        if end > cmp_act_kv:
            end = cmp_act_kv
        if begin >= thr:
            continue
        if end > thr:
            end = thr
        out.extend(range(begin, end))
    return out


def dense_cmp_ids(*, act_kv: int, act_q: int, s_local: int, cmp_ratio: int) -> List[int]:
    """golden.py:146-150 -- scenario 2 attends every compressed row below the threshold."""
    thr = cmp_threshold(act_kv, act_q, s_local, cmp_ratio)
    return list(range(max(thr, 0)))


def paged_row(block_table_row: np.ndarray, pos: int, block_size: int) -> int:
    """Closed form of golden.unpack_paged_kv (golden.py:256-267): the flat pool
    row ``page * block_size + pos % block_size`` holding logical position
    ``pos``, or ``-1`` when the page entry is negative (unpack leaves zeros)."""
    blk = pos // block_size
    if blk >= len(block_table_row):
        return -1
    page = int(block_table_row[blk])
    if page < 0:
        return -1
    return page * block_size + (pos % block_size)


def token_rows(
    *,
    b: int,
    s_local: int,
    act_q: int,
    act_kv: int,
    scenario: int,
    ori_block_table: np.ndarray,
    ori_block_size: int,
    cmp_block_table: Optional[np.ndarray],
    cmp_block_size: int,
    idx_row: Optional[np.ndarray],
    cmp_ratio: int,
    win_left: int = 127,
) -> Tuple[List[int], List[int]]:
    """Pool rows one query token attends, in the golden's walk order
    (golden.py:128-196): the window (ori pool) first, then the compressed rows
    (cmp pool) in resolved index order.  Returns ``(ori_rows, cmp_rows)``."""
    s_g = causal_position(act_kv, act_q, s_local)
    ori_rows = [paged_row(ori_block_table[b], p, ori_block_size)
                for p in window_positions(s_g, win_left)]
    if scenario == 3:
        ids = resolve_cmp_ids(idx_row, act_kv=act_kv, act_q=act_q, s_local=s_local,
                              cmp_ratio=cmp_ratio)
    elif scenario == 2:
        ids = dense_cmp_ids(act_kv=act_kv, act_q=act_q, s_local=s_local, cmp_ratio=cmp_ratio)
    else:
        ids = []
    cmp_rows = [paged_row(cmp_block_table[b], i, cmp_block_size) for i in ids]
    return ori_rows, cmp_rows


def unpack_paged(pool: np.ndarray, block_table: np.ndarray, max_len: int) -> np.ndarray:
    """golden.py:247-268 for N2=1: ``pool [NB, BS, D]`` -> dense ``[B, max_len, D]``."""
    NB, BS, D = pool.shape
    B = block_table.shape[0]
    out = np.zeros((B, max_len, D), dtype=pool.dtype)
    for b in range(B):
        for blk in range(block_table.shape[1]):
            phys = int(block_table[b, blk])
            if phys < 0:
                continue
            start = blk * BS
            if start >= max_len:
                break
            end = min(start + BS, max_len)
            out[b, start:end] = pool[phys, : end - start]
    return out


# --------------------------------------------------------------------------
# The math.
# --------------------------------------------------------------------------
def _gather(pool_flat: np.ndarray, rows: List[int]) -> np.ndarray:
    D = pool_flat.shape[-1]
    if not rows:
        return np.zeros((0, D), dtype=np.float32)
    idx = np.asarray(rows, dtype=np.int64)
    out = pool_flat[np.maximum(idx, 0)].astype(np.float32)
    out[idx < 0] = 0.0
    return out


def online_softmax_rows(
    q: np.ndarray,  # [G, D] float32
    ori_k: np.ndarray,  # [n_ori, D] float32
    cmp_k: np.ndarray,  # [n_cmp, D] float32
    sinks: np.ndarray,  # [G] float32
    softmax_scale: float,
    p_dtype: str,
    s2_tile: int = GOLDEN_S2_TILE,
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """golden.py:156-200 for one (b, n2, s): sink-seeded online softmax over
    the window tiles then the compressed tiles (tiles never mix the two
    sources), P rounded to the query dtype before PV.  Returns the float32
    un-cast output ``[G, D]``, ``row_max`` and ``row_sum``."""
    G, D = q.shape
    row_max = sinks.astype(np.float32).copy()
    row_sum = np.ones(G, dtype=np.float32)
    acc = np.zeros((G, D), dtype=np.float32)
    tiles = []
    for src in (ori_k, cmp_k):
        n = src.shape[0]
        for t in range(math.ceil(n / s2_tile) if n > 0 else 0):
            tiles.append(src[t * s2_tile:(t + 1) * s2_tile])
    with np.errstate(over="ignore", invalid="ignore"):
        for k_tile in tiles:
            score = (q @ k_tile.T).astype(np.float32) * np.float32(softmax_scale)
            row_max_old = row_max
            row_max = np.maximum(row_max, score.max(axis=1))
            alpha = np.exp(row_max_old - row_max).astype(np.float32)
            p = np.exp(score - row_max[:, None]).astype(np.float32)
            row_sum = (alpha * row_sum + p.sum(axis=1, dtype=np.float32)).astype(np.float32)
            p_low = round_to(p, p_dtype)
            acc = (acc * alpha[:, None] + p_low @ k_tile).astype(np.float32)
        out = (acc / row_sum[:, None]).astype(np.float32)
    return out, row_max, row_sum


def golden_attention(
    *,
    q: np.ndarray,  # [T, H, Dqk] float32 (values of the q dtype)
    ori_kv: np.ndarray,  # [NB1, BS1, Dqk] float32 (N2 = 1 squeezed)
    ori_block_table: np.ndarray,  # [B, L1] int
    q_prefix: Sequence[int],
    act_q: Sequence[int],
    seqused_kv: Sequence[int],
    sinks: np.ndarray,  # [H]
    softmax_scale: float,
    scenario: int,
    cmp_kv: Optional[np.ndarray] = None,  # [NB2, BS2, Dqk]
    cmp_block_table: Optional[np.ndarray] = None,
    cmp_sparse_indices: Optional[np.ndarray] = None,  # [T, K] int (N2 = 1 squeezed)
    cmp_ratio: int = 4,
    win_left: int = 127,
    d_v: Optional[int] = None,
    q_dtype: str = "bf16",
    tokens: Optional[Sequence[int]] = None,
) -> Tuple[np.ndarray, np.ndarray]:
    """golden.py:69-204 on paged TND inputs.

    Returns ``out [T, H, d_v]`` (float32 holding values of ``q_dtype``) and
    ``lse [T, H]`` (float32).  ``d_v`` columns of the reference output are the
    first ``d_v`` columns of the golden's full-width PV (V = leading columns of
    the K row; exact since PV is column-wise).  ``tokens`` restricts the work
    to a subset of flat token ids (others stay zero).
    """
    T, H, Dqk = q.shape
    d_v = Dqk if d_v is None else d_v
    out = np.zeros((T, H, d_v), dtype=np.float32)
    lse = np.zeros((T, H), dtype=np.float32)
    ori_flat = ori_kv.reshape(-1, ori_kv.shape[-1])
    cmp_flat = None if cmp_kv is None else cmp_kv.reshape(-1, cmp_kv.shape[-1])
    BS1 = ori_kv.shape[1]
    BS2 = 1 if cmp_kv is None else cmp_kv.shape[1]
    want = None if tokens is None else set(int(t) for t in tokens)
    for b in range(len(act_q)):
        aq, akv = int(act_q[b]), int(seqused_kv[b])
        for s in range(aq):
            t = int(q_prefix[b]) + s
            if want is not None and t not in want:
                continue
            ori_rows, cmp_rows = token_rows(
                b=b, s_local=s, act_q=aq, act_kv=akv, scenario=scenario,
                ori_block_table=ori_block_table, ori_block_size=BS1,
                cmp_block_table=cmp_block_table, cmp_block_size=BS2,
                idx_row=None if cmp_sparse_indices is None else cmp_sparse_indices[t],
                cmp_ratio=cmp_ratio, win_left=win_left,
            )
            ok = _gather(ori_flat, ori_rows)
            ck = _gather(cmp_flat, cmp_rows) if cmp_flat is not None else np.zeros((0, Dqk), np.float32)
            o, m, l = online_softmax_rows(q[t].astype(np.float32), ok, ck,
                                          np.asarray(sinks, np.float32), softmax_scale, q_dtype)
            out[t] = round_to(o[:, :d_v], q_dtype)
            with np.errstate(divide="ignore"):
                lse[t] = (m + np.log(l)).astype(np.float32)
    return out, lse


def sinks_softmax_reference_f64(
    q: np.ndarray, k_concat: np.ndarray, sinks: np.ndarray, softmax_scale: float
) -> Tuple[np.ndarray, np.ndarray]:
    """golden.py:207-244 in float64 without the low-precision casts: the
    textbook ``softmax(scores U sink) @ V`` with ``V = K`` and the sink as a
    zero-V logit.  ``q [G, D]``, ``k_concat [n, D]``; returns ``(out [G, D],
    lse [G])``."""
    q = q.astype(np.float64)
    k = k_concat.astype(np.float64)
    sink = np.asarray(sinks, np.float64)[:, None]
    score = (q @ k.T) * softmax_scale
    x = np.concatenate([score, sink], axis=1)
    with np.errstate(invalid="ignore"):
        x_max = np.max(x, axis=1, keepdims=True)
        y = np.exp(score - x_max)
        denom = y.sum(axis=1, keepdims=True) + np.exp(sink - x_max)
        out = (y / denom) @ k
        lse = (x_max + np.log(denom))[:, 0]
    return out, lse


# --------------------------------------------------------------------------
# Backward (no counterpart in the reference, which keeps the LSE for one:
# api.py:32-35, 176-184).  The gradient of the one-shot sink softmax over the
# same resolved rows, float64: with P_j = e^(s_j - lse), s_j = scale <q, K_j>,
# V_j = K_j[:d_v], out = sum_j P_j V_j and P_sink = e^(sink - lse):
#   D = <dO, out>,  dP_j = <dO, V_j>,  dS_j = P_j (dP_j - D)
#   dq = scale sum_j dS_j K_j,  dsink = -P_sink D,
#   dK_j += scale dS_j q,  dV_j += P_j dO  (V is the leading d_v columns of the
#   same row, so both land in that row's gradient).
# --------------------------------------------------------------------------
def golden_backward_f64(
    *,
    q: np.ndarray,  # [T, H, Dqk] values (float)
    ori_kv: np.ndarray,  # [NB1, BS1, Dqk] values
    ori_block_table: np.ndarray,
    q_prefix: Sequence[int],
    act_q: Sequence[int],
    seqused_kv: Sequence[int],
    sinks: np.ndarray,
    softmax_scale: float,
    scenario: int,
    dout: np.ndarray,  # [T, H, d_v]
    cmp_kv: Optional[np.ndarray] = None,
    cmp_block_table: Optional[np.ndarray] = None,
    cmp_sparse_indices: Optional[np.ndarray] = None,
    cmp_ratio: int = 4,
    win_left: int = 127,
    d_v: Optional[int] = None,
):
    """Returns ``(dq [T, H, Dqk], dsinks [H], dori [NB1, BS1, Dqk], dcmp or None)``
    in float64.  Rows read as zeros (unused pages) receive no gradient."""
    T, H, Dqk = q.shape
    d_v = Dqk if d_v is None else d_v
    dq = np.zeros((T, H, Dqk), np.float64)
    dsinks = np.zeros(H, np.float64)
    ori_flat = ori_kv.reshape(-1, Dqk).astype(np.float64)
    cmp_flat = None if cmp_kv is None else cmp_kv.reshape(-1, Dqk).astype(np.float64)
    dori = np.zeros_like(ori_flat)
    dcmp = None if cmp_flat is None else np.zeros_like(cmp_flat)
    BS1 = ori_kv.shape[1]
    BS2 = 1 if cmp_kv is None else cmp_kv.shape[1]
    sk = np.asarray(sinks, np.float64)
    for b in range(len(act_q)):
        aq, akv = int(act_q[b]), int(seqused_kv[b])
        for s in range(aq):
            t = int(q_prefix[b]) + s
            ori_rows, cmp_rows = token_rows(
                b=b, s_local=s, act_q=aq, act_kv=akv, scenario=scenario,
                ori_block_table=ori_block_table, ori_block_size=BS1,
                cmp_block_table=cmp_block_table, cmp_block_size=BS2,
                idx_row=None if cmp_sparse_indices is None else cmp_sparse_indices[t],
                cmp_ratio=cmp_ratio, win_left=win_left)
            src = [(ori_flat, dori, r) for r in ori_rows] + [(cmp_flat, dcmp, r) for r in cmp_rows]
            K = np.array([pool[r] if r >= 0 else np.zeros(Dqk) for pool, _, r in src]).reshape(-1, Dqk)
            qt = q[t].astype(np.float64)  # [H, Dqk]
            s_ = softmax_scale * (qt @ K.T)  # [H, n]
            m = np.maximum(sk, s_.max(axis=1) if s_.shape[1] else -np.inf)
            m = np.where(np.isfinite(m), m, 0.0)  # a head with nothing to attend: all zero
            e = np.exp(s_ - m[:, None])
            es = np.where(np.isneginf(sk), 0.0, np.exp(np.where(np.isneginf(sk), 0.0, sk) - m))
            l = es + e.sum(axis=1)
            safe = np.where(l > 0, l, 1.0)
            P = e / safe[:, None]
            Ps = es / safe
            V = K[:, :d_v]
            out = P @ V  # [H, d_v]
            dO = dout[t].astype(np.float64)
            Dh = (dO * out).sum(axis=1)
            dP = dO @ V.T
            dS = P * (dP - Dh[:, None])
            dq[t] = softmax_scale * (dS @ K)
            dsinks -= Ps * Dh
            gK = softmax_scale * (dS.T @ qt)  # [n, Dqk]
            gK[:, :d_v] += P.T @ dO
            for j, (_, grad, r) in enumerate(src):
                if r >= 0:
                    grad[r] += gK[j]
    dori = dori.reshape(ori_kv.shape)
    if dcmp is not None:
        dcmp = dcmp.reshape(cmp_kv.shape)
    return dq, dsinks, dori, dcmp


def golden_forward_f64(*, q, ori_kv, ori_block_table, q_prefix, act_q, seqused_kv, sinks,
                       softmax_scale, scenario, cmp_kv=None, cmp_block_table=None,
                       cmp_sparse_indices=None, cmp_ratio=4, win_left=127, d_v=None):
    """The one-shot sink softmax over the resolved rows in float64 (no rounding):
    ``out [T, H, d_v]``, the function golden_backward_f64 differentiates."""
    T, H, Dqk = q.shape
    d_v = Dqk if d_v is None else d_v
    out = np.zeros((T, H, d_v), np.float64)
    ori_flat = ori_kv.reshape(-1, Dqk)
    cmp_flat = None if cmp_kv is None else cmp_kv.reshape(-1, Dqk)
    BS1 = ori_kv.shape[1]
    BS2 = 1 if cmp_kv is None else cmp_kv.shape[1]
    for b in range(len(act_q)):
        aq, akv = int(act_q[b]), int(seqused_kv[b])
        for s in range(aq):
            t = int(q_prefix[b]) + s
            ori_rows, cmp_rows = token_rows(
                b=b, s_local=s, act_q=aq, act_kv=akv, scenario=scenario,
                ori_block_table=ori_block_table, ori_block_size=BS1,
                cmp_block_table=cmp_block_table, cmp_block_size=BS2,
                idx_row=None if cmp_sparse_indices is None else cmp_sparse_indices[t],
                cmp_ratio=cmp_ratio, win_left=win_left)
            rows = [(ori_flat, r) for r in ori_rows] + [(cmp_flat, r) for r in cmp_rows]
            K = np.array([pool[r] if r >= 0 else np.zeros(Dqk) for pool, r in rows],
                         np.float64).reshape(-1, Dqk)
            o, _ = sinks_softmax_reference_f64(q[t], K, sinks, softmax_scale)
            out[t] = o[:, :d_v]
    return out
