"""Synthetic inputs shared by the CPU and GPU tests.

Builds the operator's paged inputs as numpy arrays: query ``[T, H, Dqk]``,
paged raw KV ``[NB1, BS1, Dqk]`` with a randomly permuted block table (unused
table slots ``-1``), paged compressed KV at ``cmp_ratio``, per-token top-k
indices drawn without replacement from the causally valid compressed
positions and ``-1`` padded, and per-head sinks ~ U(-1, 1).  The layout follows
the reference generators (golden.py:315-473); the value distribution is
N(0, 1) as the benchmark configurations ask.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from oracle import golden_ref as G


@dataclass
class Case:
    B: int
    H: int
    D: int
    Dv: int
    T: int
    scenario: int
    cmp_ratio: int
    win_left: int
    softmax_scale: float
    q_dtype: str
    kv_dtype: str
    cu_seqlens_q: np.ndarray
    q_prefix: np.ndarray
    act_q: np.ndarray
    seqused_kv: np.ndarray
    q_bits: np.ndarray  # uint16 (bf16/fp16) or float32
    ori_kv: np.ndarray  # uint16 / uint8 (fp8) payload [NB1, BS1, D]
    ori_block_table: np.ndarray
    sinks: np.ndarray
    cmp_kv: Optional[np.ndarray] = None
    cmp_block_table: Optional[np.ndarray] = None
    idx: Optional[np.ndarray] = None  # [T, K]
    ori_scale: Optional[np.ndarray] = None  # [NB1, BS1] fp32 (fp8 only)
    cmp_scale: Optional[np.ndarray] = None
    K: int = 0
    extra: Dict = field(default_factory=dict)

    # ---- float32 views (values the oracle computes on) ----
    def q_f32(self) -> np.ndarray:
        return _payload_f32(self.q_bits, self.q_dtype)

    def ori_f32(self) -> np.ndarray:
        return _kv_f32(self.ori_kv, self.kv_dtype, self.ori_scale)

    def cmp_f32(self) -> Optional[np.ndarray]:
        if self.cmp_kv is None:
            return None
        return _kv_f32(self.cmp_kv, self.kv_dtype, self.cmp_scale)

    def oracle_numpy(self, tokens=None):
        return G.golden_attention(
            q=self.q_f32(), ori_kv=self.ori_f32(), ori_block_table=self.ori_block_table,
            q_prefix=self.q_prefix, act_q=self.act_q, seqused_kv=self.seqused_kv,
            sinks=self.sinks, softmax_scale=self.softmax_scale, scenario=self.scenario,
            cmp_kv=self.cmp_f32(), cmp_block_table=self.cmp_block_table,
            cmp_sparse_indices=self.idx, cmp_ratio=self.cmp_ratio, win_left=self.win_left,
            d_v=self.Dv, q_dtype=self.q_dtype, tokens=tokens)

    def oracle_c(self, tokens=None, nthreads=0):
        from oracle import golden_c
        return golden_c.attention(
            q=self.q_bits, ori_kv=self.ori_kv, ori_block_table=self.ori_block_table,
            q_prefix=self.q_prefix, act_q=self.act_q, seqused_kv=self.seqused_kv,
            sinks=self.sinks, softmax_scale=self.softmax_scale, scenario=self.scenario,
            cmp_kv=self.cmp_kv, cmp_block_table=self.cmp_block_table,
            cmp_sparse_indices=self.idx, cmp_ratio=self.cmp_ratio, win_left=self.win_left,
            d_v=self.Dv, q_dtype=self.q_dtype, kv_dtype=self.kv_dtype,
            ori_scale=self.ori_scale, cmp_scale=self.cmp_scale, tokens=tokens,
            nthreads=nthreads)

    def oracle_exact(self, tokens=None, nthreads=0):
        """The float64 one-shot softmax over the same rows (no rounding)."""
        from oracle import golden_c
        return golden_c.attention(
            q=self.q_bits, ori_kv=self.ori_kv, ori_block_table=self.ori_block_table,
            q_prefix=self.q_prefix, act_q=self.act_q, seqused_kv=self.seqused_kv,
            sinks=self.sinks, softmax_scale=self.softmax_scale, scenario=self.scenario,
            cmp_kv=self.cmp_kv, cmp_block_table=self.cmp_block_table,
            cmp_sparse_indices=self.idx, cmp_ratio=self.cmp_ratio, win_left=self.win_left,
            d_v=self.Dv, q_dtype=self.q_dtype, kv_dtype=self.kv_dtype,
            ori_scale=self.ori_scale, cmp_scale=self.cmp_scale, tokens=tokens,
            nthreads=nthreads, exact=True)


def _payload_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return G.bf16_bits_to_f32(a)
    if dtype == "fp16":
        return a.view(np.float16).astype(np.float32)
    return a.astype(np.float32)


def _kv_f32(a: np.ndarray, dtype: str, scale: Optional[np.ndarray]) -> np.ndarray:
    if dtype == "fp8e4m3":
        return G.fp8e4m3_to_f32(a) * scale[..., None].astype(np.float32)
    return _payload_f32(a, dtype)


def _encode(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return G.f32_to_bf16_bits(x)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    return x.astype(np.float32)


def _encode_fp8_rows(x: np.ndarray):
    """Per-row scale amax/448 and OCP e4m3fn codes (round to nearest even)."""
    import torch

    amax = np.abs(x).max(axis=-1)
    scale = np.where(amax > 0, amax / 448.0, 1.0).astype(np.float32)
    y = torch.from_numpy((x / scale[..., None]).astype(np.float32))
    codes = y.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, scale


def make_case(
    *,
    B: int,
    H: int,
    seq_kv: Sequence[int],
    q_per_seq: Sequence[int] | int = 1,
    scenario: int = 3,
    K: int = 512,
    D: int = 576,
    Dv: int = 512,
    cmp_ratio: int = 4,
    block_size: int = 64,
    cmp_block_size: int = 64,
    win_left: int = 127,
    q_dtype: str = "bf16",
    kv_dtype: str = "bf16",
    seed: int = 0,
    extra_pages: int = 3,
    softmax_scale: Optional[float] = None,
    sink_range=(-1.0, 1.0),
    value_scale: float = 1.0,
    index_mode: str = "random",
    dist: str = "normal",
    pool_pages: Optional[int] = None,
    cmp_pool_pages: Optional[int] = None,
    q_spread: bool = False,
) -> Case:
    """``dist="normal"``: q and KV ~ N(0, value_scale^2) (the benchmark
    configurations).  ``dist="reference"``: the reference suite's own draws --
    q and raw KV ~ U(-10, 10), compressed KV ~ U(-5, 10)
    (test_sparse_attn_sharedkv.py:262, golden.py:315-408).

    ``pool_pages`` / ``cmp_pool_pages``: a shared page pool of that many pages,
    each sequence's block table a random permutation of it (truncated to the
    sequence's pages), so long contexts fit host memory; otherwise every
    sequence owns its pages (one random permutation over all of them).

    ``q_spread``: every head's queries scaled by its own 2^u, u in [-6, 2], and
    every element by 2^v, v in [-12, 0]; head 0 all zeros.  Magnitudes then span
    about 2^20 within a call and 2^12 within a head."""
    rng = np.random.default_rng(seed)
    seq_kv = [int(x) for x in seq_kv]
    qps = [int(q_per_seq)] * B if isinstance(q_per_seq, int) else [int(x) for x in q_per_seq]
    cu = np.zeros(B + 1, np.int32)
    cu[1:] = np.cumsum(qps)
    T = int(cu[-1])

    def draw(shape, lo_hi):
        if dist == "reference":
            return rng.uniform(lo_hi[0], lo_hi[1], size=shape).astype(np.float32)
        x = rng.standard_normal(shape, dtype=np.float32)
        return x if value_scale == 1.0 else x * np.float32(value_scale)

    q = draw((T, H, D), (-10.0, 10.0))
    if q_spread:
        q = q * np.exp2(rng.uniform(-6.0, 2.0, size=(1, H, 1))).astype(np.float32)
        q = q * np.exp2(rng.uniform(-12.0, 0.0, size=q.shape)).astype(np.float32)
        q[:, 0, :] = 0.0
    q_bits = _encode(q, q_dtype)

    def paged_pool(lens: List[int], bs: int, lo_hi, shared: Optional[int]):
        per = [math.ceil(n / bs) if n > 0 else 0 for n in lens]
        table = np.full((B, max(max(per), 1)), -1, np.int32)
        if shared is not None:
            assert max(per) <= shared, "a sequence needs more pages than the shared pool holds"
            nb = shared
            for b, n in enumerate(per):
                table[b, :n] = rng.permutation(nb)[:n].astype(np.int32)
        else:
            nb = sum(per) + extra_pages
            perm = rng.permutation(nb).astype(np.int32)
            cur = 0
            for b, n in enumerate(per):
                table[b, :n] = perm[cur:cur + n]
                cur += n
        vals = draw((nb, bs, D), lo_hi)
        return vals, table

    ori_vals, ori_bt = paged_pool(seq_kv, block_size, (-10.0, 10.0), pool_pages)
    cmp_vals = cmp_bt = None
    if scenario >= 2:
        cmp_vals, cmp_bt = paged_pool([n // cmp_ratio for n in seq_kv], cmp_block_size,
                                      (-5.0, 10.0), cmp_pool_pages)

    ori_scale = cmp_scale = None
    if kv_dtype == "fp8e4m3":
        ori_kv, ori_scale = _encode_fp8_rows(ori_vals)
        cmp_kv = None
        if cmp_vals is not None:
            cmp_kv, cmp_scale = _encode_fp8_rows(cmp_vals)
    else:
        ori_kv = _encode(ori_vals, kv_dtype)
        cmp_kv = None if cmp_vals is None else _encode(cmp_vals, kv_dtype)

    idx = None
    if scenario == 3:
        idx = np.full((T, K), -1, np.int32)
        for b in range(B):
            for s in range(qps[b]):
                thr = max(0, math.floor((seq_kv[b] - qps[b] + s + 1) / cmp_ratio))
                take = min(thr, K)
                if take == 0:
                    continue
                t = int(cu[b]) + s
                if index_mode == "random":
                    if thr > 4 * take:
                        sel = rng.choice(thr, size=take, replace=False)
                    else:
                        sel = rng.permutation(thr)[:take]
                elif index_mode == "ascending":
                    sel = np.arange(take)
                else:
                    raise ValueError(index_mode)
                idx[t, :take] = sel.astype(np.int32)

    sinks = rng.uniform(sink_range[0], sink_range[1], size=H).astype(np.float32)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    return Case(
        B=B, H=H, D=D, Dv=Dv, T=T, scenario=scenario, cmp_ratio=cmp_ratio,
        win_left=win_left, softmax_scale=scale, q_dtype=q_dtype, kv_dtype=kv_dtype,
        cu_seqlens_q=cu, q_prefix=cu[:-1].copy(), act_q=np.asarray(qps, np.int32),
        seqused_kv=np.asarray(seq_kv, np.int32), q_bits=q_bits, ori_kv=ori_kv,
        ori_block_table=ori_bt, sinks=sinks, cmp_kv=cmp_kv, cmp_block_table=cmp_bt,
        idx=idx, ori_scale=ori_scale, cmp_scale=cmp_scale, K=K if scenario == 3 else 0,
    )


# ---- comparison rules ----
def baseline_tolerance(real: np.ndarray, expect: np.ndarray, max_abs=2e-2, mean_abs=2e-3):
    """The benchmark tolerance for bf16 outputs: max-abs 2e-2 and mean-abs 2e-3."""
    d = np.abs(real.astype(np.float64) - expect.astype(np.float64))
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def check_result_rule(real: np.ndarray, expect: np.ndarray, dtype: str = "bf16"):
    """The reference's ``check_result`` rule (test_sparse_attn_sharedkv.py:394-467):
    >= 99.5% of elements within np.isclose at the dtype tolerance and the worst
    normalised relative error below 10.  Returns (fulfill_pct, max_rel)."""
    rtol, atol = (0.0078125, 0.0001) if dtype == "bf16" else (0.005, 0.000025)
    real = real.astype(np.float32).ravel()
    expt = expect.astype(np.float32).ravel()
    ok = np.isclose(real, expt, rtol=rtol, atol=atol, equal_nan=True)
    n_err = int((~ok).sum())
    fulfill = (real.size - n_err) / max(real.size, 1) * 100.0
    floor = (1.0 / (1 << 14)) / 0.005
    bnd = np.maximum(np.maximum(np.abs(real), np.abs(expt)), floor) + 1e-9
    rel = np.abs(real - expt) / bnd
    max_rel = float(rel[~ok].max()) if n_err else 0.0
    return fulfill, max_rel


def check_lse_rule(real: np.ndarray, expect: np.ndarray, dtype: str = "bf16"):
    """The reference's ``_check_lse`` rule (test_sparse_attn_sharedkv.py:470-527)."""
    rtol, atol = (0.015, 0.005) if dtype == "bf16" else (0.01, 0.001)
    real = real.astype(np.float32).ravel()
    expt = expect.astype(np.float32).ravel()
    ok = np.isclose(real, expt, rtol=rtol, atol=atol, equal_nan=True)
    n_err = int((~ok).sum())
    fulfill = (real.size - n_err) / max(real.size, 1) * 100.0
    floor = (1.0 / (1 << 14)) / 0.005
    bnd = np.maximum(np.maximum(np.abs(real), np.abs(expt)), floor) + 1e-9
    rel = np.abs(real - expt) / bnd
    max_rel = float(rel[~ok].max()) if n_err else 0.0
    return fulfill, max_rel
