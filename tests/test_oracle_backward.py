"""The backward oracle (test infrastructure), pinned without a GPU.

The reference has no backward (it keeps the LSE for one: api.py:32-35,
176-184), so the oracle is pinned by the mathematics: central finite
differences of the float64 forward (the one-shot sink softmax over the same
resolved rows, golden.py:207-244) against the analytic gradients, on small
cases that exercise the window, the top-k list (a -1 terminator, ids beyond
the threshold, duplicates), unused pages read as zeros, sinks of -inf and
empty tokens; then the C restatement against the numpy one.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import golden_c
from oracle import golden_ref as G
from tests.cases import make_case


def _small_case(scenario, seed):
    c = make_case(B=3, H=3, D=40, Dv=32, seq_kv=[70, 9, 2], q_per_seq=[2, 3, 3],
                  scenario=scenario, K=12 if scenario == 3 else 0, block_size=8, cmp_block_size=4,
                  win_left=5, seed=seed, q_dtype="bf16", kv_dtype="bf16")
    if scenario == 3:
        c.idx[0, 4] = -1          # terminates token 0's list
        c.idx[1, 0] = 500         # beyond the threshold: skipped
        c.idx[1, 3] = c.idx[1, 2]  # a duplicate counts twice
    c.ori_block_table[0, 3] = -1   # an unused page inside token windows
    c.sinks[1] = -np.inf
    return c


def _kw(c, scale=0.3):
    return dict(ori_block_table=c.ori_block_table, q_prefix=c.q_prefix, act_q=c.act_q,
                seqused_kv=c.seqused_kv, softmax_scale=scale, scenario=c.scenario,
                cmp_block_table=c.cmp_block_table, cmp_sparse_indices=c.idx,
                cmp_ratio=c.cmp_ratio, win_left=c.win_left, d_v=c.Dv)


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_backward_f64_matches_finite_differences(scenario):
    c = _small_case(scenario, seed=10 + scenario)
    q = c.q_f32().astype(np.float64)
    ori = c.ori_f32().astype(np.float64)
    cmp = None if c.cmp_kv is None else c.cmp_f32().astype(np.float64)
    sinks = c.sinks.astype(np.float64)
    rng = np.random.default_rng(scenario)
    dO = rng.standard_normal((c.T, c.H, c.Dv))
    kw = _kw(c)
    dq, ds, dori, dcmp = G.golden_backward_f64(q=q, ori_kv=ori, cmp_kv=cmp, sinks=sinks, dout=dO,
                                                **kw)

    def loss(q_=q, o_=ori, c_=cmp, s_=sinks):
        return float((G.golden_forward_f64(q=q_, ori_kv=o_, cmp_kv=c_, sinks=s_, **kw) * dO).sum())

    h = 1e-6

    def fd(arr, i, key):
        p, m = arr.copy(), arr.copy()
        p[i] += h
        m[i] -= h
        return (loss(**{key: p}) - loss(**{key: m})) / (2 * h)

    picks = [tuple(x) for x in rng.integers(0, [c.T, c.H, c.D], size=(6, 3))]
    for i in picks:
        assert abs(fd(q, i, "q_") - dq[i]) <= 1e-6 * (1 + abs(dq[i])), ("dq", i)
    for j in range(c.H):
        if np.isfinite(sinks[j]):
            assert abs(fd(sinks, j, "s_") - ds[j]) <= 1e-6 * (1 + abs(ds[j])), ("dsink", j)
        else:
            assert ds[j] == 0.0
    for grad, arr, key in ((dori, ori, "o_"), (dcmp, cmp, "c_")):
        if arr is None:
            continue
        nz = np.argwhere(np.abs(grad) > 0)
        assert len(nz), key
        for i in [tuple(x) for x in nz[rng.choice(len(nz), size=min(6, len(nz)), replace=False)]]:
            assert abs(fd(arr, i, key) - grad[i]) <= 1e-6 * (1 + abs(grad[i])), (key, i)
    # an unused page gets no gradient; an empty token (batch 2 starts at s_global < 0) none
    pg = int(c.ori_block_table[0, 3]) if c.ori_block_table[0, 3] >= 0 else None
    assert pg is None
    assert not dq[int(c.q_prefix[2])].any()


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_c_backward_matches_numpy(scenario):
    c = make_case(B=3, H=5, D=576, seq_kv=[300, 9, 2000], q_per_seq=[2, 3, 1], scenario=scenario,
                  K=40 if scenario == 3 else 0, seed=20 + scenario,
                  cmp_ratio=4 if scenario != 2 else 64)
    rng = np.random.default_rng(scenario)
    dO = rng.standard_normal((c.T, c.H, 512)).astype(np.float32)
    kw = _kw(c, scale=c.softmax_scale)
    a = G.golden_backward_f64(q=c.q_f32(), ori_kv=c.ori_f32(),
                              cmp_kv=None if c.cmp_kv is None else c.cmp_f32(), sinks=c.sinks,
                              dout=dO, **kw)
    b = golden_c.backward_exact(q=c.q_bits, ori_kv=c.ori_kv, cmp_kv=c.cmp_kv, sinks=c.sinks,
                                dout=dO, kv_grad=True, **kw)
    for name, x, y in zip(("dq", "dsinks", "dori", "dcmp"), a, b):
        if x is None:
            assert y is None
            continue
        assert np.abs(x - y).max() <= 1e-6 * max(1.0, float(np.abs(x).max())), name


def test_planted_missing_d_term_is_caught():
    """dS = P (dP - D): dropping D (the FA-2 row term) changes dq measurably."""
    c = _small_case(3, seed=31)
    q = c.q_f32().astype(np.float64)
    dO = np.random.default_rng(1).standard_normal((c.T, c.H, c.Dv))
    kw = _kw(c)
    dq, *_ = G.golden_backward_f64(q=q, ori_kv=c.ori_f32(), cmp_kv=c.cmp_f32(), sinks=c.sinks,
                                   dout=dO, **kw)
    # the same gradient without D: differs from finite differences of the forward
    h = 1e-6
    i = (0, 0, 3)

    def loss(q_):
        return float((G.golden_forward_f64(q=q_, ori_kv=c.ori_f32(), cmp_kv=c.cmp_f32(),
                                           sinks=c.sinks, **kw) * dO).sum())

    p, m = q.copy(), q.copy()
    p[i] += h
    m[i] -= h
    fd = (loss(p) - loss(m)) / (2 * h)
    assert abs(fd - dq[i]) < 1e-6
    ori_rows, cmp_rows = G.token_rows(
        b=0, s_local=0, act_q=int(c.act_q[0]), act_kv=int(c.seqused_kv[0]), scenario=3,
        ori_block_table=c.ori_block_table, ori_block_size=c.ori_kv.shape[1],
        cmp_block_table=c.cmp_block_table, cmp_block_size=c.cmp_kv.shape[1], idx_row=c.idx[0],
        cmp_ratio=4, win_left=c.win_left)
    ori_f, cmp_f = c.ori_f32().reshape(-1, c.D), c.cmp_f32().reshape(-1, c.D)
    K = np.array([ori_f[r] if r >= 0 else np.zeros(c.D) for r in ori_rows] +
                 [cmp_f[r] for r in cmp_rows], np.float64)
    s_ = 0.3 * (K @ q[0, 0])
    mx = max(float(c.sinks[0]), s_.max())
    e = np.exp(s_ - mx)
    P = e / (e.sum() + np.exp(c.sinks[0] - mx))
    no_d = 0.3 * ((P * (K[:, :c.Dv] @ dO[0, 0])) @ K)[3]
    assert abs(no_d - fd) > 1e-3
