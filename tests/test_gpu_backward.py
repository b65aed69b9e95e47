"""GPU backward (queries, sinks and the KV pools) against the oracle's float64
gradients.

The reference has no backward (it keeps the LSE for one: api.py:32-35,
176-184), so parity is with the mathematics: the float64 gradient of the
one-shot sink softmax over the same resolved rows (oracle
``sasg_attention_bwd_exact``, itself pinned by finite differences in
tests/test_oracle_backward.py).

Tolerance.  The kernel computes in fp32 from the query dtype's inputs, rounds
dS to that dtype for the dq MFMA, and forms D = <dO, out> from the forward's
rounded output (as FlashAttention-2 does).  dS = P (dP - D) loses relative
precision where dP and D nearly cancel, so the bound is on the whole tensor:
the Frobenius error at most 0.5% of the exact gradient's norm and the largest
element error at most 1% of its largest element (measured on MI355X: 1.1e-3 to
2.7e-3 and 1.1e-3 to 3.2e-3 with bf16; 1.8e-4 with fp16); dsinks alike.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.cases import make_case
from tests.gpu_helpers import FIGURES, TORCH_DT, to_device

pytestmark = pytest.mark.gpu


def _exact_grads(c, dout, tokens=None, kv_grad=False):
    from oracle import golden_c

    kw = dict(q=c.q_bits, ori_kv=c.ori_kv, ori_block_table=c.ori_block_table, q_prefix=c.q_prefix,
              act_q=c.act_q, seqused_kv=c.seqused_kv, sinks=c.sinks, softmax_scale=c.softmax_scale,
              scenario=c.scenario, cmp_kv=c.cmp_kv, cmp_block_table=c.cmp_block_table,
              cmp_sparse_indices=c.idx, cmp_ratio=c.cmp_ratio, win_left=c.win_left, d_v=c.Dv,
              q_dtype=c.q_dtype, kv_dtype=c.kv_dtype, tokens=tokens, kv_grad=kv_grad)
    return golden_c.backward_exact(dout=dout.astype(np.float32), **kw)


def _check_grad(label, got, want, fro_tol=5e-3, max_tol=1e-2):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    nw = float(np.linalg.norm(want)) or 1.0
    mw = float(np.abs(want).max()) or 1.0
    fro, mx = float(np.linalg.norm(err)) / nw, float(err.max()) / mw
    msg = f"{label}: rel_fro={fro:.2e} rel_max={mx:.2e} (|want|max={mw:.3e})"
    print(msg, flush=True)
    FIGURES.append(dict(case=label, max_abs=float(err.max()), mean_abs=float(err.mean()),
                        cr_vs_oracle=float("nan"), lse_vs_oracle=float("nan")))
    assert np.isfinite(got).all(), label
    assert fro <= fro_tol and mx <= max_tol, msg
    return fro, mx


def _launch(c, core_num=256):
    from dsv4_planb_amd.api import build_launch

    d = to_device(c)
    cu = d["cu_seqlens_q"]
    launch, out, lse = build_launch(
        q_flat=d["q"], ori_kv=d["ori_kv"], ori_block_table=d["ori_block_table"],
        cmp_kv=d.get("cmp_kv"), cmp_block_table=d.get("cmp_block_table"),
        cmp_indices=d.get("cmp_sparse_indices"), q_prefix=cu[:-1], act_q_lens=cu[1:] - cu[:-1],
        seqused_kv=d["seqused_kv"], sinks=d["sinks"], metadata=None, scenario=c.scenario,
        topk=c.K, cmp_ratio=c.cmp_ratio, ori_win_left=c.win_left, softmax_scale=c.softmax_scale,
        core_num=core_num)
    launch.run()
    return launch, out, lse


def _dout(c, seed):
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((c.T, c.H, c.Dv)).astype(np.float32)
    t = torch.from_numpy(g).to(TORCH_DT[c.q_dtype])  # the values the kernel sees
    return t, t.float().numpy()


def _edges():
    c = make_case(B=4, H=32, seq_kv=[900, 3000, 2, 64], q_per_seq=[2, 3, 3, 1], scenario=3, K=256,
                  seed=108)
    c.idx[0, 3] = -1
    c.idx[1, 0] = 10_000
    c.idx[1, 5] = int(c.idx[1, 4])
    c.ori_block_table[1, 2] = -1
    c.sinks[:4] = -np.inf
    return c


@pytest.mark.parametrize("name,build,cores", [
    ("bwd_swa_h16", lambda: make_case(B=2, H=16, seq_kv=[1024, 700], q_per_seq=[1, 2], scenario=1,
                                      seed=101), 256),
    ("bwd_decode_h64_k512", lambda: make_case(B=4, H=64, seq_kv=[5000, 1300, 9000, 300],
                                              q_per_seq=[1, 2, 1, 3], scenario=3, K=512,
                                              seed=102), 256),
    ("bwd_mtp_h128_k2048", lambda: make_case(B=3, H=128, seq_kv=[131072] * 3, q_per_seq=2,
                                             scenario=3, K=2048, seed=103, pool_pages=2100,
                                             cmp_pool_pages=600), 256),
    ("bwd_split_tokens", lambda: make_case(B=2, H=16, seq_kv=[20000, 4000], q_per_seq=1,
                                           scenario=3, K=2048, seed=104), 1024),
    ("bwd_cfa", lambda: make_case(B=1, H=64, seq_kv=[8193], q_per_seq=2, scenario=2, K=0,
                                  cmp_ratio=128, block_size=128, cmp_block_size=128, seed=105), 256),
    ("bwd_fp16", lambda: make_case(B=3, H=64, seq_kv=[3000, 700, 9000], q_per_seq=[1, 2, 3],
                                   scenario=3, K=512, q_dtype="fp16", kv_dtype="fp16",
                                   seed=106), 256),
    ("bwd_d512", lambda: make_case(B=2, H=128, D=512, seq_kv=[5000, 12000], q_per_seq=2,
                                   scenario=3, K=1024, seed=107), 256),
    ("bwd_edges", _edges, 256),
    ("bwd_prefill", lambda: make_case(B=1, H=128, seq_kv=[512], q_per_seq=512, scenario=3, K=2048,
                                      seed=109), 256),
])
def test_backward_matches_f64_gradient(name, build, cores):
    c = build()
    print(f"\n[case] {name}: B={c.B} T={c.T} H={c.H} D={c.D} scen={c.scenario} K={c.K} "
          f"q={c.q_dtype} cores={cores}", flush=True)
    launch, out, lse = _launch(c, cores)
    g, g_np = _dout(c, seed=sum(name.encode()))
    dq, dsinks = launch.backward(g.cuda())
    torch.cuda.synchronize()
    dq_ex, ds_ex, _, _ = _exact_grads(c, g_np)
    _check_grad(f"{name}:dq", dq.cpu().numpy(), dq_ex)
    _check_grad(f"{name}:dsinks", dsinks.cpu().numpy(), ds_ex)


def test_backward_lse_gradient_enters_as_d_minus_dlse():
    """A gradient g on the LSE alone (dout = 0): dq is the gradient of <g, lse>,
    checked as a directional derivative against a central finite difference of
    the oracle's exact LSE (fp32 queries, float64 arithmetic) along a random
    direction u; dsinks = sum_t g e^(sink - lse), as d lse / d sink = P_sink."""
    from oracle import golden_c

    c = make_case(B=2, H=16, seq_kv=[3000, 900], q_per_seq=[1, 2], scenario=3, K=256, seed=111)
    launch, out, lse = _launch(c)
    zero = torch.zeros((c.T, c.H, c.Dv), dtype=torch.bfloat16, device="cuda")
    gl = torch.from_numpy(np.random.default_rng(5).standard_normal((c.T, c.H)).astype(np.float32))
    dq, dsinks = launch.backward(zero, gl.cuda())
    torch.cuda.synchronize()
    # exact: dL/dq_h = scale * sum_j g_h P_j K_j, dL/dsink_h = sum_t g P_sink
    kw = dict(ori_block_table=c.ori_block_table, q_prefix=c.q_prefix, act_q=c.act_q,
              seqused_kv=c.seqused_kv, scenario=c.scenario, cmp_kv=c.cmp_kv,
              cmp_block_table=c.cmp_block_table, cmp_sparse_indices=c.idx, cmp_ratio=c.cmp_ratio,
              win_left=c.win_left, d_v=c.Dv, q_dtype=c.q_dtype, kv_dtype=c.kv_dtype)
    rng = np.random.default_rng(6)
    u = rng.standard_normal(c.q_bits.shape).astype(np.float32) * 1e-2
    qf = c.q_f32()
    e = 1e-1

    def lse_at(qv):
        _, l = golden_c.attention(q=qv, ori_kv=c.ori_kv, sinks=c.sinks, softmax_scale=c.softmax_scale,
                                  exact=True, **dict(kw, q_dtype="fp32"))
        return l.astype(np.float64)

    fd = ((lse_at(qf + e * u) - lse_at(qf - e * u)) / (2 * e) * gl.numpy()).sum()
    got = float((dq.cpu().numpy().astype(np.float64) * u).sum())
    print(f"dlse directional: device {got:.6e} finite-difference {fd:.6e}", flush=True)
    assert abs(got - fd) <= 1e-2 * abs(fd) + 1e-6
    # the sink: d lse / d sink = P_sink = e^(sink - lse)
    want_ds = (gl.numpy() * np.exp(c.sinks[None, :] - lse.cpu().numpy())).sum(axis=0)
    _check_grad("dlse:dsinks", dsinks.cpu().numpy(), want_ds, fro_tol=1e-3, max_tol=2e-3)


@pytest.mark.parametrize("layout", ["TND", "BSND"])
def test_autograd_through_the_api(layout):
    """q and sinks requiring grad make sparse_attn_sharedkv differentiable: the
    gradients of sum(out * w) match the oracle's float64 gradient."""
    from dsv4_planb_amd import sparse_attn_sharedkv

    c = make_case(B=2, H=64, seq_kv=[5000, 1300], q_per_seq=2, scenario=3, K=512, seed=112)
    print(f"\n[case] autograd {layout}: T={c.T} H={c.H}", flush=True)
    d = to_device(c)
    q = d.pop("q")
    if layout == "BSND":
        q = q.reshape(c.B, 2, c.H, c.D)
        d["cmp_sparse_indices"] = d["cmp_sparse_indices"].reshape(c.B, 2, 1, c.K)
    q = q.detach().requires_grad_(True)
    sinks = d.pop("sinks").detach().requires_grad_(True)
    out, lse = sparse_attn_sharedkv(q, sinks=sinks, softmax_scale=c.softmax_scale, cmp_ratio=4,
                                    layout_q=layout, return_softmax_lse=True, topk_cmp=c.K, **d)
    g, g_np = _dout(c, seed=7)
    w = g.cuda().reshape(out.shape)
    (out.float() * w.float()).sum().backward()
    torch.cuda.synchronize()
    assert q.grad is not None and q.grad.dtype == q.dtype and q.grad.shape == q.shape
    assert sinks.grad is not None and sinks.grad.dtype == torch.float32
    dq_ex, ds_ex, _, _ = _exact_grads(c, g_np)
    _check_grad(f"autograd-{layout}:dq", q.grad.float().reshape(c.T, c.H, c.D).cpu().numpy(), dq_ex)
    _check_grad(f"autograd-{layout}:dsinks", sinks.grad.cpu().numpy(), ds_ex)


KV_CASES = [
    ("kv_swa_h16", lambda: make_case(B=2, H=16, seq_kv=[1024, 700], q_per_seq=[1, 2], scenario=1,
                                     seed=121), 256),
    ("kv_decode_h64_k512", lambda: make_case(B=4, H=64, seq_kv=[5000, 1300, 9000, 300],
                                             q_per_seq=[1, 2, 1, 3], scenario=3, K=512,
                                             seed=122), 256),
    ("kv_mtp_h128_k2048", lambda: make_case(B=2, H=128, seq_kv=[131072] * 2, q_per_seq=2,
                                            scenario=3, K=2048, seed=123, pool_pages=2100,
                                            cmp_pool_pages=600), 256),
    ("kv_split_tokens", lambda: make_case(B=2, H=16, seq_kv=[20000, 4000], q_per_seq=1,
                                          scenario=3, K=2048, seed=124), 1024),
    ("kv_cfa", lambda: make_case(B=1, H=64, seq_kv=[8193], q_per_seq=2, scenario=2, K=0,
                                 cmp_ratio=128, block_size=128, cmp_block_size=128, seed=125), 256),
    ("kv_fp16", lambda: make_case(B=3, H=64, seq_kv=[3000, 700, 9000], q_per_seq=[1, 2, 3],
                                  scenario=3, K=512, q_dtype="fp16", kv_dtype="fp16", seed=126), 256),
    ("kv_d512", lambda: make_case(B=2, H=128, D=512, seq_kv=[5000, 12000], q_per_seq=2,
                                  scenario=3, K=1024, seed=127), 256),
    ("kv_edges", _edges, 256),
    ("kv_prefill", lambda: make_case(B=1, H=128, seq_kv=[512], q_per_seq=512, scenario=3, K=2048,
                                     seed=129), 256),
]


def _check_pools(name, c, d_ori, d_cmp, dori_ex, dcmp_ex):
    # rows no token reads stay exactly zero on both sides
    got = d_ori.squeeze(2).cpu().numpy()
    assert np.abs(got[dori_ex == 0]).max(initial=0.0) == 0, name
    _check_grad(f"{name}:d_ori_kv", got, dori_ex)
    if c.scenario >= 2:
        gc = d_cmp.squeeze(2).cpu().numpy()
        assert np.abs(gc[dcmp_ex == 0]).max(initial=0.0) == 0, name
        _check_grad(f"{name}:d_cmp_kv", gc, dcmp_ex)
    else:
        assert d_cmp is None


@pytest.mark.parametrize("name,build,cores", KV_CASES)
def test_backward_kv_pools_match_f64_gradient(name, build, cores):
    """The pools' gradient: every row sums dK = scale sum_h dS q_h and dV = sum_h P dO_h
    over all (token, list position) pairs that read it (window overlap between a
    sequence's tokens, ids repeated in a top-k list, split tokens' units, head
    groups), against the oracle's float64 gradient over the same resolved rows."""
    c = build()
    print(f"\n[case] {name}: B={c.B} T={c.T} H={c.H} D={c.D} scen={c.scenario} K={c.K} "
          f"q={c.q_dtype} cores={cores}", flush=True)
    launch, out, lse = _launch(c, cores)
    g, g_np = _dout(c, seed=sum(name.encode()))
    dq, dsinks, d_ori, d_cmp = launch.backward(g.cuda(), kv_grad=True)
    torch.cuda.synchronize()
    dq_ex, ds_ex, dori_ex, dcmp_ex = _exact_grads(c, g_np, kv_grad=True)
    _check_grad(f"{name}:dq", dq.cpu().numpy(), dq_ex)
    _check_pools(name, c, d_ori, d_cmp, dori_ex, dcmp_ex)


def test_backward_kv_pools_with_padded_strides():
    """Pools with padded block and row strides: the gradient comes back laid out
    like the pool (its strides), and the padding is never written."""
    c = make_case(B=2, H=32, seq_kv=[5000, 1300], q_per_seq=2, scenario=3, K=512, seed=130)
    d = to_device(c)

    def padded(pool):
        nb, bs, _, D = pool.shape
        base = torch.zeros((nb, bs + 3, 1, D + 64), dtype=pool.dtype, device=pool.device)
        view = base[:, :bs, :, :D]
        view.copy_(pool)
        return view

    from dsv4_planb_amd.api import build_launch

    cu = d["cu_seqlens_q"]
    launch, out, lse = build_launch(
        q_flat=d["q"], ori_kv=padded(d["ori_kv"]), ori_block_table=d["ori_block_table"],
        cmp_kv=padded(d["cmp_kv"]), cmp_block_table=d["cmp_block_table"],
        cmp_indices=d["cmp_sparse_indices"], q_prefix=cu[:-1], act_q_lens=cu[1:] - cu[:-1],
        seqused_kv=d["seqused_kv"], sinks=d["sinks"], metadata=None, scenario=3, topk=c.K,
        cmp_ratio=4, ori_win_left=c.win_left, softmax_scale=c.softmax_scale, core_num=256)
    launch.run()
    g, g_np = _dout(c, seed=31)
    _, _, d_ori, d_cmp = launch.backward(g.cuda(), kv_grad=True)
    torch.cuda.synchronize()
    assert d_ori.stride() == launch.ori_kv.stride() and d_cmp.stride() == launch.cmp_kv.stride()
    # the padding of the strided layout (rows bs.. and dims D..) stays zero: every
    # element of the buffer outside the pool's view is 0
    for grad in (d_ori, d_cmp):
        n = grad.untyped_storage().nbytes() // 4
        flat = torch.as_strided(grad, (n,), (1,), 0).clone()
        offs = torch.as_strided(torch.arange(n, device=grad.device), grad.shape, grad.stride(), 0)
        flat[offs.reshape(-1)] = 0
        assert flat.abs().max().item() == 0
    _, _, dori_ex, dcmp_ex = _exact_grads(c, g_np, kv_grad=True)
    _check_pools("kv_strides", c, d_ori, d_cmp, dori_ex, dcmp_ex)


def test_autograd_reaches_the_kv_pools():
    """ori_kv / cmp_kv requiring grad: sum(out * w).backward() fills their .grad
    (pool dtype and shape) with the oracle's float64 gradient."""
    from dsv4_planb_amd import sparse_attn_sharedkv

    c = make_case(B=2, H=64, seq_kv=[5000, 1300], q_per_seq=2, scenario=3, K=512, seed=131)
    d = to_device(c)
    q = d.pop("q").detach().requires_grad_(True)
    ori = d.pop("ori_kv").detach().requires_grad_(True)
    cmpk = d.pop("cmp_kv").detach().requires_grad_(True)
    out = sparse_attn_sharedkv(q, ori_kv=ori, cmp_kv=cmpk, softmax_scale=c.softmax_scale,
                               cmp_ratio=4, topk_cmp=c.K, **d)
    g, g_np = _dout(c, seed=9)
    (out.float() * g.cuda().float()).sum().backward()
    torch.cuda.synchronize()
    assert ori.grad is not None and ori.grad.dtype == ori.dtype and ori.grad.shape == ori.shape
    assert cmpk.grad is not None and cmpk.grad.shape == cmpk.shape
    dq_ex, _, dori_ex, dcmp_ex = _exact_grads(c, g_np, kv_grad=True)
    _check_grad("autograd-kv:dq", q.grad.float().cpu().numpy(), dq_ex)
    # the bf16 .grad carries one more rounding of each summed row
    _check_grad("autograd-kv:d_ori_kv", ori.grad.float().squeeze(2).cpu().numpy(), dori_ex,
                fro_tol=6e-3, max_tol=1.2e-2)
    _check_grad("autograd-kv:d_cmp_kv", cmpk.grad.float().squeeze(2).cpu().numpy(), dcmp_ex,
                fro_tol=6e-3, max_tol=1.2e-2)


def test_backward_refuses_fp8():
    from dsv4_planb_amd import sparse_attn_sharedkv

    c8 = make_case(B=1, H=16, seq_kv=[900], q_per_seq=1, scenario=1, kv_dtype="fp8e4m3", seed=114)
    d8 = to_device(c8)
    q8 = d8.pop("q").requires_grad_(True)
    with pytest.raises(NotImplementedError):
        sparse_attn_sharedkv(q8, softmax_scale=c8.softmax_scale, **d8)
