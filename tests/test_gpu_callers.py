"""The reference's own caller flows, on the GPU.

* ``_get_kernel(**19 parameters)`` -> ``func(11 tensors)`` captured in a
  framework graph and replayed (test_graph_mode.py:107-209): here
  ``torch.cuda.CUDAGraph``, replays bit-equal to the eager call and the eager
  call within tolerance of the oracle.  Scenario 1 passes the reference's dummy
  compressed tensors (test_graph_mode.py:124-128).
* The metadata op's int32[1024] table at the reference's 24 cores fed to the API
  (test_sparse_attn_sharedkv.py:530-629).
* The ``return_softmax_lse`` branch contract (test_sparse_attn_sharedkv.py:654-761).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.cases import make_case
from tests.gpu_helpers import assert_parity, to_device

pytestmark = pytest.mark.gpu


def _ref_metadata(c, d, scenario):
    """The reference flow's metadata call (test_sparse_attn_sharedkv.py:566-595)."""
    from dsv4_planb_amd import sparse_attn_sharedkv_metadata

    kw = dict(num_heads_q=c.H, num_heads_kv=1, head_dim=c.D, cu_seqlens_q=d["cu_seqlens_q"],
              cu_seqlens_ori_kv=None, cu_seqlens_cmp_kv=None, seqused_q=None,
              seqused_kv=d["seqused_kv"], batch_size=c.B, max_seqlen_q=int(c.act_q.max()),
              max_seqlen_kv=int(c.seqused_kv.max()), ori_mask_mode=4, ori_win_left=c.win_left,
              ori_win_right=0, layout_q="TND", layout_kv="PA_ND", has_ori_kv=True,
              has_cmp_kv=scenario >= 2)
    if scenario >= 2:
        kw.update(cmp_ratio=c.cmp_ratio, cmp_mask_mode=3)
    if scenario == 3:
        kw["cmp_topk"] = c.K
    md = sparse_attn_sharedkv_metadata(**kw)
    assert md.dtype == torch.int32 and md.numel() == 1024
    return md


@pytest.mark.parametrize("scenario", [1, 3])
def test_get_kernel_func_replayed_from_torch_cuda_graph(scenario):
    from dsv4_planb_amd.api import DEFAULT_BLOCK_I, DEFAULT_CORE_NUM, _get_kernel

    c = make_case(B=4, H=64, seq_kv=[5000, 1300, 9000, 300], q_per_seq=[1, 2, 1, 3],
                  scenario=scenario, K=512 if scenario == 3 else 0, seed=51 + scenario)
    print(f"\n[case] _get_kernel + CUDAGraph: scenario={scenario} B={c.B} T={c.T} H={c.H}",
          flush=True)
    d = to_device(c)
    md = _ref_metadata(c, d, scenario).cuda()
    cu = d["cu_seqlens_q"].to(torch.int32)
    q_prefix = cu[:-1].contiguous()
    act_q = (cu[1:] - cu[:-1]).contiguous()
    if scenario == 3:
        cmp_kv, cmp_bt, cmp_idx = d["cmp_kv"], d["cmp_block_table"], d["cmp_sparse_indices"]
        cbn, cbs, ctl = cmp_kv.shape[0], cmp_kv.shape[1], cmp_bt.shape[1]
    else:  # the reference's dummies for SWA
        cmp_kv = torch.zeros((1, 1, 1, c.D), dtype=torch.bfloat16, device="cuda")
        cmp_bt = torch.zeros((c.B, 1), dtype=torch.int32, device="cuda")
        cmp_idx = torch.zeros((c.T, 1, DEFAULT_BLOCK_I), dtype=torch.int32, device="cuda")
        cbn = cbs = ctl = 1
    func = _get_kernel(
        batch=c.B, max_seq=int(c.act_q.max()), total_tokens=c.T,
        ori_block_num=d["ori_kv"].shape[0], ori_block_size=d["ori_kv"].shape[1],
        ori_table_len=d["ori_block_table"].shape[1], cmp_block_num=cbn, cmp_block_size=cbs,
        cmp_table_len=ctl, n_heads=c.H, n_kv_heads=1, head_dim=c.D,
        topk_cmp=c.K if scenario == 3 else 0, cmp_ratio=c.cmp_ratio, scenario=scenario,
        ori_win_left=c.win_left, softmax_scale=float(c.softmax_scale), dtype="bfloat16",
        core_num=DEFAULT_CORE_NUM)
    assert func is _get_kernel(
        batch=c.B, max_seq=int(c.act_q.max()), total_tokens=c.T,
        ori_block_num=d["ori_kv"].shape[0], ori_block_size=d["ori_kv"].shape[1],
        ori_table_len=d["ori_block_table"].shape[1], cmp_block_num=cbn, cmp_block_size=cbs,
        cmp_table_len=ctl, n_heads=c.H, n_kv_heads=1, head_dim=c.D,
        topk_cmp=c.K if scenario == 3 else 0, cmp_ratio=c.cmp_ratio, scenario=scenario,
        ori_win_left=c.win_left, softmax_scale=float(c.softmax_scale), dtype="bfloat16",
        core_num=DEFAULT_CORE_NUM), "the kernel cache returns the same callable for the same key"
    args = [a.contiguous() for a in (d["q"], d["ori_kv"], d["ori_block_table"], cmp_kv, cmp_bt,
                                     cmp_idx, q_prefix, act_q, d["seqused_kv"], d["sinks"], md)]
    for _ in range(3):  # warmup before capture, as the reference harness does
        out_e, lse_e = func(*args)
    torch.cuda.synchronize()
    ref_out, ref_lse = out_e.clone(), lse_e.clone()
    oc, lc = c.oracle_c()
    ex, exl = c.oracle_exact()
    assert_parity(ref_out.float().cpu().numpy(), ref_lse.cpu().numpy(), oc, lc,
                  label=f"get_kernel-eager-s{scenario}", exact=(ex, exl))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g, lse_g = func(*args)
    try:
        for k in range(3):
            out_g.zero_()
            lse_g.fill_(float("nan"))
            junk = torch.randn(1 << 16, device="cuda").sum()  # eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, ref_out), f"replay {k}: output differs from the eager call"
            assert torch.equal(lse_g, ref_lse), f"replay {k}: lse differs from the eager call"
            del junk
        # new query values in the captured input: the replay follows them
        args[0].copy_(torch.flip(args[0], dims=[1]))
        out2, lse2 = func(*args)
        torch.cuda.synchronize()
        out2, lse2 = out2.clone(), lse2.clone()
        assert not torch.equal(out2, ref_out)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out2) and torch.equal(lse_g, lse2), "refreshed replay differs"
    finally:
        del g


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_metadata_table_from_24_cores_into_api(scenario):
    """The metadata op at the reference's default 24 cores returns the
    int32[1024] table; the API takes it (it partitions rows over Ascend cores,
    which changes no result) and gives the oracle's answer."""
    from dsv4_planb_amd import sparse_attn_sharedkv

    kw = dict(B=3, H=64, seq_kv=[5000, 700, 9000], q_per_seq=[1, 2, 3], scenario=scenario,
              seed=60 + scenario)
    if scenario == 2:
        kw.update(cmp_ratio=128, block_size=128, cmp_block_size=128, K=0)
    elif scenario == 3:
        kw["K"] = 512
    c = make_case(**kw)
    print(f"\n[case] metadata(24) -> api: scenario={scenario} T={c.T}", flush=True)
    d = to_device(c)
    md = _ref_metadata(c, d, scenario)
    q = d.pop("q")
    out, lse = sparse_attn_sharedkv(
        q, metadata=md.cuda(), softmax_scale=c.softmax_scale,
        cmp_ratio=c.cmp_ratio if scenario >= 2 else None, ori_mask_mode=4, cmp_mask_mode=3,
        ori_win_left=c.win_left, ori_win_right=0, layout_q="TND", layout_kv="PA_ND",
        return_softmax_lse=True, topk_cmp=c.K if scenario == 3 else 0, **d)
    torch.cuda.synchronize()
    oc, lc = c.oracle_c()
    ex, exl = c.oracle_exact()
    assert_parity(out.float().cpu().numpy(), lse.cpu().numpy(), oc, lc,
                  label=f"metadata24-s{scenario}", exact=(ex, exl))


@pytest.mark.parametrize("layout", ["TND", "BSND"])
def test_return_softmax_lse_branches(layout):
    """``return_softmax_lse=False`` returns one tensor of q's dtype shaped like q
    with d_v columns; ``True`` returns ``(out, lse)`` with an fp32 lse of q's
    leading dims; both branches give the same output (reference
    test_sparse_attn_sharedkv.py:654-761, on its swa_decode case: D=512, H=64,
    page 128)."""
    from dsv4_planb_amd import sparse_attn_sharedkv

    c = make_case(B=2, H=64, D=512, seq_kv=[8193, 3000], q_per_seq=2, scenario=1, K=0,
                  block_size=128, seed=70, softmax_scale=0.04419417)
    print(f"\n[case] return_softmax_lse branches: layout={layout}", flush=True)
    d = to_device(c)
    q = d.pop("q")
    md = _ref_metadata(c, dict(d, q=q), 1).cuda()
    if layout == "BSND":
        q = q.reshape(c.B, 2, c.H, c.D)
    kw = dict(d, metadata=md, softmax_scale=c.softmax_scale, ori_mask_mode=4, cmp_mask_mode=3,
              ori_win_left=127, ori_win_right=0, layout_q=layout, layout_kv="PA_ND", topk_cmp=0)
    one = sparse_attn_sharedkv(q, return_softmax_lse=False, **kw)
    two = sparse_attn_sharedkv(q, return_softmax_lse=True, **kw)
    torch.cuda.synchronize()
    lead = (c.T,) if layout == "TND" else (c.B, 2)
    assert isinstance(one, torch.Tensor)
    assert tuple(one.shape) == lead + (c.H, 512) and one.dtype == torch.bfloat16
    assert isinstance(two, tuple) and len(two) == 2
    out, lse = two
    assert isinstance(out, torch.Tensor) and isinstance(lse, torch.Tensor)
    assert tuple(out.shape) == lead + (c.H, 512) and out.dtype == torch.bfloat16
    assert tuple(lse.shape) == lead + (c.H,) and lse.dtype == torch.float32
    assert torch.equal(out, one)
    oc, lc = c.oracle_c()
    assert_parity(out.reshape(c.T, c.H, 512).float().cpu().numpy(),
                  lse.reshape(c.T, c.H).cpu().numpy(), oc, lc, label=f"lse-branches-{layout}")
