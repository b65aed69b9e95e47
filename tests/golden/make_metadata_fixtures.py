"""Write int32[1024] scheduler tables of the reference as test fixtures.

The exact table of the reference scheduler (``sparse_attn_sharedkv_tilelang/
metadata.py``: a tolerance-greedy cursor walk) has no closed form, so its
values are pinned by running the reference function itself, in the build
container only, on the reference's own six test scenarios
(``test_sparse_attn_sharedkv.py:81-220``), on the benchmark configurations and
on seeded random argument sets.  The output, ``metadata_tables.json``, holds
the arguments and the non-zero entries of each table; nothing of the reference
is copied.  Run:  python tests/golden/make_metadata_fixtures.py
"""

from __future__ import annotations

import importlib.util
import json
import math
import os
import random
import sys

import torch

REF = "/root/reference/sparse_attn_sharedkv_tilelang/metadata.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "metadata_tables.json")


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_metadata", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # dataclasses look their module up here
    spec.loader.exec_module(mod)
    return mod


def reference_scenarios():
    """The six reference test cases (decode / prefill x SWA / CFA / SCFA, TND, B=1)."""
    base = dict(num_heads_q=64, num_heads_kv=1, head_dim=512, batch_size=1, layout_q="TND",
                ori_mask_mode=4, ori_win_left=127, ori_win_right=0)
    out = []
    for name, s1, kv, scen, ratio, k in [
        ("scfa_decode", 1, 8193, 3, 4, 512), ("scfa_prefill", 8192, 8192, 3, 4, 512),
        ("swa_decode", 1, 8193, 1, 4, 0), ("swa_prefill", 8192, 8192, 1, 4, 0),
        ("cfa_decode", 1, 8193, 2, 128, 512), ("cfa_prefill", 8192, 8192, 2, 128, 512),
    ]:
        kw = dict(base, cu_seqlens_q=[0, s1], seqused_kv=[kv], max_seqlen_q=s1, max_seqlen_kv=kv,
                  has_ori_kv=True, has_cmp_kv=scen >= 2)
        if scen >= 2:
            kw.update(cmp_ratio=ratio, cmp_mask_mode=3)
        if scen == 3:
            kw["cmp_topk"] = k
        out.append((name, kw))
    return out


def benchmark_configs():
    rng = random.Random(42)
    out = []
    common = dict(num_heads_kv=1, head_dim=576, layout_q="TND", ori_mask_mode=4, ori_win_left=127,
                  ori_win_right=0, cmp_mask_mode=3, cmp_ratio=4, has_ori_kv=True)
    # c1: SWA decode, B=2, H=16, seq 1024
    out.append(("c1", dict(common, num_heads_q=16, batch_size=2, cu_seqlens_q=[0, 1, 2],
                           seqused_kv=[1024, 1024], max_seqlen_q=1, max_seqlen_kv=1024,
                           has_cmp_kv=False)))
    # c2: B=32, H=64, seq U[4k, 32k], top-k 512
    kv = [rng.randint(4096, 32768) for _ in range(32)]
    out.append(("c2", dict(common, num_heads_q=64, batch_size=32, cu_seqlens_q=list(range(33)),
                           seqused_kv=kv, max_seqlen_q=1, max_seqlen_kv=max(kv), has_cmp_kv=True,
                           cmp_topk=512)))
    # c3: B=128, MTP 2, H=128, 128k, top-k 2048
    out.append(("c3", dict(common, num_heads_q=128, batch_size=128,
                           cu_seqlens_q=list(range(0, 257, 2)), seqused_kv=[131072] * 128,
                           max_seqlen_q=2, max_seqlen_kv=131072, has_cmp_kv=True, cmp_topk=2048)))
    # c4: prefill B=1, 8192 tokens, H=128, top-k 2048
    out.append(("c4", dict(common, num_heads_q=128, batch_size=1, cu_seqlens_q=[0, 8192],
                           seqused_kv=[8192], max_seqlen_q=8192, max_seqlen_kv=8192,
                           has_cmp_kv=True, cmp_topk=2048)))
    # c5: ragged B=64, seq log-uniform [256, 128k], q in {1, 2, 4}
    qn = [rng.choice([1, 2, 4]) for _ in range(64)]
    kvs = [int(math.exp(rng.uniform(math.log(256), math.log(131072)))) for _ in range(64)]
    cu = [0]
    for n in qn:
        cu.append(cu[-1] + n)
    out.append(("c5", dict(common, num_heads_q=128, batch_size=64, cu_seqlens_q=cu, seqused_kv=kvs,
                           max_seqlen_q=max(qn), max_seqlen_kv=max(kvs), has_cmp_kv=True,
                           cmp_topk=2048)))
    return out


def random_cases(n=40, seed=7):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        B = rng.randint(1, 9)
        layout = rng.choice(["TND", "BSND"])
        n1 = rng.choice([16, 64, 128])
        n2 = rng.choice([1, 1, 1, 2])
        scen = rng.choice([1, 2, 3])
        qn = [rng.choice([0, 1, 2, 4, 17, 300]) for _ in range(B)]
        kv = [rng.choice([0, 1, 5, 127, 128, 129, 1000, 4096, 20000]) for _ in range(B)]
        kw = dict(num_heads_q=n1, num_heads_kv=n2, head_dim=rng.choice([512, 576]), batch_size=B,
                  layout_q=layout, ori_mask_mode=rng.choice([4, 4, 4, 3, 0]),
                  ori_win_left=rng.choice([127, 127, 63, 0, -1]), ori_win_right=0,
                  seqused_kv=kv, max_seqlen_kv=max(kv), has_ori_kv=True, has_cmp_kv=scen >= 2,
                  aic_core_num=rng.choice([1, 3, 7, 24, 36]), aiv_core_num=rng.choice([2, 48, 72]))
        if layout == "TND":
            cu = [0]
            for x in qn:
                cu.append(cu[-1] + x)
            kw.update(cu_seqlens_q=cu, max_seqlen_q=max(max(qn), 1))
        else:
            kw.update(max_seqlen_q=max(max(qn), 1))
            if rng.random() < 0.3:
                kw["seqused_q"] = qn
        if scen >= 2:
            kw.update(cmp_ratio=rng.choice([1, 4, 128]), cmp_mask_mode=3)
        if scen == 3:
            kw["cmp_topk"] = rng.choice([1, 128, 512, 2048])
        out.append((f"rand{i}", kw))
    return out


def main():
    ref = load_reference()
    cases = []
    groups = [(n, kw, core) for n, kw in reference_scenarios() for core in (24, 36)]
    groups += [(n, kw, core) for n, kw in benchmark_configs() for core in (24, 36)]
    groups += [(n, kw, None) for n, kw in random_cases()]
    for name, kw, core in groups:
        call = dict(kw)
        if core is not None:
            call["aic_core_num"] = core
            call["aiv_core_num"] = 2 * core
        tensor_args = {k: torch.tensor(v, dtype=torch.int32)
                       for k, v in call.items() if k in ("cu_seqlens_q", "seqused_kv", "seqused_q")}
        args = {k: v for k, v in call.items() if k not in tensor_args}
        try:
            table = ref.sparse_attn_sharedkv_metadata(**args, **tensor_args)
            res = {"nonzero": [[i, int(v)] for i, v in enumerate(table.tolist()) if v != 0]}
        except Exception as exc:  # noqa: BLE001 -- record that the reference rejects it
            res = {"error": type(exc).__name__}
        cases.append({"name": name, "args": call, **res})
        print(name, call.get("aic_core_num"), "error" if "error" in res else len(res["nonzero"]))
    with open(OUT, "w") as f:
        json.dump({"source": "reference sparse_attn_sharedkv_metadata (metadata.py:1018-1086)",
                   "cases": cases}, f, separators=(",", ":"))
    print("wrote", OUT, len(cases), "cases")


if __name__ == "__main__":
    main()
