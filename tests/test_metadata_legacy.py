"""The reference scheduler table (int32[1024]) from ``sas_metadata_legacy``.

Pinned two ways: bit-exact against tables the reference scheduler itself wrote
(``tests/golden/metadata_tables.json``, made by
``tests/golden/make_metadata_fixtures.py``), and by the reference's own
invariant tests (``test_sparse_attn_sharedkv.py:767-970``): continuity of the
per-core ranges, exactly-once coverage of every (b, s) and a full core fan-out
for the 8K prefill.  CPU only.
"""

from __future__ import annotations

import json
import os

import pytest
import torch

from dsv4_planb_amd import metadata as M

FIX = os.path.join(os.path.dirname(__file__), "golden", "metadata_tables.json")
CASES = json.load(open(FIX))["cases"]


def _call(args):
    kw = dict(args)
    for k in ("cu_seqlens_q", "seqused_kv", "seqused_q"):
        if k in kw:
            kw[k] = torch.tensor(kw[k], dtype=torch.int32)
    return M.sparse_attn_sharedkv_metadata(**kw)


@pytest.mark.parametrize("case", CASES, ids=[f"{c['name']}-{c['args'].get('aic_core_num')}" for c in CASES])
def test_matches_reference_tables(case):
    if "error" in case:
        with pytest.raises(Exception):
            _call(case["args"])
        return
    got = _call(case["args"])
    assert got.dtype == torch.int32 and got.shape == (M.SAS_META_SIZE,)
    want = torch.zeros(M.SAS_META_SIZE, dtype=torch.int32)
    for i, v in case["nonzero"]:
        want[i] = v
    diff = (got != want).nonzero().flatten().tolist()
    assert not diff, f"{len(diff)} entries differ, first {[(i, int(got[i]), int(want[i])) for i in diff[:8]]}"


# ---------------------------------------------------------------------------
# The reference's own invariants (test_sparse_attn_sharedkv.py:767-970), run on
# the table sas_metadata_legacy produces for every fixture argument set.
# ---------------------------------------------------------------------------
AIC, FA_W = 36, 8
OK_CASES = [c for c in CASES if "error" not in c and c["args"].get("aic_core_num", 24) <= AIC]


def _q_lens(args):
    B = args["batch_size"]
    if args.get("seqused_q"):
        return [int(x) for x in args["seqused_q"]]
    if args["layout_q"] == "TND":
        cu = args["cu_seqlens_q"]
        return [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    return [args["max_seqlen_q"]] * B


def _fa_rows(args):
    md = _call(args)
    return md[: AIC * FA_W].view(AIC, FA_W).tolist()


@pytest.mark.parametrize("case", OK_CASES, ids=[f"{c['name']}-{c['args'].get('aic_core_num')}" for c in OK_CASES])
def test_enabled_cores_form_a_contiguous_chain(case):
    """Each enabled core resumes at its predecessor's end cursor
    (test_sparse_attn_sharedkv.py:767-834)."""
    args = case["args"]
    rows = [r for r in _fa_rows(args) if r[0] == 1]
    assert rows, "at least one core must be enabled"
    prev = (0, 0, 0)
    for r in rows:
        assert (r[1], r[2], r[3]) == prev, f"core resumes at {(r[1], r[2], r[3])}, previous end {prev}"
        prev = (r[4], r[5], r[6])
    B = len(_q_lens(args))
    assert prev[0] in (B * args["num_heads_kv"], 0)


@pytest.mark.parametrize("case", OK_CASES, ids=[f"{c['name']}-{c['args'].get('aic_core_num')}" for c in OK_CASES])
def test_core_windows_cover_every_token_exactly_once(case):
    """Simulate the reference kernel's outer loop over each core's
    [bn2_start * max_seq + m_start, bn2_end * max_seq + m_end) window with its
    s < act_q guard: every valid (b, s) is visited exactly once
    (test_sparse_attn_sharedkv.py:837-943)."""
    args = case["args"]
    if args["num_heads_kv"] != 1:
        pytest.skip("the kernel walk below is the reference's N2=1 form")
    act = _q_lens(args)
    B = len(act)
    max_seq = max(act) if args["layout_q"] == "TND" else args["max_seqlen_q"]
    if max_seq == 0:
        pytest.skip("no query rows")
    seen, dup = set(), []
    for cid, r in enumerate(_fa_rows(args)):
        if r[0] != 1:
            continue
        for pid in range(r[1] * max_seq + r[2], r[4] * max_seq + r[5]):
            b, s = divmod(pid, max_seq)
            if b < B and s < act[b]:
                if (b, s) in seen:
                    dup.append((cid, b, s))
                seen.add((b, s))
    want = {(b, s) for b in range(B) for s in range(act[b])}
    assert not dup, f"overlapping windows: {dup[:5]}"
    assert seen == want, f"missing {sorted(want - seen)[:5]}, stray {sorted(seen - want)[:5]}"


def test_prefill_uses_every_core():
    """The 8192-token prefill spreads over all 24 cores
    (test_sparse_attn_sharedkv.py:946-970)."""
    case = next(c for c in CASES if c["name"] == "scfa_prefill" and c["args"]["aic_core_num"] == 24)
    rows = _fa_rows(case["args"])
    assert sum(r[0] for r in rows) == 24
