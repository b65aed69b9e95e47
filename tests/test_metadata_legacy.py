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
