"""Oracle for the sparse shared-KV attention path -- TEST INFRASTRUCTURE ONLY.

Everything under ``oracle/`` checks the product and is never part of it:

* ``golden_ref``   -- numpy restatement of the reference golden model
  (``sparse_attn_sharedkv_tilelang/golden.py``): index resolution, paging,
  the 512-row tiled online softmax with the sink seed, the one-shot closed form.
* ``sas_golden.c`` -- the same algorithm in C (OpenMP over tokens), used for
  larger parity cases and as the CPU baseline in ``bench.py``; loaded through
  ``golden_c``.
* ``metadata_ref`` -- restatement of the reference scheduler
  (``sparse_attn_sharedkv_tilelang/metadata.py``) emitting the int32[1024]
  table.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package.  The product package (``dsv4_planb_amd``) never does.

Pinning (what checks each function against something other than itself):

* ``resolve_cmp_ids`` / ``window_positions`` / ``paged_row`` -- brute-force
  special cases (thr=0, -1 terminator, skip >= thr, K > thr) and the
  closed-form page map checked against a dense unpack, ``tests/test_oracle.py``.
* ``golden_attention`` -- the reference's own known-answer test (chunked online
  softmax == one-shot softmax with the sink), redone in float64; reduction
  cases (sink=-inf -> plain softmax, single key, no key -> 0 / lse=sink,
  SWA == banded causal mask attention); planted-mistake tests show that a
  dropped sink, a wrong window edge or a skipped -1 terminator fail them.
* ``golden_c`` -- agrees with ``golden_attention`` on shared cases.
* ``metadata_ref`` -- the int32[1024] tables of the real reference scheduler,
  stored as fixtures under ``tests/golden/`` (written in the build container by
  ``tests/golden/make_metadata_fixtures.py``), plus the reference's continuity
  and coverage invariants.
"""
