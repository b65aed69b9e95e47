"""Oracle for the sparse shared-KV attention path -- TEST INFRASTRUCTURE ONLY.

Everything under ``oracle/`` checks the product and is never part of it:

* ``golden_ref``   -- numpy restatement of the reference golden model
  (``sparse_attn_sharedkv_tilelang/golden.py``): index resolution, paging,
  the 512-row tiled online softmax with the sink seed, the one-shot closed form,
  and the float64 gradient of the one-shot sink softmax (``golden_backward_f64``).
* ``sas_golden.c`` -- the same algorithm in C (OpenMP over tokens), used for
  larger parity cases and as the CPU baseline in ``bench.py``; loaded through
  ``golden_c``.

The scheduler table (``sparse_attn_sharedkv_tilelang/metadata.py``) has no
restatement here: its tolerance-greedy cursor walk has no closed form, so the
product's table is compared with tables the reference's own scheduler wrote,
stored as fixtures under ``tests/golden/``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package.  The product package (``dsv4_planb_amd``) never does.

Pinning (what checks each function against something other than itself):

* ``resolve_cmp_ids`` / ``window_positions`` / ``paged_row`` -- brute-force
  special cases (thr=0, -1 terminator, skip >= thr, K > thr) and the
  closed-form page map checked against a dense unpack, ``tests/test_oracle.py``.
* ``round_bf16`` / ``round_fp16`` -- against torch's conversions on every
  rounding-tie pattern, ``tests/test_oracle.py``.
* ``golden_attention`` -- the reference's own known-answer test (chunked online
  softmax == one-shot softmax with the sink), redone in float64; reduction
  cases (sink=-inf -> plain softmax, single key, no key -> 0 / lse=sink,
  SWA == banded causal mask attention); planted-mistake tests show that a
  dropped sink, a wrong window edge, a skipped -1 terminator or a dropped or
  truncating P rounding fail them.
* ``golden_c`` -- agrees with ``golden_attention`` on shared cases; its exact
  mode equals the float64 one-shot closed form.
* ``golden_backward_f64`` and its C twin -- central finite
  differences of the float64 forward, ``tests/test_oracle_backward.py``.
"""
