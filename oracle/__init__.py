"""CPU oracle for the SSPA packed-KV decode path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline), never as the thing measured
or shipped.  The product path (``r2-omni_amd/r2omni_amd``) never imports it.

Modules:
  quant      numpy restatement of the reference quantisers and packers (bit-exact).
  cache      numpy restatement of the three-pool cache builder and append/flush.
  attention  torch-CPU fp32 restatement of ``triton_mixed_reference`` + output FWHT.

How each function is pinned (closed forms, invariants, golden fixtures written by the
reference's own CPU path) is listed in each module's header.  No function here is
"parity unpinned".
"""
