"""CPU oracle for the fused GDN decode path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (`lightdelta_amd/`) imports this package.  Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, always to check
results or as the timed CPU baseline, never as the thing measured on the GPU.

Modules and what pins each one (details in each module's header):
  gdn       fp32 Torch restatement of the reference's unfused post-conv GDN
            (python/lightdelta/reference/gdn.py:70-128).  Pinned by golden vectors written by
            the reference itself (tests/golden/), the closed-form scalar recurrence of
            tests/test_gdn.py:47-55, an fp64 per-element brute force (`brute`), and the
            delta-rule invariants (decay=1/beta=0 identity, beta=1 projection, q=e1 column).
  brute     fp64 per-element loops of the same math, for tiny shapes (pins `gdn`).
  decode    the slot-indexed op semantics of lightdelta::decode / GDNBackend
            (csrc/gdn_decode.cu:142-168,303-316; backend.py:30-91) on top of `gdn`.
            Pinned by the reference's own edge-case tests restated as tests (padding slot,
            invalid accepted, ragged cu, discarded candidates) and by equality with a packed
            restatement of backend.py's gather / compute / index_copy_ path.
  state_io  numpy gather / scatter / slot copy (csrc/state_io.cu:11-27).  Pinned by brute
            force element loops on tiny pools and by the reference test's fixed expectations
            (tests/test_gdn.py:125-143).
"""
