"""CPU oracle for the MTP speculative-decoding verify step. TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import this package, and only as the
checker (or the timed CPU baseline), never as part of the product path: the HIP library under
`qwen38-27b-aws_amd/` never calls into it and fails loudly when its own extension is missing.

`oracle.model` restates the reference's CPU path (qwen38_inf2/model.py, generate.py, scheduler.py) in torch CPU ops
at the same rounding points, with this build's weight format (FP8 e4m3 + E8M0 per 32) in place of the reference's
e5m2 bytes. `oracle.scheduler` restates the speculative step the reference's `Scheduler` runs (`_mtp_drafts`,
`_verify_step`, scheduler.py:160-193, 269-301), its input builders (generate.py:25-107) and the run loop's prefill
and verify parts, with graph adapters over `oracle.model`. Pinning (which check fixes each function) is listed in each
module's header and each function's docstring; a function with no such check says "parity unpinned".
"""
