"""CPU oracle for the tiered decode-attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in `lazykv_amd/` imports, calls or links anything here: the
product path runs the HIP kernels and fails loudly when they are missing. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use this package, and only
as the reference results are compared against (or, for `cpu_path`, as the timed CPU baseline).

Modules:

* `oracle.reference`  -- numpy restatement of the reference's hot-path functions
  (`lazykv/selection.py`, `attention.py`, `exact.py`, `quant.py`, `tiered.py`), each function
  citing the reference file:line it follows. Float work is in float64 where it serves as the
  truth; the int8 quantiser is restated bit-for-bit in float32.
* `oracle.quant_c`    -- ctypes wrapper of `quant_ref.c`, an independent C restatement of the
  int8 pack/unpack with its own float16/bfloat16 rounding; cross-checks the numpy restatement.
* `oracle.cpu_path`   -- the reference's CPU decode path in torch CPU ops, in the reference's
  order (bound, topk, gather, explicit attention with LSE, merge), timed as the CPU baseline.

How each function is pinned (golden vectors, known answers from the reference's tests, closed
forms, brute force) is stated in each module's header.
"""
