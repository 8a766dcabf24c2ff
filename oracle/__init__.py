"""oracle — CPU restatement of the reference's matmul hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the
checker (or, for cpu_baseline, as the timed reference CPU path).  The
product path (scaffolding_amd) never imports it.

Contents
  quant.py     bfloat16 / float16 round-to-nearest-even quantizers (NumPy bit
               arithmetic), the storage convention of the device path.
  cpu_path.py  the reference's Linux CPU path restated in NumPy (fp32), plus
               fp64 closed forms on the quantized inputs.
  configs.py   seeded generators for BASELINE.json's five configs, their
               algorithmic FLOP / byte counts and the tolerance functions.

Pinning (each function's checks live in tests/test_oracle.py):
  * quantizers: IEEE known answers (ties-to-even, NaN/Inf/-0, overflow,
    subnormals) and agreement with NumPy's own float16 cast;
  * matmul / linear: pure-Python triple loops on ragged tiny shapes and the
    committed golden fixtures in tests/golden/;
  * silu / gelu_tanh: closed-form special values and the identities
    silu(x) = x/2 (1 + tanh(x/2)) and gelu(x) - gelu(-x) = x;
  * softmax / sdpa: rows sum to 1, shift invariance, a known answer
    softmax([0, ln 2]) = [1/3, 2/3], uniform weights for equal scores;
  * tolerances: BASELINE.json's north_star formulas at tabulated sizes.
"""
