"""CPU oracle of the paged-attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the reference that GPU results are
compared with (or the timed CPU baseline): the product path
(llm-inference-runtime_amd/pagedattn) never imports it and fails loudly
when libpagedattn.so is missing.

The reference's arithmetic lives in flashinfer-python 0.6.11.post3
(pyproject.toml:13, uv.lock:526-547), which is not vendored and is CUDA-only,
so this package restates the semantics that the reference's call sites
(src/models/llama.py:70-245) and metadata builders
(src/engine/runtime/step_executor.py:98-165, 204-243) fix, in fp32/fp64 torch
for floating point and numpy for integer/byte work.  Each function cites the
call site it follows; tests/test_oracle.py pins every function against
closed forms, brute force, invariants and transformers' RoPE (see the
"pinned by" line of each docstring).
"""

from .paged_ref import *  # noqa: F401,F403
