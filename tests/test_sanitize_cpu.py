"""The host planners (decode_plan.cpp, prefill_plan.cpp, plan.cpp: the
metadata validation and partitioning behind BatchDecode/BatchPrefill
plan(), src/models/llama.py:86-147) built with AddressSanitizer and
UndefinedBehaviorSanitizer and driven with randomized and malformed metadata
(tests/sanitize/plan_fuzz.cpp).  Bad metadata must come back as an error
status, which the Python layer raises (the reference's callers fail the batch,
process_loop.py:129-132), never as undefined behaviour.  CPU only: without a
GPU the planners run up to the work-list upload."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None,
                    reason="needs hipcc and make")
def test_planners_under_sanitizers():
    subprocess.run(["make", "-C", HERE, f"HIPCC={HIPCC}"], check=True, capture_output=True,
                   timeout=600)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    for seed in (1, 2, 3):
        r = subprocess.run([os.path.join(HERE, "plan_fuzz"), "3000", str(seed)], env=env,
                           capture_output=True, text=True, timeout=600)
        report = r.stdout[-2000:] + r.stderr[-6000:]
        assert r.returncode == 0, report
        assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, report
        assert "0 failures" in r.stdout, report
