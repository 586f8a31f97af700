"""The library's host code (GGUF reader, weight repacks, host encoders) and the CPU
oracle under AddressSanitizer + UndefinedBehaviorSanitizer: tests/sanitize/harness.cpp
opens a valid GGUF file and 4000 mutated copies of it (bit flips, extreme length /
count / offset values, truncations, insertions), queries every tensor and key of each
file that opens and takes it through the weight repack; repacks random bytes of every
format and layout; runs the encoders on random, tiny, huge and non-finite values; and
runs the oracle's decoders, linears, MoE and sampling.  Any sanitizer report fails it."""
import os
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.mark.skipif(not os.path.exists("/opt/rocm/llvm/bin/clang++"), reason="needs ROCm's clang as host compiler")
def test_host_code_under_asan_ubsan(tmp_path):
    subprocess.run(["make", "-s", "-C", HERE], check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([os.path.join(HERE, "_build", "harness"), "4000", str(tmp_path)], capture_output=True, text=True,
                       timeout=300, env=env)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stderr[-4000:]
