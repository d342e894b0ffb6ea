"""The library's host code -- the token-range matcher (token_matcher.hip),
the DMA run planner of the store path (cbk_memcpy_runs_commands,
host_slab.hip) and the error helpers -- built with sanitizers on the host pass
only, and driven through its C ABI by tests/native/matcher_sanitize.cpp:
seeded register / re-register / unregister / match sequences against a
brute-force model of the reference's matcher (cacheblend_vllm/matcher.py:53-126),
with exactly sized token and output buffers, planted hash collisions,
too-small capacities, four threads matching while a fifth registers and
unregisters, and random run tables for the planner.

- AddressSanitizer + UndefinedBehaviorSanitizer: out-of-bounds reads of the
  prompt or a record, writes past the caller's output arrays, use after free
  in unregister / re-register, leaks at destroy, and undefined integer or
  pointer arithmetic all end the run with a report.
- ThreadSanitizer: data races between concurrent match and register calls.

No GPU is touched; the device pass is built without instrumentation."""

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "pic-kvcache_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"

SANITIZERS = {
    "address_undefined": ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                          "-Xarch_host", "-fno-sanitize-recover=all"],
    "thread": ["-Xarch_host", "-fsanitize=thread"],
}


@pytest.mark.parametrize("name", sorted(SANITIZERS))
def test_matcher_host_code_under_sanitizer(tmp_path, name):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc is not installed")
    exe = tmp_path / f"matcher_{name}"
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           *SANITIZERS[name], f"-I{ROOT / 'include'}", f"-I{CSRC}",
           str(CSRC / "token_matcher.hip"), str(CSRC / "errors.hip"), str(CSRC / "host_slab.hip"),
           str(ROOT / "tests" / "native" / "matcher_sanitize.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1", TSAN_OPTIONS="halt_on_error=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-6000:])
    assert "Sanitizer" not in run.stderr, run.stderr[-6000:]
    last = run.stdout.strip().splitlines()[-1]
    assert last.startswith("ok: "), run.stdout[-2000:]
    found = int(last.split()[1])
    assert found > 10_000, last  # the sequences exercise matching, not only misses
