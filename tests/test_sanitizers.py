"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer.

Builds the host-sanitized variant of libvoxhip.so (device code unchanged) and runs
the GGUF parser and C-ABI tests against it in a child process with the ASan
runtime preloaded: well-formed, truncated, bad-magic and overflowing files must
parse or fail with an error code without a single sanitizer report.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def _stale(lib: Path) -> bool:
    if not lib.exists():
        return True
    t = lib.stat().st_mtime
    srcs = list((ROOT / "voxgen_amd" / "csrc").iterdir()) + [ROOT / "include" / "voxhip.h"]
    return any(p.stat().st_mtime > t for p in srcs)


def test_gguf_and_abi_tests_are_clean_under_asan_and_ubsan():
    from voxgen_amd import build
    lib = build.ASAN_DIR / "libvoxhip.so"
    if _stale(lib):
        build.build_voxhip(sanitize=True)
    runtime = build.asan_runtime()
    if not Path(runtime).exists():
        pytest.skip(f"no ASan runtime at {runtime}")
    env = dict(os.environ)
    env.update(LD_PRELOAD=runtime, VOXHIP_LIBRARY=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                           str(ROOT / "tests" / "test_gguf.py"), str(ROOT / "tests" / "test_abi.py")],
                          cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=600)
    out = proc.stdout
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
