"""The host code of the C ABI under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

The library is rebuilt with the host side instrumented (kdn.build.build_host_sanitized; -fsanitize behind
-Xarch_host, the device code as usual) and the host-path tests -- every argument check, workspace and
segment layout, error status and the slab pool's bookkeeping (tests/test_abi.py, tests/test_pool.py) --
run against it in a child process with the ASan runtime preloaded; any sanitizer report fails that
process (ASan aborts on the first error, UBSan's checks do not recover).
"""
import os
import subprocess
import sys

import pytest

from kdn import build as kbuild

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(900)
def test_host_paths_clean_under_asan_and_ubsan(tmp_path):
    runtime = kbuild.asan_runtime()
    if not runtime or not os.path.exists(kbuild.hipcc()):
        pytest.skip("hipcc's ASan runtime is not installed")
    lib = kbuild.build_host_sanitized(str(tmp_path / "hostsan"))
    undefined = subprocess.run(["nm", "-D", "--undefined-only", lib], capture_output=True, text=True, check=True).stdout
    assert "__asan_report" in undefined and "__ubsan_handle" in undefined  # the host code is instrumented
    env = dict(os.environ)
    env.update(KDN_LIBRARY=lib, LD_PRELOAD=runtime,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=87")
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                          os.path.join(REPO, "tests", "test_abi.py"), os.path.join(REPO, "tests", "test_pool.py")],
                         cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    report = res.stdout[-3000:] + res.stderr[-3000:]
    assert res.returncode == 0, report
    assert "ERROR: AddressSanitizer" not in report and "runtime error" not in report, report
    assert res.stdout.count(".") >= 15 and "F" not in res.stdout.split("[")[0], report
