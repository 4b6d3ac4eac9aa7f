"""The C-ABI layer (argument validation, workspace planning, error strings)
under AddressSanitizer, on the CPU: capi.hip's host code built with
-fsanitize=address (make -C flaggems-sglang_amd/csrc asan) and linked with
the ordinary kernel objects, then the C-ABI tests of test_capi.py run
against that library in a child process with the sanitizer runtime
preloaded. Any invalid read or write in the host paths those tests drive --
every entry point called with bad arguments, the workspace-size queries,
the schedule query, the thread-local error string -- aborts the child."""

import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "flaggems-sglang_amd", "csrc")
ASAN_LIB = os.path.join(CSRC, "_build", "libfgs_moe_asan.so")


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def _child_env(rt):
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt
    # the interpreter and the HIP runtime are not instrumented: leaks at exit
    # are theirs, and the runtime need not come first in the link order
    env["ASAN_OPTIONS"] = "detect_leaks=0:verify_asan_link_order=0:halt_on_error=1"
    env["FGS_MOE_LIB"] = ASAN_LIB
    return env


@pytest.fixture(scope="module")
def asan_setup():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("no AddressSanitizer runtime under /opt/rocm/llvm")
    r = subprocess.run(["make", "-C", CSRC, "-j8", "asan"], capture_output=True, text=True)
    if r.returncode != 0 or not os.path.exists(ASAN_LIB):
        pytest.fail("ASan build failed:\n" + r.stdout[-2000:] + r.stderr[-2000:])
    return rt


def test_asan_library_is_the_one_loaded(asan_setup):
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "from flaggems_sglang import _capi\n"
        "_capi.load()\n"
        "maps = open('/proc/self/maps').read()\n"
        "assert %r in maps, 'ASan library not mapped'\n"
        "assert 'libclang_rt.asan' in maps, 'sanitizer runtime not mapped'\n"
        "print('ok')\n" % (ROOT, os.path.join(ROOT, "flaggems-sglang_amd"), ASAN_LIB))
    r = subprocess.run([sys.executable, "-c", code], env=_child_env(asan_setup),
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_capi_validation_under_asan(asan_setup):
    r = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
         os.path.join(ROOT, "tests", "test_capi.py")],
        cwd=ROOT, env=_child_env(asan_setup), capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
