"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer: the safetensors,
.p12 and auxiliary readers, the .p12 packer, the tokenizer and its stream, the document plan
and the C ABI's argument checks (everything the no-GPU tests reach through the library, and
the seeded mutations of every file format in tests/test_host_fuzz.py) run in a child
process against lib/libplamo_hip_asan.so (`make asan`: host units built with
-fsanitize=address,undefined, device objects unchanged), with the sanitizer runtime
preloaded.  Any report fails the child.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "plamo3-0.8b-runtime_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.slow


def _runtime():
    out = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(not (os.path.exists(HIPCC) and shutil.which("make")), reason="needs hipcc and make")
def test_host_code_is_clean_under_asan():
    runtime = _runtime()
    if runtime is None:
        pytest.skip("no AddressSanitizer runtime beside hipcc")
    build = subprocess.run(["make", "-C", PKG, "-j8", "asan"], capture_output=True, text=True)
    assert build.returncode == 0, build.stdout[-2000:] + build.stderr[-2000:]
    env = dict(os.environ, LD_PRELOAD=runtime, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               PYTHONPATH=os.pathsep.join([ROOT, PKG]))
    code = ("import sys, pytest\n"
            "from plamo_hip import native\n"
            "native.LIB_PATH = native.ASAN_LIB_PATH\n"
            "lib = native.load()\n"
            "assert any(native.ASAN_LIB_PATH in l for l in open('/proc/self/maps'))\n"
            "sys.exit(pytest.main(['-q', '-x', '-p', 'no:cacheprovider', '-m', 'not gpu',\n"
            "                      'tests/test_native_cpu.py', 'tests/test_tokenizer.py',\n"
            "                      'tests/test_ordered.py', 'tests/test_cli.py', 'tests/test_host_fuzz.py']))\n")
    run = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=900)
    tail = run.stdout[-3000:] + run.stderr[-3000:]
    assert run.returncode == 0, tail
    assert "AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr, tail
    print("  " + run.stdout.strip().splitlines()[-1])
