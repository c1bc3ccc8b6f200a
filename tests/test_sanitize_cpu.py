"""The host C-ABI layer under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

The reference runs its tests under compute-sanitizer memcheck / synccheck
(tests/test_sanitizer.py:53-75). No device sanitizer is available on this stack,
so what is sanitized here is the host layer every call goes through: argument
validation, recipe and layout checks, descriptor handling and error reporting
(deepgemm-amd_amd/csrc/dg_api.cpp), rebuilt with -fsanitize=address,undefined and
loaded in place of the regular library (DG_LIBRARY) with the ASan runtime
preloaded. The CPU tests of the C ABI, the Python shim and the oracle then run in a
child process; any sanitizer report aborts it."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, 'tests', 'sanitize', 'build_asan.sh')


def test_cpu_abi_tests_under_asan_and_ubsan(tmp_path):
    if not glob.glob(os.path.join(ROOT, 'deepgemm-amd_amd', '_build', '*.hip.o')):
        pytest.skip('the library objects are not built (run __graft_entry__.build())')
    if not os.path.exists(SCRIPT):
        pytest.skip('sanitizer build recipe not present')
    b = subprocess.run(['bash', SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stderr[-3000:]
    runtime = b.stdout.strip().splitlines()[-1]
    lib = str(tmp_path / 'libdeepgemm_mi355x_asan.so')
    # the host layer is instrumented (it calls into the ASan runtime)
    nm = subprocess.run(['nm', '-D', '--undefined-only', lib], capture_output=True, text=True)
    assert '__asan_report' in nm.stdout and '__ubsan_handle' in nm.stdout
    env = dict(os.environ, DG_LIBRARY=lib, LD_PRELOAD=runtime,
               ASAN_OPTIONS='detect_leaks=0:halt_on_error=1:abort_on_error=1',
               UBSAN_OPTIONS='halt_on_error=1:print_stacktrace=1',
               PYTHONPATH=os.pathsep.join([os.path.join(ROOT, 'deepgemm-amd_amd'), ROOT]))
    # the child loads the sanitized library, with the runtime mapped
    probe = subprocess.run([sys.executable, '-c',
                            'from deep_gemm import _ffi; m = open("/proc/self/maps").read(); '
                            'print(_ffi.LIB_PATH, "libclang_rt.asan" in m, "libdeepgemm_mi355x_asan" in m)'],
                           env=env, capture_output=True, text=True, timeout=300)
    assert probe.returncode == 0, probe.stderr[-3000:]
    assert probe.stdout.split() == [lib, 'True', 'True'], probe.stdout
    run = subprocess.run([sys.executable, '-m', 'pytest', '-q', '-x', '-p', 'no:cacheprovider',
                          'tests/test_abi_cpu.py', 'tests/test_shim_cpu.py', 'tests/test_oracle.py'],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    print(run.stdout[-600:])
    assert run.returncode == 0, (run.stdout[-3000:], run.stderr[-3000:])
    assert 'AddressSanitizer' not in run.stderr and 'runtime error' not in run.stderr
