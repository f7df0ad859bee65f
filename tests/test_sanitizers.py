"""AddressSanitizer + UndefinedBehaviorSanitizer over the host code: the
oracle and the engine's C++ (the .rinn parser, config parsing, Layer /
Inference plumbing and the C-ABI's argument checks) are rebuilt with
-fsanitize=address,undefined (g++ / gcc only, no HIP sources), and the CPU
tests that drive them (.rinn format and error paths, the oracle pins, the
ABI export checks) run again in a subprocess that loads those builds.  Any
out-of-bounds access, use after free or undefined behaviour aborts the
subprocess."""
import importlib.util
import os
import subprocess
import sys

from conftest import PKG_DIR, ROOT

TESTS = ["tests/test_rinn.py", "tests/test_oracle_formats.py", "tests/test_oracle_math.py",
         "tests/test_oracle_mla.py", "tests/test_oracle_jamba.py", "tests/test_abi.py"]

PROBE = """
import sys
sys.path.insert(0, %r)
sys.path.insert(0, %r)
import conftest, oracle
conftest.load_pkg().load_engine()
oracle.load()
maps = open("/proc/self/maps").read()
print("engine:", %r in maps, "oracle:", %r in maps, "asan:", "libasan" in maps)
"""


def test_host_code_under_asan_ubsan():
    spec = importlib.util.spec_from_file_location("rina_amd_build", os.path.join(PKG_DIR, "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    eng_so, orc_so = b.build_sanitized()
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], stdout=subprocess.PIPE, text=True,
                             check=True).stdout.strip()
    env = dict(os.environ)
    # the sanitizer runtime goes first; anything the environment already
    # preloads stays after it
    env["LD_PRELOAD"] = libasan + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["RINA_ENGINE_SO"] = eng_so
    env["RINA_ORACLE_SO"] = orc_so
    probe = subprocess.run([sys.executable, "-c", PROBE % (ROOT, os.path.join(ROOT, "tests"), eng_so, orc_so)],
                           cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert probe.returncode == 0 and "engine: True oracle: True asan: True" in probe.stdout, probe.stdout
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu"] + TESTS,
                       cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=900)
    tail = "\n".join(r.stdout.splitlines()[-30:])
    assert r.returncode == 0, tail
    assert "passed" in tail and "ERROR: AddressSanitizer" not in r.stdout and "runtime error" not in r.stdout, tail
