"""The host tests again, in a child process whose library is the sanitizer build (make sanitized:
the C++ host mirror under AddressSanitizer and UndefinedBehaviorSanitizer, any report aborting the
process): GGUF parsing and its rejections, the synthetic writers, batch planning, finish and the
GGUF directory checks."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_LIB = os.path.join(ROOT, "gemma-embed-swift_amd", "_build", "libgemmaembed_san.so")


def gcc_runtime(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], check=True, capture_output=True, text=True).stdout.strip()


def test_host_tests_under_address_and_ub_sanitizers():
    assert os.path.exists(SAN_LIB), f"{SAN_LIB} is not built (make -C gemma-embed-swift_amd sanitized)"
    env = dict(os.environ)
    # gcc's ASan runtime must be the first library of the process; libstdc++ is preloaded with it
    # so the runtime finds the C++ exception entry points it wraps (the interpreter does not link them)
    env["LD_PRELOAD"] = f"{gcc_runtime('libasan.so')} {gcc_runtime('libstdc++.so')}"
    env["ASAN_OPTIONS"] = "detect_leaks=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    env["GE_LIBRARY"] = SAN_LIB
    probe = ("import gemma_embed as ge; maps = open('/proc/self/maps').read(); "
             "assert 'libgemmaembed_san.so' in maps and 'libasan' in maps, 'sanitizer build not loaded'; "
             "print(ge.LIB_PATH)")
    r = subprocess.run([sys.executable, "-c", probe], cwd=os.path.join(ROOT, "gemma-embed-swift_amd"), env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == SAN_LIB
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-s", "-p", "no:cacheprovider", "-m", "not gpu",
                        "tests/test_host.py", "tests/test_gguf_directory.py", "tests/test_abi.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout + r.stderr)[-6000:]
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-6000:]
