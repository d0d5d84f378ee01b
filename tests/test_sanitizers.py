"""AddressSanitizer + UndefinedBehaviorSanitizer over the CPU code: the oracle
(oracle/uocr_oracle.c) and the host loaders behind the C ABI (csrc/host:
safetensors checkpoints, the INT8 overlay, model configs, JSON, SHA-256, the
C++ surface of include/uocr.hpp).

Both are rebuilt with gcc/g++ -fsanitize=address,undefined (no recovery)
into a temporary directory; the host library is linked with the device
entry points stubbed out (tests/cpp/gpu_abi_stub.cpp: they report
Unsupported). The existing oracle, loader and C++-surface test modules then
run against those builds in a child pytest with libasan (and libstdc++, for
exceptions thrown from the host library) preloaded. Any sanitizer report
fails the child run."""
import os
import shutil
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1", "-fPIC"]


def _runtime(name):
    out = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


needs_toolchain = pytest.mark.skipif(
    shutil.which("gcc") is None or shutil.which("g++") is None or _runtime("libasan.so") is None,
    reason="needs gcc/g++ with libasan")


def _child(tmp_path, env_extra, modules):
    env = dict(os.environ)
    env.update(env_extra)
    env["LD_PRELOAD"] = f"{_runtime('libasan.so')}:{_runtime('libstdc++.so.6')}"
    env["ASAN_OPTIONS"] = f"detect_leaks=0:log_path={tmp_path}/asan"
    env["UBSAN_OPTIONS"] = f"print_stacktrace=1:halt_on_error=1:log_path={tmp_path}/ubsan"
    run = subprocess.run([sys.executable, "-m", "pytest", "-p", "no:cacheprovider", "-q", "-x",
                          "-m", "not gpu"] + [os.path.join(REPO, "tests", m) for m in modules],
                         cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    reports = [p for p in os.listdir(tmp_path) if p.startswith(("asan", "ubsan"))]
    text = "".join(open(os.path.join(tmp_path, p)).read() for p in reports)
    assert not reports, text[:4000]
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert " passed" in run.stdout, run.stdout[-2000:]
    return run.stdout


@needs_toolchain
def test_oracle_under_asan_ubsan(tmp_path):
    lib = tmp_path / "liboracle.so"
    subprocess.run(["gcc", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", *SAN,
                    "-shared", "-o", str(lib), os.path.join(REPO, "oracle", "uocr_oracle.c"),
                    "-lm"], check=True)
    out = _child(tmp_path, {"UOCR_ORACLE_LIB": str(lib)},
                 ["test_oracle_kats.py", "test_oracle_moe.py"])
    print(out.strip().splitlines()[-1])


@needs_toolchain
def test_host_loaders_under_asan_ubsan(tmp_path):
    host = os.path.join(REPO, "unlimited-ocr-kernel_amd", "csrc", "host")
    srcs = sorted(os.path.join(host, f) for f in os.listdir(host) if f.endswith(".cpp"))
    lib = tmp_path / "libuocr_moe.so"
    subprocess.run(["g++", "-std=c++17", *SAN, "-I", os.path.join(REPO, "include"), "-shared",
                    "-o", str(lib), *srcs, os.path.join(REPO, "tests", "cpp", "gpu_abi_stub.cpp")],
                   check=True)
    out = _child(tmp_path, {"UOCR_MOE_LIB": str(lib)},
                 ["test_loaders.py", "test_cpp_surface.py"])
    print(out.strip().splitlines()[-1])
