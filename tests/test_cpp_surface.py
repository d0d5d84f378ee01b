"""The C++ host surface (include/uocr.hpp) compiled by a C++ caller against the
library, run on the CPU (tests/cpp/host_surface.cpp)."""
import os
import shutil
import struct
import subprocess

import pytest

import model_files as mf
import uocr_moe as um

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_cpp_host_surface(tmp_path):
    fx = tmp_path / "fixture"
    fx.mkdir()
    source = fx / "source.safetensors"
    mf.write(source, {"lm_head.weight": ("F32", [1, 2], struct.pack("<2f", 1.0, -2.0))})
    h = mf.sha256(source)
    data = mf.write(fx / "q.safetensors",
                    {"lm_head.weight": ("I8", [1, 2], bytes([1, 254])),
                     "lm_head.weight.q8_scales": ("F32", [1, 1], struct.pack("<f", 1.0))},
                    {"format": mf.FORMAT, "block_size": "32", "source_sha256": h})
    mf.write_manifest(fx / "q.safetensors", h, data, 1)
    model = tmp_path / "model"
    model.mkdir()
    mf.model_dir(model)
    mf.overlay(model / "model-00001-of-000001.safetensors", model / "overlay.safetensors")
    libdir = os.path.dirname(um.LIB_PATH)
    exe = tmp_path / "host_surface"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    os.path.join(REPO, "tests", "cpp", "host_surface.cpp"),
                    "-I", os.path.join(REPO, "include"), "-L", libdir, "-luocr_moe",
                    f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    run = subprocess.run([str(exe), str(fx), str(model), h], capture_output=True, text=True)
    print(run.stdout)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "0 failures" in run.stdout
