"""Builds and runs tests/cpp/test_gguf.cpp (the host GGUF C++ API) on the CPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_gguf_cpp_api(tmp_path):
    exe = tmp_path / "test_gguf"
    src = [os.path.join(ROOT, "tests", "cpp", "test_gguf.cpp"),
           os.path.join(ROOT, "agention-infer_amd", "host", "gguf.cpp")]
    r = subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Wextra", "-Werror", *src, "-o",
                        str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, cwd=tmp_path, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
