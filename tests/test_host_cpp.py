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


def test_model_config_cpp(tmp_path):
    """ModelConfig::from_gguf and the host-side F32/F16 dequant (links libgq,
    makes no GPU call)."""
    pkg = os.path.join(ROOT, "agention-infer_amd")
    assert os.path.exists(os.path.join(pkg, "libgq.so")), "run __graft_entry__.build() first"
    exe = tmp_path / "test_model_config"
    src = [os.path.join(ROOT, "tests", "cpp", "test_model_config.cpp")] + \
        [os.path.join(pkg, "host", f) for f in ("gguf.cpp", "model.cpp", "hip_backend.cpp")]
    r = subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Wextra", "-Werror", *src,
                        f"-L{pkg}", "-lgq", f"-Wl,-rpath,{pkg}", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
