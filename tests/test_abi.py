"""The C-ABI library loads and exports every entry point include/gq.h declares
(no compute: this runs without a GPU)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gq.h")
LIB = os.path.join(ROOT, "agention-infer_amd", "libgq.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    for n in ("gq_init", "gq_upload", "gq_matvec", "gq_gemm", "gq_matmul_dequant_host",
              "gq_dequant_rows", "gq_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


def test_ctypes_signatures_cover_header():
    import gq
    assert sorted(gq.SIGNATURES) == declared()
    L = gq.lib()
    for n in declared():
        assert hasattr(L, n)


def test_host_only_calls():
    import gq
    L = gq.lib()
    assert L.gq_backend_name() == b"hip"
    assert L.gq_type_size(12, 3584) == 2016
    assert L.gq_type_size(14, 18944) == 15540
    assert L.gq_type_size(8, 33) == 68
    assert L.gq_type_size(18, 3072) == 1176
    assert L.gq_type_size(999, 256) == 0


def test_no_device_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import gq
    with pytest.raises(gq.GqError):
        gq.create_backend("hip")
    with pytest.raises(gq.GqError):
        gq.create_backend("cpu")  # no CPU arm inside libgq: never a silent fallback


HOST_HEADER = os.path.join(ROOT, "include", "gq_host.h")
HOST_LIB = os.path.join(ROOT, "agention-infer_amd", "libgq_host.so")


def declared_host():
    text = open(HOST_HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(gqh_[a-z0-9_]+)\s*\(", text)))


def test_host_library_exports_every_declared_symbol():
    assert os.path.exists(HOST_LIB), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", HOST_LIB], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    names = declared_host()
    assert "gqh_gguf_open" in names and "gqh_gguf_upload" in names
    missing = [n for n in names if n not in exported]
    assert not missing, missing


def test_host_ctypes_signatures_cover_header():
    import gq
    assert sorted(gq.HOST_SIGNATURES) == declared_host()
    L = gq.host_lib()
    for n in declared_host():
        assert hasattr(L, n)
