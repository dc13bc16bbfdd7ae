"""The C-ABI library loads, exports every function include/kq_gemv.h declares,
and its host logic follows the reference's error convention (no GPU needed:
nothing here launches a kernel)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import stratum_amd as K

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "kq_gemv.h")
GGUF_HEADER = os.path.join(ROOT, "include", "kq_gguf.h")


def declared_in(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kq_[a-z0-9_]+)\s*\(", text)))


def declared_functions():
    return sorted(set(declared_in(HEADER)) | set(declared_in(GGUF_HEADER)))


def test_header_and_python_export_list_agree():
    assert declared_in(HEADER) == sorted(K.EXPORTS)
    assert declared_in(GGUF_HEADER) == sorted(K.GGUF_EXPORTS)


def test_library_exports_every_declared_symbol():
    L = K.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", K.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(kq_[a-z0-9_]+)\b", out))
    assert set(declared_functions()) <= exported


def test_header_compiles_as_c_and_struct_matches_ggufensor():
    """kq_tensor is layout-compatible with GgufTensor (stratum_gguf.h:129-137):
    name@0, n_dims@8, dims@16, type@80, offset@88, nelem@96, nbytes@104."""
    src = r"""
#include "kq_gemv.h"
#include <stddef.h>
#include <stdio.h>
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(kq_tensor),
         offsetof(kq_tensor, name), offsetof(kq_tensor, n_dims), offsetof(kq_tensor, dims),
         offsetof(kq_tensor, type), offsetof(kq_tensor, offset), offsetof(kq_tensor, nelem),
         offsetof(kq_tensor, nbytes));
  return 0;
}
"""
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        c = os.path.join(td, "t.c")
        exe = os.path.join(td, "t")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                        c, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True,
                                               check=True).stdout.split()]
    assert vals == [112, 0, 8, 16, 80, 88, 96, 104]
    assert ctypes.sizeof(K.KqTensor) == 112


def test_row_bytes_and_type_table():
    L = K.lib()
    assert L.kq_row_bytes(12, 5120) == 20 * 144
    assert L.kq_row_bytes(14, 17408) == 68 * 210
    assert L.kq_row_bytes(10, 5120) == 20 * 84
    assert L.kq_row_bytes(42, 5120) == 20 * 148
    # every type of st_linear_dispatch's switch (stratum_linear.h:533-541):
    # GGUF row bytes (stratum_gguf.h:57-79)
    assert L.kq_row_bytes(8, 1024) == 32 * 34       # Q8_0
    assert L.kq_row_bytes(11, 5120) == 20 * 110     # Q3_K
    assert L.kq_row_bytes(13, 5120) == 20 * 176     # Q5_K
    assert L.kq_row_bytes(1, 2048) == 2048 * 2      # F16
    assert L.kq_row_bytes(0, 2048) == 2048 * 4      # F32
    for t in (2, 3, 6, 7, 9, 15, 16, 43, 44):        # no kernel -> -1
        assert L.kq_row_bytes(t, 1024) == -1, t
    assert L.kq_row_bytes(12, 1000) == -1     # K % 256 != 0


def test_errors_return_minus_one_with_message():
    """Unsupported type / bad shape return -1 and set kq_last_error, the
    reference's convention (stratum_linear.h:553-556); never exit()."""
    L = K.lib()
    x = np.zeros(1024, np.float32)
    y = np.zeros(16, np.float32)
    t = K.make_tensor(12, 16, 1024, 0)
    t.type = 7        # Q5_1: in GGUF's table, no kernel here or in the reference switch
    rc = L.kq_linear_dispatch(ctypes.byref(t), K._fptr(x), K._fptr(y), 16, 1024)
    assert rc == -1
    assert b"type" in L.kq_last_error()
    t.type = 12
    rc = L.kq_linear_dispatch(ctypes.byref(t), K._fptr(x), K._fptr(y), 16, 1000)
    assert rc == -1
    rc = L.kq_gemv_dev(99, None, None, None, None, 16, 1024, None)
    assert rc == -1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(K, "_LIB", None)
    monkeypatch.setattr(K, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError):
        K.lib()
