"""The C-ABI library loads, exports every symbol include/ainfer_moe.h
declares, and rejects bad arguments before touching the GPU.  CPU only: no
call here reaches a kernel."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def L():
    from ainfer_amd import _lib
    return _lib


def declared_symbols():
    txt = (ROOT / "include" / "ainfer_moe.h").read_text()
    return sorted(set(re.findall(r"\b(ainfer_(?:moe|binfer)_\w+)\s*\(", txt)))


def test_exports_every_declared_symbol(L):
    lib = L.lib()
    decl = declared_symbols()
    assert set(decl) == set(L.EXPORTS)
    for name in decl:
        assert hasattr(lib, name), name


def shape(L, **kw):
    d = dict(hidden=2048, n_experts=512, top_k=10, inter=512, shared_inter=512, group=128,
             scale_dtype=L.SCALE_FP16, precision=0)
    d.update(kw)
    return L.Shape(**d)


def test_validate(L):
    lib = L.lib()
    assert lib.ainfer_moe_validate(C.byref(shape(L))) == L.OK
    for bad in (dict(group=64), dict(hidden=1000), dict(top_k=0), dict(top_k=600),
                dict(n_experts=2048), dict(inter=100), dict(shared_inter=-128),
                dict(scale_dtype=7), dict(precision=2), dict(precision=-1), dict(hidden=16384)):
        assert lib.ainfer_moe_validate(C.byref(shape(L, **bad))) == L.ERR_SHAPE, bad
    assert lib.ainfer_moe_validate(None) == L.ERR_NULL


def test_workspace_bytes(L):
    lib = L.lib()
    s = shape(L)
    b1 = lib.ainfer_moe_workspace_bytes(C.byref(s), 1)
    b16 = lib.ainfer_moe_workspace_bytes(C.byref(s), 16)
    b4096 = lib.ainfer_moe_workspace_bytes(C.byref(s), 4096)
    assert 0 < b1 < b16 < b4096
    assert lib.ainfer_moe_workspace_bytes(C.byref(s), -1) == 0
    assert lib.ainfer_moe_workspace_bytes(C.byref(s), L.MAX_TOKENS + 1) == 0
    assert lib.ainfer_moe_workspace_bytes(C.byref(shape(L, group=32)), 4) == 0


def test_forward_rejects_bad_arguments_without_gpu(L):
    lib = L.lib()
    s = shape(L)
    w = L.Weights()
    # weights missing -> ERR_NULL, bad T -> ERR_TOKENS, bad shape first
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), None, None, 1, None, 0, None) == L.ERR_NULL
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), None, None, -1, None, 0, None) == L.ERR_TOKENS
    assert lib.ainfer_moe_forward(C.byref(shape(L, top_k=0)), C.byref(w), None, None, 1, None, 0,
                                  None) == L.ERR_SHAPE
    fake = C.c_void_p(0x1000)
    w = L.Weights(*([fake] * len(L.Weights._fields_)))
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), None, None, 1, None, 0, None) == L.ERR_NULL
    # misaligned / small workspace
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), fake, fake, 1, C.c_void_p(0x1010), 1 << 40,
                                  None) == L.ERR_WORKSPACE
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), fake, fake, 1, C.c_void_p(0x1000), 16,
                                  None) == L.ERR_WORKSPACE
    # T == 0 is a no-op
    assert lib.ainfer_moe_forward(C.byref(s), C.byref(w), None, None, 0, None, 0, None) == L.OK
    assert lib.ainfer_moe_block_forward(C.byref(s), C.byref(w), None, 5, 1e-6, fake, fake, 1, fake,
                                        1 << 40, None) == L.ERR_ARG
    assert lib.ainfer_moe_fill(9, 0, 1.0, 10, fake, None) == L.ERR_ARG
    assert lib.ainfer_moe_rmsnorm(fake, None, 0, 1e-6, fake, 1, 7, None) == L.ERR_SHAPE
    assert L.lib().ainfer_moe_strerror(L.ERR_WORKSPACE).startswith(b"workspace")


def test_stage_entries_reject_bad_arguments_without_gpu(L):
    lib = L.lib()
    s = shape(L)
    fake = C.c_void_p(0x1000)
    w = L.Weights(*([fake] * len(L.Weights._fields_)))
    # experts: one chunk at most, W4A16 only, 16-byte aligned x and o, a real workspace
    assert lib.ainfer_moe_experts(C.byref(s), C.byref(w), fake, fake, 4097, fake, fake, 1 << 40,
                                  None) == L.ERR_TOKENS
    assert lib.ainfer_moe_experts(C.byref(s), C.byref(w), None, fake, 1, fake, fake, 1 << 40,
                                  None) == L.ERR_NULL
    assert lib.ainfer_moe_experts(C.byref(s), C.byref(w), fake, fake, 1, C.c_void_p(0x1008), fake,
                                  1 << 40, None) == L.ERR_ARG
    assert lib.ainfer_moe_experts(C.byref(s), C.byref(w), fake, fake, 1, fake, fake, 16,
                                  None) == L.ERR_WORKSPACE
    s8 = shape(L)
    s8.precision = L.PRECISION_W4A8
    assert lib.ainfer_moe_experts(C.byref(s8), C.byref(w), fake, fake, 1, fake, fake, 1 << 40,
                                  None) == L.ERR_ARG
    assert lib.ainfer_moe_experts(C.byref(s), C.byref(w), None, None, 0, None, None, 0, None) == L.OK
    # combine: the shared gate is required with a shared expert; aligned rows
    assert lib.ainfer_moe_combine(C.byref(s), fake, fake, None, None, fake, 1, None) == L.ERR_NULL
    assert lib.ainfer_moe_combine(C.byref(s), fake, fake, fake, C.c_void_p(0x1004), fake, 1,
                                  None) == L.ERR_ARG
    assert lib.ainfer_moe_combine(C.byref(s), fake, fake, fake, None, fake, -1, None) == L.ERR_TOKENS
    assert lib.ainfer_moe_combine(C.byref(shape(L, top_k=0)), fake, fake, fake, None, fake, 1,
                                  None) == L.ERR_SHAPE



def test_mfma_probe_rejects_bad_arguments_without_gpu(L):
    r = C.c_float()
    lib = L.lib()
    for args in ((5, 1, 10), (-1, 1, 10), (0, 0, 10), (0, 5, 10), (0, 1, 0), (0, 1, 1 << 21)):
        assert lib.ainfer_moe_mfma_probe(*args, None, C.byref(r)) == L.ERR_ARG, args
    assert lib.ainfer_moe_mfma_probe(0, 1, 10, None, None) == L.ERR_ARG


def test_missing_library_fails_loudly(L, monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(L.MoeError):
        L.lib()
