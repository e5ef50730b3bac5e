""".binfer containers (CPU only): files written by ainfer_amd/binfer.py pass
the C validator (ainfer_binfer_open), and every rule of the reference's
loader (docs/binfer_spec.md:112-116, tools/binfer.py:383-499) rejects a file
that breaks it, with a message naming the failure.  The writer takes its
CRC-32 and SHA-256 from Python's binascii and hashlib, so a file the C side
accepts also pins its own CRC-32 and SHA-256 to those; the negatives show the
checks are live.  The reference's own negative-test file (two tensors,
tools/binfer.py:502-560) is rebuilt here and must be accepted as well."""
import ctypes as C
import struct
import json
from pathlib import Path

import numpy as np
import pytest

from ainfer_amd import binfer as B


@pytest.fixture(scope="module")
def L():
    from ainfer_amd import _lib
    return _lib


@pytest.fixture(scope="module")
def c0_layers(oracle):
    from ainfer_amd.synthetic import CONFIGS
    cfg = CONFIGS["c0"]
    out = []
    for l in range(2):
        a = dict(oracle.HostLayer.synthetic(cfg, layer=l).a)
        a["norm_w"] = (oracle.f32_to_bf16((np.arange(cfg.hidden) % 7 * 0.1 + 0.5)
                                          .astype(np.float32)))
        out.append(a)
    c = dict(hidden=cfg.hidden, n_experts=cfg.n_experts, top_k=cfg.top_k, inter=cfg.inter,
             shared_inter=cfg.shared_inter)
    return c, out


def _open(L, path):
    h = C.c_void_p()
    err = C.create_string_buffer(512)
    rc = L.lib().ainfer_binfer_open(str(path).encode(), C.byref(h), err, len(err))
    if rc == L.OK:
        L.lib().ainfer_binfer_close(h)
    return rc, err.value.decode()


def test_valid_moe_file_and_info(L, tmp_path, c0_layers):
    cfg, layers = c0_layers
    p = tmp_path / "m.binfer"
    B.write_moe(p, cfg, layers)
    rc, err = _open(L, p)
    assert rc == L.OK, err
    bf = L.BinferFile(p)
    s, n, eps = bf.moe_info()
    assert (s.hidden, s.n_experts, s.top_k, s.inter, s.shared_inter) == (
        cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["inter"], cfg["shared_inter"])
    assert s.scale_dtype == L.SCALE_FP16 and n == 2 and abs(eps - 1e-6) < 1e-12
    # the arena holds every tensor of the layer, each 256-byte aligned
    want = sum((len(t.payload) + 255) // 256 * 256 + ((len(t.scales) + 255) // 256 * 256 if t.scales else 0)
               for t in B.moe_layer_tensors(1, cfg, layers[1]))
    assert bf.layer_bytes(1) == want
    bf.close()


def test_reference_negative_test_file_is_valid(L, tmp_path):
    """The reference's tiny file: a.weight INT4 [256] and b.weight BF16 [256]."""
    ts = [B.Tensor("a.weight", [256], B.DT["INT4_SYM_G128"], bytes(128), b"\x01\x02" * 2),
          B.Tensor("b.weight", [256], B.DT["BF16"], bytes(512))]
    sections = [{"source_repo": "t", "source_revision": "0" * 40}, {"arch": "t"},
                {"format": "x"}, {"default": "y"}]
    p = tmp_path / "tiny.binfer"
    p.write_bytes(B.serialize(ts, sections))
    rc, err = _open(L, p)
    assert rc == L.OK, err


def _tiny(tmp_path, name, **kw):
    ts = [B.Tensor("a.weight", [256], B.DT["INT4_SYM_G128"], bytes(range(128)), b"\x01\x02" * 2),
          B.Tensor("b.weight", [256], B.DT["BF16"], bytes(range(256)) * 2),
          B.Tensor("c.weight", [2, 2, 128], B.DT["INT4_SYM_G128"], bytes(256), b"\x03\x04" * 4,
                   B.LAYOUT_EXPERTS)]
    sections = [{"source_repo": "t", "source_revision": "0" * 40}, {"arch": "t"},
                {"format": "x"}, {"default": "y"}]
    p = tmp_path / (name + ".binfer")
    p.write_bytes(B.serialize(ts, sections, **kw))
    return p, ts


def _set(fmt, off, val):
    def f(i, e):
        if i == 0 or fmt.startswith("all"):
            struct.pack_into(fmt.replace("all", ""), e, off, val)
    return f


CASES = {
    # name: (serialize kwargs, post-write byte mutation, expected message part)
    "bad_magic": (dict(mutate=lambda b: b.__setitem__(0, 0xFF)), None, "bad magic"),
    "bad_version": (dict(mutate=lambda b: struct.pack_into("<I", b, 8, 999)), None, "bad version"),
    "reserved_flags": (dict(mutate=lambda b: struct.pack_into("<I", b, 12, 3)), None,
                       "reserved flags"),
    "bad_alignment": (dict(mutate=lambda b: struct.pack_into("<I", b, 36, 32)), None,
                      "alignment"),
    "total_mismatch": (dict(), lambda d: d + b"\x00", "total mismatch"),
    "truncated": (dict(), lambda d: d[:len(d) // 2], "total mismatch"),
    "section_crc": (dict(mutate=lambda b: b.__setitem__(b.index(b'{"arch"') + 3, 0x41)), None,
                    "section 2 CRC"),
    "dir_crc": (dict(mutate=lambda b: b.__setitem__(
        struct.unpack_from("<Q", b, 128 + 4 * 32 + 4)[0] + 1, 0x41)), None, "dir) CRC"),
    "payload_crc": (dict(mutate=lambda b: b.__setitem__(
        struct.unpack_from("<Q", b, struct.unpack_from("<Q", b, 128 + 4 * 32 + 4)[0] + 160)[0],
        0x7F)), None, "payload CRC a.weight"),
    "unknown_layout": (dict(mutate_entry=_set("<H", 138, 7)), None, "unknown layout_id 7"),
    "layout32_not_3d": (dict(mutate_entry=_set("<H", 138, B.LAYOUT_EXPERTS)), None,
                        "layout_id 32 needs"),
    "visual_tensor": (dict(mutate_entry=lambda i, e: e.__setitem__(
        slice(0, 20), b"m.visual.w\x00".ljust(20, b"\x00")) if i == 1 else None), None,
        "visual tensor present"),
    "duplicate_name": (dict(mutate_entry=lambda i, e: e.__setitem__(
        slice(0, 9), b"a.weight\x00") if i == 1 else None), None, "duplicate name a.weight"),
    "unsupported_dtype": (dict(mutate_entry=lambda i, e: e.__setitem__(137, 9) if i == 1 else None),
                          None, "unsupported dtype"),
    "bad_quant_params": (dict(mutate_entry=_set("<Q", 152, 6)), None, "bad quant params a.weight"),
    "bad_packed_size": (dict(mutate_entry=_set("<Q", 168, 64)), None, "bad packed size a.weight"),
    "bad_scale_dtype": (dict(mutate_entry=lambda i, e: e.__setitem__(180, 5) if i == 0 else None),
                        None, "unknown scale dtype"),
    "overlap": (dict(mutate_entry=lambda i, e: struct.pack_into(
        "<Q", e, 160, struct.unpack_from("<Q", e, 160)[0] - 64) if i == 1 else None), None,
        "overlap"),
    "out_of_range": (dict(mutate_entry=lambda i, e: struct.pack_into("<Q", e, 160, 1 << 40)
                          if i == 1 else None), None, "span out of range"),
    "unaligned_payload": (dict(mutate_entry=lambda i, e: struct.pack_into(
        "<Q", e, 160, struct.unpack_from("<Q", e, 160)[0] + 8) if i == 1 else None), None,
        "not 64-byte aligned"),
    "sha_mismatch": (dict(fix_sha=False), None, "trailing sha256"),
    "dir_size": (dict(mutate=lambda b: struct.pack_into("<Q", b, 16, 4)), None, "dir size"),
    # 3 + 2**58 entries: the count times 192 wraps to the real 576-byte directory
    "dir_count_overflow": (dict(mutate=lambda b: struct.pack_into("<Q", b, 16, 3 + (1 << 58))),
                           None, "dir size"),
    # three dims of 2**32: the element count overflows 64 bits (it would wrap to 0)
    "numel_overflow": (dict(mutate_entry=lambda i, e: (e.__setitem__(64, 3), struct.pack_into(
        "<QQQ", e, 72, 1 << 32, 1 << 32, 1 << 32)) if i == 1 else None), None,
        "b.weight: implausible shape"),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_validator_rejects(L, tmp_path, case):
    kw, post, msg = CASES[case]
    p, _ = _tiny(tmp_path, case, **kw)
    if post:
        p.write_bytes(post(p.read_bytes()))
    rc, err = _open(L, p)
    assert rc == L.ERR_FORMAT, (case, rc, err)
    assert msg in err, (case, err)


def test_valid_tiny_and_missing_file(L, tmp_path):
    p, _ = _tiny(tmp_path, "ok")
    rc, err = _open(L, p)
    assert rc == L.OK, err
    rc, err = _open(L, tmp_path / "absent.binfer")
    assert rc == L.ERR_IO and "cannot open" in err


def test_sha256_and_crc32_agree_with_python(L, tmp_path):
    """Files whose payloads and sections take every byte value: the C CRC-32
    and SHA-256 accept exactly what binascii and hashlib wrote, over lengths
    that cross SHA block boundaries (55, 56, 64 and 1 MiB + 1 bytes)."""
    for n in (1, 55, 56, 63, 64, 65, 1000, (1 << 20) + 1):
        data = bytes((i * 131 + 7) & 0xFF for i in range(n))
        pad = (-n) % 2
        ts = [B.Tensor("x.weight", [(n + pad) // 2], B.DT["BF16"], data + b"\x00" * pad)]
        p = tmp_path / f"s{n}.binfer"
        p.write_bytes(B.serialize(ts, [{"a": n}, {"b": 1}, {"c": 2}, {"d": 3}]))
        rc, err = _open(L, p)
        assert rc == L.OK, (n, err)


def test_load_checks_layer_shape(L, tmp_path, c0_layers):
    """The loader checks a layer's tensors against the architecture section:
    a file whose router is [E][H/2] is rejected when the layer is loaded."""
    import ainfer_amd._lib as LL
    cfg, layers = c0_layers
    bad = dict(layers[0])
    bad["router_w"] = bad["router_w"][: bad["router_w"].size // 2]
    tensors = B.moe_layer_tensors(0, cfg, bad)
    tensors[0].shape = [cfg["n_experts"], cfg["hidden"] // 2]
    p = tmp_path / "badshape.binfer"
    p.write_bytes(B.serialize(tensors, B.moe_sections(cfg, 1)))
    bf = LL.BinferFile(p)
    w = LL.Weights()
    nw = C.c_void_p()
    # no device memory is touched before the shape check fails
    rc = LL.lib().ainfer_binfer_load_moe_layer(bf.h, 0, C.c_void_p(256), 1 << 30, C.byref(w),
                                               C.byref(nw), None)
    assert rc == LL.ERR_FORMAT
    assert "mlp.gate.weight" in LL.lib().ainfer_binfer_error(bf.h).decode()
    assert LL.lib().ainfer_binfer_load_moe_layer(bf.h, 5, C.c_void_p(256), 1 << 30, C.byref(w),
                                                 C.byref(nw), None) == LL.ERR_ARG
    bf.close()


GOLDEN = Path(__file__).resolve().parent / "golden" / "binfer"


def test_reference_validator_verdicts(L):
    """Files the reference's own negatives command emitted, and files this
    writer made, with the reference validator's verdict on each
    (tests/golden/make_binfer_fixtures.py): ainfer_binfer_open accepts
    exactly what the reference accepts.  The one difference is deliberate:
    layout_id 32 (expert-stacked tensors) is this format's extension, which
    the v1 reference rejects as an unsupported layout."""
    verdicts = json.loads((GOLDEN / "verdicts.json").read_text())
    assert len(verdicts) == 8
    for name, v in sorted(verdicts.items()):
        rc, err = _open(L, GOLDEN / name)
        if name == "ours_layout32.binfer":
            assert v["rc"] == 1 and v["errors"] == ["unsupported layout_id"]
            assert rc == L.OK, (name, err)
            continue
        assert (rc == L.OK) == (v["rc"] == 0), (name, rc, err, v)
        if v["rc"] != 0:
            assert rc == L.ERR_FORMAT
            # same first failure where the reference reports a single one
            if len(v["errors"]) == 1:
                assert v["errors"][0] in err, (name, err, v["errors"])
