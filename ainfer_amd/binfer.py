"""Writer of `.binfer` containers holding INT4 mixture-of-experts layers.

The container is the reference's v1 format (docs/binfer_spec.md): a 128-byte
header, a section table (32-byte entries: id, offset, bytes, crc32), sections
1-4 (identity, architecture, tokenizer, quantization policy) as a u64 length
and a compact JSON body with the CRC over both, section 5 the tensor
directory (raw 192-byte entries, CRC over the raw bytes), a scale pool, 64-byte
aligned payloads and a trailing SHA-256 of every byte before it -- the layout
tools/binfer.py writes and validates (:383-499, :502-622).  What this writer
adds uses fields v1 reserves: expert tensors [E][rows][K] in layout_id 32
(E stacked row-major matrices, the weight layout of include/ainfer_moe.h) and
the scale dtype of an INT4 tensor in byte 180 of its entry (1 = fp16).

The C reader (ainfer_binfer_open) validates these files and loads layers into
device memory; this module only writes them.
"""
import binascii
import hashlib
import json
import struct

import numpy as np

MAGIC = b"BINFER\x00\x01"
VERSION = 1
ALIGN = 64
GROUP = 128
DT = {"BF16": 0, "FP16": 1, "FP32": 2, "INT4_SYM_G128": 3, "INT8": 4, "FP8_E4M3": 5}
LAYOUT_ROW_MAJOR = 0
LAYOUT_EXPERTS = 32


def align_up(n, a=ALIGN):
    return (n + a - 1) // a * a


def _blob(obj):
    return json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()


class Tensor:
    """One directory entry: name, logical shape, storage dtype, layout and
    the payload (and scale) bytes as stored."""

    def __init__(self, name, shape, storage, payload, scales=b"", layout=LAYOUT_ROW_MAJOR,
                 scale_fp16=False, logical=None):
        self.name = name
        self.shape = list(shape)
        self.storage = storage
        self.logical = DT["BF16"] if logical is None else logical
        self.layout = layout
        self.payload = bytes(payload)
        self.scales = bytes(scales)
        self.group = GROUP if storage == DT["INT4_SYM_G128"] else 0
        self.scale_dtype = 1 if (scale_fp16 and storage == DT["INT4_SYM_G128"]) else 0
        # filled in by serialize()
        self.d_off = self.sc_off = 0

    def entry(self):
        nb = self.name.encode() + b"\x00"
        assert len(nb) <= 64, self.name
        e = nb + b"\x00" * (64 - len(nb))
        e += struct.pack("<B", len(self.shape)) + b"\x00" * 7
        e += struct.pack("<8Q", *(self.shape + [0] * (8 - len(self.shape))))
        e += struct.pack("<BBHI", self.logical, self.storage, self.layout, self.group)
        e += struct.pack("<QQ", self.sc_off if self.scales else 0, len(self.scales))
        e += struct.pack("<QQ", self.d_off, len(self.payload))
        e += struct.pack("<I", binascii.crc32(self.payload) & 0xFFFFFFFF)
        e += struct.pack("<B", self.scale_dtype) + b"\x00" * 11
        assert len(e) == 192
        return bytearray(e)


def serialize(tensors, sections, mutate_entry=None, mutate=None, fix_sha=True):
    """The file's bytes.  sections: the four section objects (identity,
    architecture, tokenizer, policy).  mutate_entry(i, entry_bytearray) may
    alter a directory entry before the directory CRC is taken; mutate(buf)
    may alter the file before the trailing SHA-256 is taken (tests)."""
    blobs = [_blob(s) for s in sections]
    n = len(tensors)
    off = align_up(128 + 5 * 32)
    sect = []
    for i, b in enumerate(blobs, 1):
        sect.append([i, off, 8 + len(b)])
        off = align_up(off + 8 + len(b))
    doff = off
    off = align_up(off + n * 192)
    for t in tensors:  # scale pool: each tensor's scales contiguous, 64-byte aligned
        if t.scales:
            t.sc_off = off
            off = align_up(off + len(t.scales))
    for t in tensors:
        t.d_off = off
        off = align_up(off + len(t.payload))
    total = off + 32
    dir_blob = bytearray()
    for i, t in enumerate(tensors):
        e = t.entry()
        if mutate_entry:
            mutate_entry(i, e)
        dir_blob += e
    sect.append([5, doff, len(dir_blob)])
    buf = bytearray(total - 32)
    buf[0:128] = (MAGIC + struct.pack("<IIQQIIQ", VERSION, 1, n, 128, 5, ALIGN, total)
                  + b"\x00" * 80)
    for k, (sid, soff, sb) in enumerate(sect):
        if sid == 5:
            crc = binascii.crc32(bytes(dir_blob)) & 0xFFFFFFFF
        else:
            crc = binascii.crc32(struct.pack("<Q", sb - 8) + blobs[sid - 1]) & 0xFFFFFFFF
        buf[128 + 32 * k:160 + 32 * k] = struct.pack("<IQQIII", sid, soff, sb, crc, 0, 0)
    for (sid, soff, sb), b in zip(sect[:4], blobs):
        buf[soff:soff + 8 + len(b)] = struct.pack("<Q", len(b)) + b
    buf[doff:doff + len(dir_blob)] = dir_blob
    for t in tensors:
        if t.scales:
            buf[t.sc_off:t.sc_off + len(t.scales)] = t.scales
        buf[t.d_off:t.d_off + len(t.payload)] = t.payload
    if mutate:
        mutate(buf)
    digest = hashlib.sha256(bytes(buf)).digest() if fix_sha else b"\x00" * 32
    return bytes(buf) + digest


def _u8(a):
    return np.ascontiguousarray(a).view(np.uint8).tobytes()


def moe_layer_tensors(l, cfg, a, scale_fp16=True):
    """The directory entries of MoE layer l from its raw arrays (the names of
    oracle.HostLayer / ainfer_amd.moe.MoeLayer: router_w, router_bias,
    shared_gate_w, w_gate, s_gate, ..., ws_down, ss_down, and norm_w)."""
    H, E, I, Is = cfg["hidden"], cfg["n_experts"], cfg["inter"], cfg["shared_inter"]
    p = f"model.layers.{l}."
    q = DT["INT4_SYM_G128"]
    ts = [Tensor(p + "mlp.gate.weight", [E, H], DT["BF16"], _u8(a["router_w"]))]
    if a.get("router_bias") is not None:
        ts.append(Tensor(p + "mlp.gate.bias", [E], DT["FP32"], _u8(a["router_bias"]),
                         logical=DT["FP32"]))
    if a.get("shared_gate_w") is not None:
        ts.append(Tensor(p + "mlp.shared_expert_gate.weight", [1, H], DT["BF16"],
                         _u8(a["shared_gate_w"])))
    for nm, rows, K in (("gate", I, H), ("up", I, H), ("down", H, I)):
        ts.append(Tensor(p + f"mlp.experts.{nm}_proj.weight", [E, rows, K], q,
                         _u8(a["w_" + nm]), _u8(a["s_" + nm]), LAYOUT_EXPERTS, scale_fp16))
    if Is > 0:
        for nm, rows, K in (("gate", Is, H), ("up", Is, H), ("down", H, Is)):
            ts.append(Tensor(p + f"mlp.shared_expert.{nm}_proj.weight", [rows, K], q,
                             _u8(a["ws_" + nm]), _u8(a["ss_" + nm]), LAYOUT_ROW_MAJOR, scale_fp16))
    if a.get("norm_w") is not None:
        ts.append(Tensor(p + "post_attention_layernorm.weight", [H], DT["BF16"], _u8(a["norm_w"])))
    return ts


def moe_sections(cfg, n_layers, scale_fp16=True, rms_eps=1e-6):
    ident = {"source_repo": "synthetic", "source_revision": "0" * 40,
             "converter": "ainfer_amd.binfer", "converter_version": "1"}
    arch = {"arch": "moe_int4", "hidden": cfg["hidden"], "n_experts": cfg["n_experts"],
            "top_k": cfg["top_k"], "inter": cfg["inter"], "shared_inter": cfg["shared_inter"],
            "layers": n_layers, "scale_fp16": 1 if scale_fp16 else 0, "rms_eps": rms_eps}
    tok = {"tokenizer_format": "none"}
    pol = {"default_scheme": 1, "group_size": GROUP, "scale_dtype": "fp16" if scale_fp16 else "bf16"}
    return [ident, arch, tok, pol]


def write_moe(path, cfg, layers, scale_fp16=True, rms_eps=1e-6, **kw):
    """Write n MoE layers (list of raw-array dicts) to path; cfg holds hidden,
    n_experts, top_k, inter, shared_inter."""
    tensors = []
    for l, a in enumerate(layers):
        tensors += moe_layer_tensors(l, cfg, a, scale_fp16)
    data = serialize(tensors, moe_sections(cfg, len(layers), scale_fp16, rms_eps), **kw)
    with open(path, "wb") as f:
        f.write(data)
    return tensors
