"""Write tests/golden/binfer/: .binfer files and the reference validator's
verdict on each, so that ainfer_binfer_open can be held to the reference's
own accept/reject decisions without the reference present.

Run in the build container only (it imports /root/reference/tools/binfer.py,
whose validate/negatives commands need only the standard library):
  - the files the reference's `negatives` command emits (binfer.py:502-622):
    its minimal valid file, bad magic, bad version, truncated, payload CRC and
    unknown layout, kept instead of deleted;
  - files written by this repository's writer (ainfer_amd/binfer.py): one in
    layout 0 only (row-major INT4 with bf16 and fp16 scales, a BF16 tensor),
    which the reference must accept, and one with an expert-stacked tensor in
    layout_id 32, which the reference rejects ("unsupported layout_id": the
    one extension this format makes);
  - verdicts.json: file -> the return code of the reference's cmd_validate
    (0 = valid) and its error messages.
"""
import contextlib
import importlib.util
import io
import json
import shutil
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "binfer"
REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tools/binfer.py")
sys.path.insert(0, str(HERE.parent.parent))
from ainfer_amd import binfer as B  # noqa: E402


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_binfer", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ours():
    sec = [{"source_repo": "ainfer_amd", "source_revision": "0" * 40}, {"arch": "moe-test"},
           {"format": "none"}, {"default": "int4_sym_g128"}]
    q = bytes((i * 37 + 11) & 0xFF for i in range(4 * 256 // 2))
    s_bf16 = bytes.fromhex("3c3c") * (4 * 256 // 128)
    s_fp16 = bytes.fromhex("0020") * (4 * 256 // 128)
    row = [B.Tensor("blk.0.mlp.gate.weight", [4, 256], B.DT["INT4_SYM_G128"], q, s_bf16),
           B.Tensor("blk.0.mlp.up.weight", [4, 256], B.DT["INT4_SYM_G128"], q[::-1], s_fp16,
                    scale_fp16=True),
           B.Tensor("blk.0.norm.weight", [256], B.DT["BF16"], bytes(range(256)) * 2)]
    stacked = row[:2] + [B.Tensor("blk.0.mlp.experts.down.weight", [2, 2, 128],
                                  B.DT["INT4_SYM_G128"], bytes(256), b"\x03\x04" * 4,
                                  B.LAYOUT_EXPERTS)]
    return {"ours_layout0.binfer": B.serialize(row, sec),
            "ours_layout32.binfer": B.serialize(stacked, sec)}


def main():
    ref = load_reference()
    if OUT.exists():
        shutil.rmtree(OUT)
    OUT.mkdir(parents=True)
    # the negatives command writes into a fresh temporary directory and
    # deletes it at the end; point it at a directory kept for collection
    work = Path(tempfile.mkdtemp())
    real_mkdtemp, real_rmtree = tempfile.mkdtemp, shutil.rmtree
    tempfile.mkdtemp = lambda *a, **k: str(work)
    shutil.rmtree = lambda *a, **k: None
    try:
        with contextlib.redirect_stdout(io.StringIO()):
            rc = ref.cmd_negatives()
    finally:
        tempfile.mkdtemp, shutil.rmtree = real_mkdtemp, real_rmtree
    assert rc == 0, "the reference's own negative tests failed"
    for p in sorted(work.glob("*.binfer")):
        if p.name == "tiny.binfer":
            continue
        shutil.copy(p, OUT / ("ref_" + p.name))
    real_rmtree(work)
    for name, data in ours().items():
        (OUT / name).write_bytes(data)
    verdicts = {}
    for p in sorted(OUT.glob("*.binfer")):
        buf = io.StringIO()
        with contextlib.redirect_stdout(buf):
            rc = ref.cmd_validate(str(p))
        verdicts[p.name] = {"rc": rc, "errors": list(ref.ERRORS)}
    (OUT / "verdicts.json").write_text(json.dumps(verdicts, indent=1, sort_keys=True) + "\n")
    print(json.dumps({k: v["rc"] for k, v in verdicts.items()}))


if __name__ == "__main__":
    main()
