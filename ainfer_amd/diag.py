"""Diagnostics on a trace build of the library (not used by the product path).

  AINFER_HIPFLAGS=-DAINFER_GEMM_TRACE python -m ainfer_amd._build /tmp/gemm_trace.so
  python -m ainfer_amd.diag gemm-phases /tmp/gemm_trace.so

gemm-phases runs the c2 prefill layer (T = 4096, Zipf routing) a few times and
prints, per grouped-GEMM kind, the mean shader-clock span of an item's
prologue (tables, first DMA), main loop and epilogue, from the per-item
s_memtime stamps of k_expert_gemm (moe_gemm.hip, AINFER_GEMM_TRACE)."""
import ctypes as C
import sys
from pathlib import Path


def gemm_phases(lib_path, steps=3):
    import numpy as np
    from . import _lib as L
    L.LIB_PATH = Path(lib_path).resolve()
    import torch
    from .moe import MoeLayer, make_input
    from .synthetic import CONFIGS
    cfg = CONFIGS["c2"]
    T = 4096
    layer = MoeLayer(cfg)
    x = make_input(cfg, T, tag=4242)
    ws = layer.workspace(T)
    y = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    for _ in range(steps):
        layer.forward(x, y, ws)
    torch.cuda.synchronize()
    buf = np.zeros(2 * 16384 * 4, dtype=np.uint64)
    if L.lib().ainfer_debug_gemm_trace(buf.ctypes.data_as(C.c_void_p)) != 0:
        raise RuntimeError("not a -DAINFER_GEMM_TRACE build")
    out = {}
    for mode, name in ((0, "gate_up"), (1, "down")):
        ts = buf.reshape(2, 16384, 4)[mode].astype(np.int64)
        ts = ts[ts[:, 0] > 0]
        pro, loop, epi = ts[:, 1] - ts[:, 0], ts[:, 2] - ts[:, 1], ts[:, 3] - ts[:, 2]
        tot = (ts[:, 3] - ts[:, 0]).mean()
        out[name] = {"items": len(ts), "prologue": pro.mean(), "loop": loop.mean(),
                     "epilogue": epi.mean(), "total": tot}
        print(f"{name}: {len(ts)} items, clocks per item: prologue {pro.mean():.0f} "
              f"({pro.mean() / tot:.0%}), loop {loop.mean():.0f} ({loop.mean() / tot:.0%}), "
              f"epilogue {epi.mean():.0f} ({epi.mean() / tot:.0%})", flush=True)
    return out


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "gemm-phases":
        gemm_phases(sys.argv[2])
    else:
        print(__doc__)
        sys.exit(2)
