"""Diagnostics on a trace build of the library (not used by the product path).

  AINFER_HIPFLAGS=-DAINFER_GEMM_TRACE python -m ainfer_amd._build /tmp/gemm_trace.so
  python -m ainfer_amd.diag gemm-phases /tmp/gemm_trace.so
  AINFER_HIPFLAGS=-DAINFER_DECODE_TRACE python -m ainfer_amd._build /tmp/decode_trace.so
  python -m ainfer_amd.diag decode-phases /tmp/decode_trace.so

decode-phases runs 8 blocks of config 4 at T = 1 (or the T given after the
library path) through the replayed stack, three steps,
and prints the last block's timeline in microseconds from the routing
kernel's first workgroup (s_memrealtime stamps per workgroup, moe_decode.hip
and moe_expert_item.h): the router waves' RMSNorm and dot, the selection's
poll, top-k and dispatch, and the gate/up and down items' start, weight
arrival and stores.

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


def decode_phases(lib_path, n_layers=8, T=1):
    import numpy as np
    from . import _lib as L
    L.LIB_PATH = Path(lib_path).resolve()
    import torch
    from .moe import MoeLayer, MoeStack, make_input
    from .synthetic import CONFIGS
    cfg = CONFIGS["c4"]
    layers = [MoeLayer(cfg, layer=i) for i in range(n_layers)]
    stack = MoeStack(layers)
    ws = stack.workspace(T)
    x = make_input(cfg, T, tag=5000) * 4
    y = torch.empty_like(x)
    for _ in range(3):
        stack.forward(x, y, ws)
    torch.cuda.synchronize()
    lib = L.lib()
    tr = np.zeros((2, 1 << 15, 5), dtype=np.uint64)
    ld = np.zeros((2, 1 << 14, 3), dtype=np.uint64)
    if lib.ainfer_debug_trace(tr.ctypes.data_as(C.c_void_p)) != 0 or \
            lib.ainfer_debug_land_expert(ld.ctypes.data_as(C.c_void_p)) != 0:
        raise RuntimeError("not a -DAINFER_DECODE_TRACE build")
    r = tr[0].astype(np.int64)
    nr = int((r[:, 0] > 0).sum())  # router units, the selection (nr - 2), the x copy
    t0 = r[:nr, 0].min()
    us = lambda v: (v - t0) / 100.0
    rr = r[:nr - 2]
    sel = r[nr - 2]
    print(f"T={T}: {nr - 2} router workgroups: start max {us(rr[:, 0].max()):.2f}, "
          f"RMSNorm done {us(np.median(rr[:, 2])):.2f} (max {us(rr[:, 2].max()):.2f}), "
          f"dot done {us(np.median(rr[:, 3])):.2f}, logits stored {us(np.median(rr[:, 1])):.2f} "
          f"(max {us(rr[:, 1].max()):.2f})")
    print(f"selection: start {us(sel[0]):.2f}, slots seen {us(sel[4]):.2f}, top-k {us(sel[1]):.2f}, "
          f"weights {us(sel[2]):.2f}, dispatch {us(sel[3]):.2f}")
    # the stand-alone expert kernel (k_expert_lds): MODE 0 gate/up, 1 down
    for m, name in ((0, "gate/up"), (1, "down")):
        g = ld[m].astype(np.int64)
        g = g[g[:, 0] > 0]
        if len(g) and T > 1 or (m == 0 and len(g)):
            print(f"{name} items ({len(g)}): start {us(g[:, 0].min()):.2f} - {us(np.median(g[:, 0])):.2f} "
                  f"(median), weights landed {us(np.median(g[:, 1])):.2f} (max {us(g[:, 1].max()):.2f}), "
                  f"written max {us(g[:, 2].max()):.2f}")
    d = tr[1].astype(np.int64)
    d = d[(d[:, 0] > 0) & (d[:, 4] == 0)]
    if len(d) and T <= 2:
        print(f"down items ({len(d)}): start {us(np.median(d[:, 0])):.2f}, stores max {us(d[:, 2].max()):.2f}, "
              f"last arrival {us(d[:, 3].max()):.2f}")
        # the fused kernel's own item stamps (start, weights landed, partials written)
        ldd = np.zeros((2, 1 << 14, 3), dtype=np.uint64)
        if lib.ainfer_debug_land(ldd.ctypes.data_as(C.c_void_p)) == 0:
            g = ldd[1].astype(np.int64)
            g = g[(g[:, 0] > 0) & (g[:, 0] >= t0)]
            if len(g):
                p = lambda v, q: us(np.percentile(v, q))
                print(f"down items, weights landed: 10/50/90% {p(g[:, 1], 10):.2f} / {p(g[:, 1], 50):.2f} / "
                      f"{p(g[:, 1], 90):.2f}, max {us(g[:, 1].max()):.2f}; start 10/50/90% "
                      f"{p(g[:, 0], 10):.2f} / {p(g[:, 0], 50):.2f} / {p(g[:, 0], 90):.2f}; "
                      f"written max {us(g[:, 2].max()):.2f}")

if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "gemm-phases":
        gemm_phases(sys.argv[2])
    elif len(sys.argv) >= 3 and sys.argv[1] == "decode-phases":
        decode_phases(sys.argv[2], T=int(sys.argv[3]) if len(sys.argv) > 3 else 1)
    else:
        print(__doc__)
        sys.exit(2)
