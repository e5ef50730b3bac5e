"""Write tests/golden/operators_t14_subset.npz from the reference's own
operator fixture, reference/operators_t14.npz (float64, seed 0; keys listed
in reference/operators_t14_meta.json).  Only the arrays that pin this path
are kept: SiLU-gate (g, u, silu_gate_out) and RMSNorm (rmsnorm_in, _w, _out).
Data only: numpy.load with allow_pickle=False."""
import sys
from pathlib import Path

import numpy as np

SRC = Path(sys.argv[1] if len(sys.argv) > 1 else
           "/root/reference/reference/operators_t14.npz")
DST = Path(__file__).resolve().parent / "operators_t14_subset.npz"
KEYS = ("g", "u", "silu_gate_out", "rmsnorm_in", "rmsnorm_w", "rmsnorm_out")

with np.load(SRC, allow_pickle=False) as d:
    np.savez(DST, **{k: d[k] for k in KEYS})
print(f"wrote {DST}")
