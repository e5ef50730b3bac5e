#!/usr/bin/env python3
"""Benchmark of the INT4 MoE layer on one MI355X.

Headline (the JSON line's `value`): config c4, the 60-block decode step at 1
token -- microseconds per token of the whole step (each block: RMSNorm ->
MoE layer H4096, 512 experts, top-10, I1024 + shared expert, INT4 g128 fp16
scales -> residual add; 200 GB of weights resident).  It is the largest
BASELINE config that fits one GPU.  `details` adds c4 at 8 tokens, c1 decode
at 1/4/16 tokens, the c2 prefill (4096 tokens, Zipf(1.1) routing) in tokens/s
and % of bf16 MFMA peak, c3 (64 tokens) and the W4A8 GEMV.

`roofline` prices the dominant kernel of a c4 block: its algorithmic bytes
per launch over its mean device time (HIP events on the launch stream, each
pair also spanning the launch gap before the kernel, so an upper bound on
the time).  `roofline.traffic` (HBM bytes per launch of that kernel) is read
from the committed rocprofv3 PMC summary
profiles/<kernel>_c4_T<T>_traffic.md (FETCH_SIZE + WRITE_SIZE, scaled by the
same counters on a copy of known size, made with --calib-copy); null when
that file is absent.

Inputs are resident in HBM before the timed region.  c4 reads 60 distinct
layers per step (200 GB, far above the 256 MB MALL).  c1 decode steps cycle
over NL distinct layer copies and NX distinct token batches for the same
reason.  Per-kernel device times come from HIP events the library records on
the launch stream (ainfer_moe_profile_*) in a second pass over the same
steps; the headline timed region runs without them.

The CPU baseline is the C oracle (oracle/libmoe_oracle.so, `port`) on the
box's host cores: one c4 block (layer 0, the same synthetic weights) timed
for a bounded sample, median x 60 blocks.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "MoE layer decode us/token + % HBM peak; prefill tokens/s + % MFMA peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def unique_experts(layer, x, ws):
    import torch
    idx, _, _, _ = layer.route(x, ws)
    return int(torch.unique(idx).numel())


def gateup_bytes(cfg, U):
    """INT4 nibbles + fp16 scales of gate and up for U routed experts and the
    shared expert (the gate/up kernel's weight bytes)."""
    per = lambda I: 2 * (cfg.hidden * I // 2 + cfg.hidden * I // 128 * 2)
    return U * per(cfg.inter) + (per(cfg.shared_inter) if cfg.shared_inter else 0)


def experts_bytes(cfg, U, T):
    """Algorithmic bytes of the decode expert kernel (k_experts_decode): INT4
    nibbles + fp16 scales of gate, up and down for U routed experts and the
    shared expert, plus the bf16 tokens read and the bf16 outputs written."""
    per = lambda I: 3 * (cfg.hidden * I // 2 + cfg.hidden * I // 128 * 2)
    w = U * per(cfg.inter) + (per(cfg.shared_inter) if cfg.shared_inter else 0)
    return w + 2 * T * cfg.hidden * 2


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    profiles/<kernel>_<workload>_traffic.md, or None."""
    f = ROOT / "profiles" / f"{kernel}_{workload}_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def run_decode(layers, cfg, T, steps, warmup, NX, stream):
    import torch
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    NL = len(layers)
    xs = [make_input(cfg, T, tag=1000 + 7 * T + i) for i in range(NX)]
    ws = layers[0].workspace(T)
    y = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    for s in range(warmup):
        layers[s % NL].forward(xs[s % NX], y, ws, stream)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for s in range(steps):
        layers[s % NL].forward(xs[s % NX], y, ws, stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # profiled pass: per-kernel device times on the launch stream
    L.profile_enable(True)
    for s in range(steps):
        layers[s % NL].forward(xs[s % NX], y, ws, stream)
    torch.cuda.synchronize()
    stages, ncalls = L.profile_read()
    L.profile_enable(False)
    # routing statistics of the pairs the loop visited
    pairs = sorted({(s % NL, s % NX) for s in range(steps)})
    U = sum(unique_experts(layers[l], xs[i], ws) for l, i in pairs) / len(pairs)
    torch.cuda.synchronize()
    return ms, stages, U


def run_prefill(layer, cfg, T, steps, warmup, stream):
    import torch
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    x = make_input(cfg, T, tag=4242)
    ws = layer.workspace(T)
    y = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        layer.forward(x, y, ws, stream)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        layer.forward(x, y, ws, stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    L.profile_enable(True)
    for _ in range(steps):
        layer.forward(x, y, ws, stream)
    torch.cuda.synchronize()
    stages, _ = L.profile_read()
    L.profile_enable(False)
    U = unique_experts(layer, x, ws)
    return ms, stages, U


def run_gemv_w4a8(steps, copies=8, M=17408, K=5120):
    """The reference's headline GEMV shape (tools/cmdlist/gemv_replay.cpp:57)
    in its W4A8 numerics: activation quantisation + INT4 x int8 GEMV per
    step, `copies` distinct weight matrices cycled so none stays in the MALL."""
    import ctypes as C
    import torch
    from ainfer_amd import _lib as L
    lib = L.lib()
    p = lambda t: C.c_void_p(t.data_ptr())
    G = K // 128
    Ws, Ss = [], []
    for i in range(copies):
        w = torch.empty(M * K // 2, dtype=torch.uint8, device="cuda")
        s = torch.empty(M * G, dtype=torch.int16, device="cuda")
        L.check(lib.ainfer_moe_fill(L.FILL_BYTES, 77 + i, 0.0, w.numel(), p(w), None))
        L.check(lib.ainfer_moe_fill(L.FILL_BF16_ABSNORMAL, 177 + i, 0.02, s.numel(), p(s), None))
        Ws.append(w)
        Ss.append(s)
    x = torch.randn(1, K, device="cuda", dtype=torch.float32) * 50
    q = torch.empty(1, K, dtype=torch.int8, device="cuda")
    sq = torch.empty(1, G, dtype=torch.float32, device="cuda")
    y = torch.empty(1, M, dtype=torch.float32, device="cuda")

    def step(i, quant=True):
        if quant:
            L.check(lib.ainfer_moe_act_quant_i8(p(x), L.ACT_F32, 1, K, p(q), p(sq), None))
        L.check(lib.ainfer_moe_int4_gemv_i8(p(Ws[i % copies]), p(Ss[i % copies]), L.SCALE_BF16,
                                            p(q), p(sq), M, K, 1, p(y), None))
    res = {}
    for quant in (False, True):
        for i in range(10):
            step(i, quant)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(steps):
            step(i, quant)
        t1.record()
        torch.cuda.synchronize()
        res[quant] = t0.elapsed_time(t1) / steps * 1e3
    nbytes = M * K // 2 + M * G * 2 + K + G * 4 + M * 4
    return {"shape": f"M={M} K={K} T=1 (gemv_replay.cpp:57)", "gemv_us": round(res[False], 3),
            "gemv_gbs": round(nbytes / (res[False] * 1e-6) / 1e9, 1),
            "gemv_hbm_frac": round(nbytes / (res[False] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "quant_plus_gemv_us": round(res[True], 3), "alg_bytes": nbytes,
            "reference_b60_replay_us": 283.0}


def run_c3(steps, warmup=5):
    """H4096 E512 k10 I1024 + shared, 64 tokens (the
    16-token-tile streaming kernels).  One layer is 3.3 GB, far above the
    256 MB MALL, so one copy suffices."""
    import torch
    from ainfer_amd.moe import MoeLayer, make_input
    from ainfer_amd.synthetic import CONFIGS, algorithmic_bytes
    cfg, T = CONFIGS["c3"], 64
    layer = MoeLayer(cfg)
    xs = [make_input(cfg, T, tag=3000 + i) for i in range(8)]
    ws = layer.workspace(T)
    y = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    for i in range(warmup):
        layer.forward(xs[i % 8], y, ws)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        layer.forward(xs[i % 8], y, ws)
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / steps
    U = sum(unique_experts(layer, x, ws) for x in xs) / len(xs)
    nbytes = algorithmic_bytes(cfg, T, round(U))
    out = {"us_per_step": round(us, 2), "us_per_token": round(us / T, 3), "unique_experts": U,
           "alg_bytes": nbytes, "layer_hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "layer_hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del layer, ws, xs, y
    torch.cuda.empty_cache()
    return out


def run_c4(steps, tokens=(1, 8), warmup=3, keep_layer0=False, stack=True):
    """60 blocks of config 3 (RMSNorm -> MoE -> residual),
    one decode step = all 60 blocks in sequence on a bf16 residual stream,
    200 GB of weights resident.  The step is one ainfer_moe_stack_forward
    call (the layers' kernels replayed; from T = 5 on each layer's combine
    computes the next layer's RMSNorm).  Beside it: the same step as 60
    chained ainfer_moe_block_forward calls, and (T <= 4) as the one-launch
    persistent kernel.  A second pass over the stack's steps reads per-stage
    device times (HIP events on the launch stream, mean per block)."""
    import torch
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeLayer, MoeStack, make_input, rmsnorm
    from ainfer_amd.synthetic import CONFIGS, algorithmic_bytes
    cfg = CONFIGS["c4"]
    log(f"[bench] c4: allocating {cfg.layers} layers "
        f"({cfg.layers * cfg.layer_weight_bytes() / 1e9:.1f} GB)")
    layers = [MoeLayer(cfg, layer=i) for i in range(cfg.layers)]
    stk = MoeStack(layers)
    torch.cuda.synchronize()
    out = {}
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)

    def timed(step):
        for s in range(warmup):
            step(s)
        torch.cuda.synchronize()
        t0.record()
        for s in range(steps):
            step(s)
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e3 / steps

    for T in tokens:
        log(f"[bench] c4 T={T}")
        ws = layers[0].workspace(T)
        sws = stk.workspace(T)
        r0 = make_input(cfg, T, tag=4000 + T) * 4
        # distinct routed experts per layer along the actual residual stream
        U = 0.0
        h = torch.empty_like(r0)
        cur = r0.clone()
        for L_ in layers:
            rmsnorm(cur, h)
            U += unique_experts(L_, h, ws)
            nxt = torch.empty_like(cur)
            L_.block_forward(cur, nxt, ws)
            cur = nxt
        # one decode step = one fresh token batch through all 60 blocks: block
        # 0 reads x_s, the others update the residual in place
        xs = [make_input(cfg, T, tag=4100 + 16 * T + i) * 4 for i in range(8)]
        y = torch.empty_like(r0)

        def step(s):
            stk.forward(xs[s % len(xs)], y, sws)
        us = timed(step)
        # a bounded device wait that ran out leaves NaN rows: such a step is not a result
        if not bool(torch.isfinite(y).all()):
            raise RuntimeError(f"c4 T={T}: the 60-block residual is not finite")
        L.check(layers[0].workspace_check(sws))
        y_stack = y.clone()

        def step_blocks(s):
            layers[0].block_forward(xs[s % len(xs)], y, ws)
            for L_ in layers[1:]:
                L_.block_forward(y, y, ws)
        blocks_us = timed(step_blocks)
        # the last steps of both forms ran the same input: the same bits
        if not torch.equal(y.view(torch.int16), y_stack.view(torch.int16)):
            raise RuntimeError(f"c4 T={T}: stack and chained blocks differ")
        # profiled pass: mean device time per stage and block
        L.profile_enable(True)
        for s in range(steps):
            step(s)
        torch.cuda.synchronize()
        st, _ = L.profile_read()
        k_us, _ = L.profile_kernel()  # the gate/up kernel's own duration
        L.profile_enable(False)
        Ul = U / len(layers)
        nbytes = sum(algorithmic_bytes(cfg, T, 0) for _ in layers) + round(U) * cfg.expert_bytes()
        # dominant kernel of a block: the gate/up expert kernel when it runs
        # on its own (stage 4), else the fused expert kernel (stage 5)
        if st["gate_up"] > 0:
            dom = {"kernel": "k_expert_lds<fp16, gate/up> (gate/up + SiLU of the routed and "
                             "shared experts)", "file": "k_expert_gate_up",
                   "alg_bytes": gateup_bytes(cfg, Ul), "us": k_us if k_us > 0 else st["gate_up"],
                   "us_stage_events": st["gate_up"]}
        else:
            dom = {"kernel": "k_experts_decode (gate/up + down + combine)",
                   "file": "k_experts_decode",
                   "alg_bytes": experts_bytes(cfg, Ul, T), "us": st["down"]}
        dom["gbs"] = dom["alg_bytes"] / (dom["us"] * 1e-6) / 1e9 if dom["us"] else 0.0
        pers_us = None
        if stack and T <= L.STACK_MAX_TOKENS:
            # the same step as one persistent launch (ainfer_moe_stack_forward_persistent)
            def step_p(s):
                stk.forward(xs[s % len(xs)], y, sws, persistent=True)
            pers_us = round(timed(step_p), 1)
            if not bool(torch.isfinite(y).all()):
                raise RuntimeError(f"c4 T={T}: the persistent stack's residual is not finite")
        w8_us = None
        if T == 1:
            # the same step in the reference's W4A8 numerics (row f3: int8
            # activations per group of 128, Int4Gemv products, fp32 SiluMul
            # and combine), on the same resident weights
            from ainfer_amd.moe import with_precision
            w8 = MoeStack([with_precision(L_, L.PRECISION_W4A8) for L_ in layers])
            ws8 = w8.workspace(T)

            def step8(s):
                w8.forward(xs[s % len(xs)], y, ws8)
            w8_us = round(timed(step8), 1)
            del w8, ws8
        out[str(T)] = {"us_per_step": round(us, 1), "us_per_token": round(us / T, 2),
                       "us_per_block": round(us / len(layers), 2),
                       "unique_experts_per_layer": round(Ul, 2),
                       "alg_bytes_per_step": nbytes,
                       "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                       "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "stage_us_per_block": {k: round(v, 3) for k, v in st.items() if v > 0},
                       "dominant": dom,
                       "chained_blocks_us_per_step": round(blocks_us, 1),
                       "stack_persistent_us_per_step": pers_us,
                       "w4a8_us_per_step": w8_us,
                       "w4a8_hbm_frac": (round(nbytes / (w8_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                                         if w8_us else None)}
        log(f"[bench]   c4 T={T}: {json.dumps(out[str(T)])}")
        del ws, sws
    keep = layers[0] if keep_layer0 else None
    del layers, stk
    torch.cuda.empty_cache()
    return out, keep


def add_read_roof_fracs(details, read_gbs):
    """Beside every decode line's fraction of the 8 TB/s spec, its fraction of
    the read roof this box sustained in the same run (hbm_read_gbs)."""
    for d in (details.get("c4_stack60") or {}).values():
        d["hbm_frac_of_read_roof"] = round(d["hbm_gbs"] / read_gbs, 4)
    for d in (details.get("decode_c1") or {}).values():
        d["layer_hbm_frac_of_read_roof"] = round(d["layer_hbm_gbs"] / read_gbs, 4)
    c3 = details.get("c3_T64")
    if c3:
        c3["layer_hbm_frac_of_read_roof"] = round(c3["layer_hbm_frac"] * HBM_PEAK_GBS / read_gbs, 4)
    g = details.get("gemv_w4a8")
    if g:
        g["gemv_hbm_frac_of_read_roof"] = round(g["gemv_hbm_frac"] * HBM_PEAK_GBS / read_gbs, 4)


def measured_peaks():
    """What this box sustains, beside the spec peaks: a 1 GiB device copy
    (read + write bytes), a bf16 8192^3 GEMM through the vendor BLAS, and the
    MFMA rate of a loop with a given VALU load (ainfer_moe_mfma_probe)."""
    import torch
    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(10):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * n * 10 / (t0.elapsed_time(t1) * 1e-3) / 1e9
    del src, dst
    # read-only roof: the decode path streams weights and writes almost
    # nothing; random bytes over 4 GiB (far beyond the 256 MB MALL), best of a
    # sweep over loads in flight per lane and blocks per CU
    import ctypes as C
    from ainfer_amd import _lib
    nr = 4 << 30
    rbuf = torch.randint(0, 256, (nr,), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    read = {}
    for unroll in (4, 8, 16):
        for bpc in (2, 4, 8):
            r = C.c_float()
            rc = _lib.lib().ainfer_moe_read_probe(C.c_void_p(rbuf.data_ptr()), nr, unroll, bpc, 5,
                                                  C.c_void_p(torch.cuda.current_stream().cuda_stream),
                                                  C.byref(r))
            if rc != _lib.OK:
                raise RuntimeError(f"ainfer_moe_read_probe failed: {rc}")
            read[f"u{unroll}_b{bpc}"] = round(r.value, 1)
    del rbuf
    torch.cuda.empty_cache()
    m = 8192
    a = torch.randn(m, m, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(m, m, device="cuda", dtype=torch.bfloat16)
    for _ in range(3):
        c = a @ b
    torch.cuda.synchronize()
    t0.record()
    for _ in range(10):
        c = a @ b
    t1.record()
    torch.cuda.synchronize()
    tfs = 2 * m ** 3 * 10 / (t0.elapsed_time(t1) * 1e-3) / 1e12
    del a, b, c
    torch.cuda.empty_cache()
    # the bf16 MFMA rate with 0-4 fp32 VALU instructions issued per MFMA, 1
    # and 2 waves per SIMD: the ceiling of an MFMA main loop that spends that
    # much VALU work (the prefill GEMM's dequantisation and scale step)
    mf = {}
    for wps in (1, 2):
        for nv in range(5):
            r = C.c_float()
            rc = _lib.lib().ainfer_moe_mfma_probe(nv, wps, 4000, C.c_void_p(torch.cuda.current_stream().cuda_stream),
                                                  C.byref(r))
            if rc != _lib.OK:
                raise RuntimeError(f"ainfer_moe_mfma_probe failed: {rc}")
            mf[f"w{wps}_v{nv}"] = round(r.value, 1)
    read_gbs = max(read.values())
    return {"hbm_copy_gbs": round(copy_gbs, 1), "hbm_copy_frac_of_spec": round(copy_gbs / HBM_PEAK_GBS, 4),
            "hbm_read_gbs": read_gbs, "hbm_read_frac_of_spec": round(read_gbs / HBM_PEAK_GBS, 4),
            "hbm_read_sweep_gbs_unroll_blocks_per_cu": read,
            "bf16_gemm_8192_tflops": round(tfs, 1),
            "bf16_gemm_frac_of_spec": round(tfs / MFMA_BF16_PEAK_TFS, 4),
            "mfma_probe_tflops_waves_per_simd_valu_per_mfma": mf}


def host_cpu():
    """(cores this process may run on, CPU model name) of the host."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, model


def cpu_baseline(cfg, T, budget_s, blocks=1, layer=0):
    """The C oracle's block (RMSNorm -> MoE -> residual) on host cores,
    bounded to about budget_s seconds; the median block time is scaled by
    `blocks` (the stack's depth: its blocks are alike in work)."""
    import numpy as np
    from oracle import oracle as O
    from ainfer_amd.synthetic import input_seed

    hl = O.HostLayer.synthetic(cfg, layer=layer)
    avail, model = host_cpu()
    threads = max(1, min(avail, 16))
    # residual rows ~ 4 N(0,1) in bf16 bits, the same generator as the GPU's inputs
    xs = [O.f32_to_bf16(O.bf16_to_f32(O.fill(O.FILL_BF16_NORMAL, input_seed(cfg.seed, 9000 + i),
                                             1.0, T * cfg.hidden)) * 4).reshape(T, cfg.hidden)
          for i in range(8)]
    hl.block_forward(xs[0], T, threads=threads)  # warm
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while (time.perf_counter() < t_end or len(times) < 3) and len(times) < 2000:
        t = time.perf_counter()
        hl.block_forward(xs[i % len(xs)], T, threads=threads)
        times.append(time.perf_counter() - t)
        i += 1
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(med * blocks * 1e6 / T, 1), "unit": "us/token", "cores": threads,
            "kind": "port", "host_cpus": avail, "cpu_model": model,
            "sample": f"{cfg.name} T={T}: {len(times)} calls of the C oracle's block "
                      f"(RMSNorm + MoE layer + residual) on layer {layer}, median "
                      f"{med * 1e3:.2f} ms x {blocks} blocks, {threads} threads, "
                      f"{len(xs)} distinct inputs"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10,
                    help="timed 60-block c4 steps (the headline); c1 decode runs 20x as many")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=8, help="distinct c1 layer copies cycled")
    ap.add_argument("--tokens", default="1,4,16", help="c1 decode batch sizes")
    ap.add_argument("--c4-tokens", default="1,8", help="c4 batch sizes (the first is the headline)")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the c1 decode lines")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true", help="skip the W4A8 GEMV line")
    ap.add_argument("--no-c3", action="store_true", help="skip config 3 (H4096, 64 tokens)")
    ap.add_argument("--no-c4", action="store_true",
                    help="skip config 4 (no headline line: prints the details only)")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured-peak probes")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the persistent one-launch timing of c4 "
                         "(ainfer_moe_stack_forward_persistent)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="finally copy MIB MiB device-to-device 5 times (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(expert parallelism is a design only)", file=sys.stderr)
        sys.exit(2)

    import torch
    from ainfer_amd.moe import MoeLayer
    from ainfer_amd.synthetic import CONFIGS, algorithmic_bytes, algorithmic_flops

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    stream = torch.cuda.current_stream()
    c4cfg = CONFIGS["c4"]

    # ---- headline: the 60-block c4 decode step -----------------------------
    c4 = None
    c4_tokens = [int(v) for v in args.c4_tokens.split(",")]
    if not args.no_c4:
        c4, _ = run_c4(args.steps, tokens=c4_tokens, warmup=args.warmup, stack=not args.no_stack)

    # ---- details -----------------------------------------------------------
    c1 = CONFIGS["c1"]
    decode = {}
    if not args.no_decode:
        log(f"[bench] allocating {args.layers} c1 layers "
            f"({args.layers * c1.layer_weight_bytes() / 1e9:.1f} GB)")
        layers = [MoeLayer(c1, layer=i) for i in range(args.layers)]
        torch.cuda.synchronize()
        for T in [int(v) for v in args.tokens.split(",")]:
            log(f"[bench] c1 decode T={T}")
            ms, st, U = run_decode(layers, c1, T, 20 * args.steps, 20 * args.warmup, 64, stream)
            nbytes = algorithmic_bytes(c1, T, round(U))
            ex_us = st["gate_up"] + st["down"] + st["combine"]
            ex_bytes = experts_bytes(c1, U, T)
            decode[T] = {
                "us_per_step": ms * 1e3, "us_per_token": ms * 1e3 / T,
                "unique_experts": U, "alg_bytes": nbytes,
                "layer_hbm_gbs": nbytes / (ms * 1e-3) / 1e9,
                "layer_hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "route_us": round(st["topk"], 3), "experts_us": round(ex_us, 3),
                "experts_gbs": ex_bytes / (ex_us * 1e-6) / 1e9 if ex_us > 0 else 0.0,
                "stage_us": {k: round(v, 3) for k, v in st.items() if v > 0},
            }
            if st["gate_up"] > 0:
                decode[T]["gate_up_gbs"] = gateup_bytes(c1, U) / (st["gate_up"] * 1e-6) / 1e9
            log(f"[bench]   {json.dumps(decode[T])}")
        del layers
        torch.cuda.empty_cache()

    prefill = None
    if not args.no_prefill:
        c2 = CONFIGS["c2"]
        T = 4096
        log("[bench] c2 prefill T=4096")
        layer2 = MoeLayer(c2)
        ms, st, U = run_prefill(layer2, c2, T, args.prefill_steps, 2, stream)
        fl = algorithmic_flops(c2, T)
        gu_flops = 2 * T * (c2.top_k + 1) * 2 * c2.hidden * c2.inter
        prefill = {
            "tokens_per_s": T / (ms * 1e-3), "ms_per_step": ms, "unique_experts": U,
            "alg_flops": fl, "layer_tflops": fl / (ms * 1e-3) / 1e12,
            "layer_mfma_frac": fl / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFS,
            "stage_us": {k: round(v, 3) for k, v in st.items()},
            "gate_up_tflops": gu_flops / (st["gate_up"] * 1e-6) / 1e12 if st["gate_up"] else 0,
        }
        log(f"[bench]   {json.dumps(prefill)}")
        # chunked prefill: 16384 tokens as four 4096-token chunks on one workspace
        T2 = 16384
        ms2, st2, _ = run_prefill(layer2, c2, T2, max(2, args.prefill_steps // 2), 1, stream)
        fl2 = algorithmic_flops(c2, T2)
        prefill["chunked_T16384"] = {
            "tokens_per_s": T2 / (ms2 * 1e-3), "ms_per_step": ms2,
            "layer_mfma_frac": fl2 / (ms2 * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFS}
        log(f"[bench]   chunked T=16384: {json.dumps(prefill['chunked_T16384'])}")
        del layer2
        torch.cuda.empty_cache()

    gemv = None
    if not args.no_gemv:
        log("[bench] W4A8 GEMV 17408x5120")
        gemv = run_gemv_w4a8(20 * args.steps)
        log(f"[bench]   {json.dumps(gemv)}")

    c3 = run_c3(100) if not args.no_c3 else None
    if c3:
        log(f"[bench] c3 T=64: {json.dumps(c3)}")
    peaks = measured_peaks() if not args.no_peaks else None

    if args.calib_copy > 0:
        n = args.calib_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: 5 x {n} bytes")

    details = {
        "c4_stack60": c4,
        "decode_c1": {str(T): {k: (round(v, 4) if isinstance(v, float) else v)
                               for k, v in d.items()} for T, d in decode.items()},
        "prefill_c2_T4096": prefill,
        "gemv_w4a8": gemv,
        "c3_T64": c3,
        "measured_peaks": peaks,
    }
    if peaks:
        add_read_roof_fracs(details, peaks["hbm_read_gbs"])
    if c4 is None:
        print(json.dumps(details), flush=True)
        return
    Th = c4_tokens[0]
    h = c4[str(Th)]
    dom = h["dominant"]

    cpu = None
    if not args.no_cpu:
        log(f"[bench] cpu baseline: c4 block T={Th}, x{c4cfg.layers}")
        cpu = cpu_baseline(c4cfg, Th, args.cpu_seconds, blocks=c4cfg.layers)
        log(f"[bench]   {json.dumps(cpu)}")
    out = {
        "metric": METRIC,
        "value": h["us_per_token"],
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["us_per_step"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded counter-based generator; random-init INT4 weights)",
        "config": {"workload": f"c4 decode T={Th}: 60 sequential blocks (RMSNorm -> MoE layer "
                               "-> residual), each H4096 E512 top-10 I1024 + 1 shared expert "
                               "(sigmoid gate), INT4 g128 fp16 scales, 200 GB resident",
                   "global_batch": Th, "layers": c4cfg.layers, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4),
                     "frac_of_read_roof": (round(dom["gbs"] / peaks["hbm_read_gbs"], 4)
                                           if peaks else None),
                     "traffic": measured_traffic(dom["file"], f"c4_T{Th}"),
                     "kernel": dom["kernel"],
                     "alg_bytes_per_launch": round(dom["alg_bytes"]),
                     "us_per_launch": round(dom["us"], 3)},
        "cpu_baseline": cpu,
        "details": dict(step_hbm_frac=h["hbm_frac"], **details),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
