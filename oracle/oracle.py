"""ctypes wrapper of the CPU oracle (oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product never imports it.
"""
import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libmoe_oracle.so"
REF_SAMPLER = HERE / "_ref" / "libref_sampler.so"

SCALE_BF16, SCALE_FP16 = 0, 1
FILL_BYTES, FILL_BF16_NORMAL, FILL_FP16_ABSNORMAL, FILL_BF16_ABSNORMAL = 0, 1, 2, 3
NORM_PLAIN, NORM_ONE_PLUS = 0, 1


class Shape(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32),
                ("inter", C.c_int32), ("shared_inter", C.c_int32), ("group", C.c_int32),
                ("scale_dtype", C.c_int32), ("precision", C.c_int32)]


class Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "router_w", "router_bias", "shared_gate_w", "w_gate", "s_gate", "w_up", "s_up",
        "w_down", "s_down", "ws_gate", "ss_gate", "ws_up", "ss_up", "ws_down", "ss_down")]


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if Path("/root/reference/tools/sample/sampler.h").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P, I, F = C.c_void_p, C.c_int, C.c_float
        L.mo_bf16_to_f32.restype = F
        L.mo_bf16_to_f32.argtypes = [C.c_uint16]
        L.mo_f32_to_bf16.restype = C.c_uint16
        L.mo_f32_to_bf16.argtypes = [F]
        L.mo_fp16_to_f32.restype = F
        L.mo_fp16_to_f32.argtypes = [C.c_uint16]
        L.mo_f32_to_fp16.restype = C.c_uint16
        L.mo_f32_to_fp16.argtypes = [F]
        L.mo_rnd.restype = C.c_uint64
        L.mo_rnd.argtypes = [C.c_uint64, C.c_uint64]
        L.mo_fill.argtypes = [I, C.c_uint64, F, C.c_size_t, P]
        L.mo_dequant_int4.argtypes = [P, P, I, I, I, P]
        L.mo_quantize_int4.argtypes = [P, I, I, P, P]
        L.mo_silu_mul.argtypes = [P, P, P, I]
        L.mo_rms_sumsq.restype = C.c_double
        L.mo_rms_sumsq.argtypes = [P, I]
        L.mo_rmsnorm_f32.argtypes = [P, P, I, F, P, I, I]
        L.mo_rmsnorm_bf16.argtypes = [P, P, I, F, P, I, I]
        L.mo_router_dot.restype = F
        L.mo_router_dot.argtypes = [P, P, I]
        L.mo_router.argtypes = [P, P, P, I, P, P, I]
        L.mo_topk.argtypes = [P, I, I, I, P, P]
        L.mo_route.argtypes = [P, P, P, I, P, P, P, P, I]
        L.mo_dispatch.argtypes = [P, I, I, I, P, P, P, P]
        L.mo_forward.argtypes = [P, P, P, I, P, P, I]
        L.mo_block_forward.argtypes = [P, P, P, I, F, P, P, I, I]
        L.mo_forward_dense.argtypes = [P, P, P, I, P, P, P, P]
        L.mo_forward_w4a8.argtypes = [P, P, P, I, P, I]
        L.mo_act_quant_i8.argtypes = [P, P, I, I, P, P]
        L.mo_int4_gemv_i8.argtypes = [P, P, I, P, P, I, I, I, P]
        L.mo_ref_gemv_inputs.argtypes = [I, I, I, P, P, P]
        _lib = L
    return _lib


def ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def nthreads():
    return max(1, min(os.cpu_count() or 1, 16))


# ---- bit helpers -----------------------------------------------------------
def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def fill(kind, seed, std, n):
    dt = np.uint8 if kind == FILL_BYTES else np.uint16
    out = np.empty(n, dtype=dt)
    lib().mo_fill(kind, C.c_uint64(seed), C.c_float(std), n, ptr(out))
    return out


# ---- host copy of a synthetic layer ---------------------------------------
class HostLayer:
    """A layer's tensors as numpy arrays (raw bits), with the ctypes structs."""

    def __init__(self, shape_tuple, arrays: dict, scale_dtype=SCALE_FP16):
        H, E, k, I, Is = shape_tuple
        self.H, self.E, self.k, self.I, self.Is = H, E, k, I, Is
        self.a = {n: (np.ascontiguousarray(v) if v is not None else None)
                  for n, v in arrays.items()}
        self.shape = Shape(H, E, k, I, Is, 128, scale_dtype, 0)
        self.weights = Weights(*[ptr(self.a.get(n)) for n, _ in Weights._fields_])

    @classmethod
    def synthetic(cls, cfg, layer=0, scale_dtype=SCALE_FP16):
        """Generate the layer on the host with the oracle's own fill."""
        import sys
        sys.path.insert(0, str(HERE.parent))
        from ainfer_amd.synthetic import tensor_seed, layer_seed, zipf_bias
        H, E, I, Is = cfg.hidden, cfg.n_experts, cfg.inter, cfg.shared_inter
        ls = layer_seed(cfg.seed, layer)
        sk = FILL_FP16_ABSNORMAL if scale_dtype == SCALE_FP16 else FILL_BF16_ABSNORMAL
        a = {
            "router_w": fill(FILL_BF16_NORMAL, tensor_seed(ls, "router_w"), cfg.weight_std, E * H),
            "shared_gate_w": (fill(FILL_BF16_NORMAL, tensor_seed(ls, "shared_gate_w"),
                                   cfg.weight_std, H) if cfg.shared_gate and Is > 0 else None),
            "router_bias": zipf_bias(cfg, layer) if cfg.zipf > 0 else None,
        }
        for nm, rows, K, n_mat in (("gate", I, H, E), ("up", I, H, E), ("down", H, I, E)):
            a["w_" + nm] = fill(FILL_BYTES, tensor_seed(ls, "w_" + nm), 0, n_mat * rows * K // 2)
            a["s_" + nm] = fill(sk, tensor_seed(ls, "s_" + nm), cfg.scale_std,
                                n_mat * rows * K // 128)
        if Is > 0:
            for nm, rows, K in (("gate", Is, H), ("up", Is, H), ("down", H, Is)):
                a["ws_" + nm] = fill(FILL_BYTES, tensor_seed(ls, "ws_" + nm), 0, rows * K // 2)
                a["ss_" + nm] = fill(sk, tensor_seed(ls, "ss_" + nm), cfg.scale_std,
                                     rows * K // 128)
        return cls(cfg.shape_tuple(), a, scale_dtype)

    # ---- oracle calls ------------------------------------------------------
    def route(self, x: np.ndarray, T: int, threads=None):
        idx = np.empty((T, self.k), np.int32)
        w = np.empty((T, self.k), np.float32)
        sg = np.empty(T, np.float32)
        lg = np.empty((T, self.E), np.float32)
        lib().mo_route(C.byref(self.shape), C.byref(self.weights), ptr(x), T, ptr(idx), ptr(w),
                       ptr(sg), ptr(lg), threads or nthreads())
        return idx, w, sg, lg

    def forward(self, x: np.ndarray, T: int, threads=None):
        y = np.empty((T, self.H), np.float32)
        lib().mo_forward(C.byref(self.shape), C.byref(self.weights), ptr(x), T, ptr(y), None,
                         threads or nthreads())
        return y

    def forward_w4a8(self, x: np.ndarray, T: int, threads=None):
        """The layer in W4A8 numerics (fp32 output)."""
        y = np.empty((T, self.H), np.float32)
        lib().mo_forward_w4a8(C.byref(self.shape), C.byref(self.weights), ptr(x), T, ptr(y),
                              threads or nthreads())
        return y

    def block_forward(self, resid: np.ndarray, T: int, norm_w=None, mode=NORM_PLAIN, eps=1e-6,
                      threads=None):
        out = np.empty((T, self.H), np.uint16)
        lib().mo_block_forward(C.byref(self.shape), C.byref(self.weights), ptr(norm_w), mode,
                               C.c_float(eps), ptr(resid), ptr(out), T, threads or nthreads())
        return out

    def forward_dense(self, x, T, idx, w, sg):
        y = np.empty((T, self.H), np.float64)
        lib().mo_forward_dense(C.byref(self.shape), C.byref(self.weights), ptr(x), T, ptr(idx),
                               ptr(w), ptr(sg), ptr(y))
        return y


def dispatch(idx: np.ndarray, E: int):
    T, k = idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(max(T * k, 1), np.int32)
    inv = np.empty(max(T * k, 1), np.int32)
    lib().mo_dispatch(ptr(np.ascontiguousarray(idx, dtype=np.int32)), T, k, E, ptr(counts),
                      ptr(offsets), ptr(perm), ptr(inv))
    return counts, offsets, perm[:T * k], inv[:T * k]


def topk(logits: np.ndarray, k: int):
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib().mo_topk(ptr(np.ascontiguousarray(logits, dtype=np.float32)), T, E, k, ptr(idx), ptr(w))
    return idx, w


def router_dot(x: np.ndarray, w: np.ndarray) -> float:
    return lib().mo_router_dot(ptr(np.ascontiguousarray(x, np.uint16)),
                               ptr(np.ascontiguousarray(w, np.uint16)), x.size)


def rmsnorm_f32(x, w, mode, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    y = np.empty_like(x)
    lib().mo_rmsnorm_f32(ptr(x), ptr(None if w is None else np.ascontiguousarray(w, np.float32)),
                         mode, C.c_float(eps), ptr(y), T, H)
    return y


def rms_sumsq(x) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().mo_rms_sumsq(ptr(x), x.size)


def rmsnorm_bf16(x, w, mode, eps=1e-6):
    x = np.ascontiguousarray(x, np.uint16)
    T, H = x.shape
    y = np.empty_like(x)
    lib().mo_rmsnorm_bf16(ptr(x), ptr(w), mode, C.c_float(eps), ptr(y), T, H)
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float64)
    u = np.ascontiguousarray(u, np.float64)
    out = np.empty_like(g)
    lib().mo_silu_mul(ptr(g), ptr(u), ptr(out), g.size)
    return out


def dequant(packed, scales, scale_dtype, rows, K):
    out = np.empty((rows, K), np.float32)
    lib().mo_dequant_int4(ptr(np.ascontiguousarray(packed, np.uint8)),
                          ptr(np.ascontiguousarray(scales, np.uint16)), scale_dtype, rows, K,
                          ptr(out))
    return out


def quantize(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, K = w.shape
    packed = np.zeros(rows * K // 2, np.uint8)
    scales = np.zeros(rows * K // 128, np.uint16)
    lib().mo_quantize_int4(ptr(w), rows, K, ptr(packed), ptr(scales))
    return packed, scales


def act_quant_i8(x: np.ndarray):
    """x [T][K] float32 or bf16 bits (uint16) -> (q int8 [T][K], sq float32 [T][K/128])."""
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    sq = np.empty((T, K // 128), np.float32)
    if x.dtype == np.uint16:
        lib().mo_act_quant_i8(None, ptr(np.ascontiguousarray(x)), T, K, ptr(q), ptr(sq))
    else:
        lib().mo_act_quant_i8(ptr(np.ascontiguousarray(x, np.float32)), None, T, K, ptr(q), ptr(sq))
    return q, sq


def int4_gemv_i8(packed, scales, scale_dtype, q, sq, M, K):
    """y [T][M] float32 of the reference's Int4Gemv arithmetic."""
    T = q.shape[0]
    y = np.empty((T, M), np.float32)
    lib().mo_int4_gemv_i8(ptr(np.ascontiguousarray(packed, np.uint8)),
                          ptr(np.ascontiguousarray(scales, np.uint16)), scale_dtype,
                          ptr(np.ascontiguousarray(q, np.int8)),
                          ptr(np.ascontiguousarray(sq, np.float32)), M, K, T, ptr(y))
    return y


def ref_gemv_inputs(M, K, n_vec):
    """The reference GEMV test's inputs (gemv_replay.cpp:158-192 generator):
    packed [M][K/2], bf16 scales [M][K/128], x [n_vec][K] float32."""
    packed = np.empty(M * K // 2, np.uint8)
    scales = np.empty(M * K // 128, np.uint16)
    x = np.empty((n_vec, K), np.float32)
    lib().mo_ref_gemv_inputs(M, K, n_vec, ptr(packed), ptr(scales), ptr(x))
    return packed, scales, x


_ref = None


def ref_sampler():
    """The reference's own tools/sample/sampler.h, built into oracle/_ref
    (None when it was not built: needs /root/reference at build time)."""
    global _ref
    if _ref is None and REF_SAMPLER.exists():
        L = C.CDLL(str(REF_SAMPLER))
        L.ref_topk_probs.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        L.ref_topk_probs.restype = C.c_int
        _ref = L
    return _ref


def ref_topk_probs(logits: np.ndarray, k: int):
    L = ref_sampler()
    logits = np.ascontiguousarray(logits, np.float32)
    probs = np.empty(logits.size, np.float32)
    L.ref_topk_probs(ptr(logits), logits.size, k, ptr(probs))
    return probs
