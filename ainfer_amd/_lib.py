"""ctypes binding of include/ainfer_moe.h (libainfer_moe.so, built in-tree).

Loading fails loudly: there is no CPU fallback behind this module.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libainfer_moe.so"

OK = 0
ERR_SHAPE, ERR_NULL, ERR_WORKSPACE, ERR_TOKENS, ERR_HIP, ERR_ARG, ERR_SYNC, ERR_SCRATCH = (
    -1, -2, -3, -4, -5, -6, -7, -8)
ERR_FORMAT, ERR_IO = -9, -10
BINFER_LAYOUT_EXPERTS = 32
NOALLOC_SCRATCH_BYTES = 16 << 20
SCALE_BF16, SCALE_FP16 = 0, 1
PRECISION_W4A16, PRECISION_W4A8 = 0, 1
NORM_PLAIN, NORM_ONE_PLUS = 0, 1
ACT_F32, ACT_BF16 = 0, 1
FILL_BYTES, FILL_BF16_NORMAL, FILL_FP16_ABSNORMAL, FILL_BF16_ABSNORMAL = 0, 1, 2, 3
MAX_TOKENS = 65536
STACK_MAX_TOKENS = 4

# every symbol include/ainfer_moe.h declares
EXPORTS = (
    "ainfer_moe_strerror", "ainfer_moe_validate", "ainfer_moe_workspace_bytes",
    "ainfer_moe_workspace_init", "ainfer_moe_workspace_check",
    "ainfer_moe_forward", "ainfer_moe_block_forward", "ainfer_moe_block_forward_noalloc",
    "ainfer_moe_stack_workspace_bytes", "ainfer_moe_stack_table_bytes", "ainfer_moe_stack_prepare", "ainfer_moe_stack_forward",
    "ainfer_moe_stack_forward_persistent",
    "ainfer_moe_route",
    "ainfer_moe_dispatch", "ainfer_moe_experts", "ainfer_moe_combine", "ainfer_moe_rmsnorm", "ainfer_moe_fill",
    "ainfer_moe_act_quant_i8", "ainfer_moe_int4_gemv_i8",
    "ainfer_moe_profile_enable", "ainfer_moe_profile_read", "ainfer_moe_profile_kernel", "ainfer_moe_debug_spin_limit",
    "ainfer_moe_set_strict",
    "ainfer_moe_mfma_probe", "ainfer_moe_read_probe",
    "ainfer_binfer_open", "ainfer_binfer_close", "ainfer_binfer_error", "ainfer_binfer_moe_info",
    "ainfer_binfer_moe_layer_bytes", "ainfer_binfer_load_moe_layer",
)
N_STAGES = 7
STAGES = ("rmsnorm", "router", "topk", "dispatch", "gate_up", "down", "combine")


class Shape(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32),
                ("inter", C.c_int32), ("shared_inter", C.c_int32), ("group", C.c_int32),
                ("scale_dtype", C.c_int32), ("precision", C.c_int32)]


class Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "router_w", "router_bias", "shared_gate_w", "w_gate", "s_gate", "w_up", "s_up",
        "w_down", "s_down", "ws_gate", "ss_gate", "ws_up", "ss_up", "ws_down", "ss_down")]


class MoeError(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise MoeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first "
                           "(there is no fallback path)")
        L = C.CDLL(str(LIB_PATH))
        P, I32, SZ, F = C.c_void_p, C.c_int32, C.c_size_t, C.c_float
        sp, wp = C.POINTER(Shape), C.POINTER(Weights)
        L.ainfer_moe_strerror.restype = C.c_char_p
        L.ainfer_moe_strerror.argtypes = [C.c_int]
        L.ainfer_moe_validate.argtypes = [sp]
        L.ainfer_moe_workspace_bytes.restype = SZ
        L.ainfer_moe_workspace_bytes.argtypes = [sp, I32]
        L.ainfer_moe_workspace_init.argtypes = [sp, P, SZ, P]
        L.ainfer_moe_workspace_check.argtypes = [sp, P, SZ, P]
        L.ainfer_moe_forward.argtypes = [sp, wp, P, P, I32, P, SZ, P]
        L.ainfer_moe_block_forward.argtypes = [sp, wp, P, I32, F, P, P, I32, P, SZ, P]
        L.ainfer_moe_block_forward_noalloc.argtypes = [sp, wp, P, I32, F, P, P, I32, P]
        L.ainfer_moe_stack_workspace_bytes.restype = SZ
        L.ainfer_moe_stack_workspace_bytes.argtypes = [sp, I32, I32]
        L.ainfer_moe_stack_table_bytes.restype = SZ
        L.ainfer_moe_stack_table_bytes.argtypes = [I32]
        L.ainfer_moe_stack_prepare.argtypes = [sp, wp, C.POINTER(C.c_void_p), I32, P, SZ, P]
        L.ainfer_moe_stack_forward.argtypes = [sp, P, I32, I32, F, P, P, I32, P, SZ, P]
        L.ainfer_moe_stack_forward_persistent.argtypes = [sp, P, I32, I32, F, P, P, I32, P, SZ, P]
        L.ainfer_moe_route.argtypes = [sp, wp, P, I32, P, P, P, P, P, SZ, P]
        L.ainfer_moe_dispatch.argtypes = [sp, P, I32, P, P, P, P, P, SZ, P]
        L.ainfer_moe_experts.argtypes = [sp, wp, P, P, I32, P, P, SZ, P]
        L.ainfer_moe_combine.argtypes = [sp, P, P, P, P, P, I32, P]
        L.ainfer_moe_rmsnorm.argtypes = [P, P, I32, F, P, I32, I32, P]
        L.ainfer_moe_fill.argtypes = [I32, C.c_uint64, F, SZ, P, P]
        L.ainfer_moe_act_quant_i8.argtypes = [P, I32, I32, I32, P, P, P]
        L.ainfer_moe_int4_gemv_i8.argtypes = [P, P, I32, P, P, I32, I32, I32, P, P]
        L.ainfer_moe_profile_enable.argtypes = [I32]
        L.ainfer_moe_profile_kernel.argtypes = [C.POINTER(C.c_float), C.POINTER(I32)]
        L.ainfer_moe_mfma_probe.argtypes = [I32, I32, I32, P, C.POINTER(C.c_float)]
        L.ainfer_moe_read_probe.argtypes = [P, C.c_uint64, I32, I32, I32, P, C.POINTER(C.c_float)]
        L.ainfer_binfer_open.argtypes = [C.c_char_p, C.POINTER(P), C.c_char_p, SZ]
        L.ainfer_binfer_close.restype = None
        L.ainfer_binfer_close.argtypes = [P]
        L.ainfer_binfer_error.restype = C.c_char_p
        L.ainfer_binfer_error.argtypes = [P]
        L.ainfer_binfer_moe_info.argtypes = [P, sp, C.POINTER(I32), C.POINTER(F)]
        L.ainfer_binfer_moe_layer_bytes.restype = SZ
        L.ainfer_binfer_moe_layer_bytes.argtypes = [P, I32]
        L.ainfer_binfer_load_moe_layer.argtypes = [P, I32, P, SZ, wp, C.POINTER(P), P]
        L.ainfer_moe_debug_spin_limit.argtypes = [I32]
        L.ainfer_moe_set_strict.argtypes = [I32]
        L.ainfer_moe_profile_read.argtypes = [C.POINTER(C.c_float), I32, C.POINTER(I32)]
        for name in EXPORTS:
            if name != "ainfer_binfer_close":
                getattr(L, name).restype = getattr(L, name).restype or C.c_int
        _lib = L
    return _lib


def check(rc):
    if rc != OK:
        raise MoeError(f"ainfer_moe status {rc}: {lib().ainfer_moe_strerror(rc).decode()}")
    return rc


def profile_enable(on: bool):
    check(lib().ainfer_moe_profile_enable(1 if on else 0))


def profile_kernel():
    """Mean device microseconds of the decode gate/up kernel itself (its
    dispatch-stamped start/end) since profile_enable(True), and the count."""
    v = C.c_float(0.0)
    n = C.c_int32(0)
    check(lib().ainfer_moe_profile_kernel(C.byref(v), C.byref(n)))
    return float(v.value), int(n.value)


def profile_read():
    """Mean device microseconds per stage since profile_enable(True)."""
    arr = (C.c_float * N_STAGES)()
    n = C.c_int32(0)
    check(lib().ainfer_moe_profile_read(arr, N_STAGES, C.byref(n)))
    return dict(zip(STAGES, list(arr))), n.value


class BinferFile:
    """An opened, fully validated .binfer container (ainfer_binfer_open)."""

    def __init__(self, path):
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = lib().ainfer_binfer_open(str(path).encode(), C.byref(h), err, len(err))
        if rc != OK:
            raise MoeError(f"ainfer_binfer_open status {rc}: {err.value.decode()}")
        self.h = h

    def close(self):
        if self.h:
            lib().ainfer_binfer_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def moe_info(self):
        s = Shape()
        n = C.c_int32(0)
        eps = C.c_float(0.0)
        check(lib().ainfer_binfer_moe_info(self.h, C.byref(s), C.byref(n), C.byref(eps)))
        return s, n.value, eps.value

    def layer_bytes(self, layer):
        return lib().ainfer_binfer_moe_layer_bytes(self.h, layer)
