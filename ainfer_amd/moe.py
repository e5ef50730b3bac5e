"""Host-side operator surface over the C ABI (device memory via torch).

MoeLayer owns one layer's device weights in the layout include/ainfer_moe.h
documents; forward/route/dispatch/block_forward enqueue on a HIP stream and
return immediately, like the C entry points they wrap.  Every call goes to
libainfer_moe.so; there is no other implementation behind these names.
"""
import ctypes as C

import numpy as np
import torch

from . import _lib as L
from .synthetic import MoeConfig, tensor_seed, layer_seed, input_seed, zipf_bias


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p(0)


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def fill_(kind: int, seed: int, std: float, t: torch.Tensor, stream=None):
    """Fill a device tensor with the counter-based synthetic generator."""
    n = t.numel() * t.element_size() if kind == L.FILL_BYTES else t.numel()
    L.check(L.lib().ainfer_moe_fill(kind, C.c_uint64(seed), C.c_float(std), n, _ptr(t),
                                    _stream(stream)))
    return t


class MoeLayer:
    """One INT4 MoE layer resident in HBM (synthetic seeded weights)."""

    def __init__(self, cfg: MoeConfig, layer: int = 0, device="cuda",
                 scale_dtype: int = L.SCALE_FP16, stream=None,
                 precision: int = L.PRECISION_W4A16):
        self.cfg, self.layer, self.device = cfg, layer, device
        H, E, I, Is = cfg.hidden, cfg.n_experts, cfg.inter, cfg.shared_inter
        self.shape = L.Shape(H, E, cfg.top_k, I, Is, 128, scale_dtype, precision)
        L.check(L.lib().ainfer_moe_validate(C.byref(self.shape)))
        ls = layer_seed(cfg.seed, layer)
        sdt = torch.float16 if scale_dtype == L.SCALE_FP16 else torch.bfloat16
        skind = L.FILL_FP16_ABSNORMAL if scale_dtype == L.SCALE_FP16 else L.FILL_BF16_ABSNORMAL
        u8 = dict(dtype=torch.uint8, device=device)

        def packed(name, rows, K, n_mat=1):
            return fill_(L.FILL_BYTES, tensor_seed(ls, name), 0.0,
                         torch.empty(n_mat * rows * K // 2, **u8), stream)

        def scales(name, rows, K, n_mat=1):
            return fill_(skind, tensor_seed(ls, name), cfg.scale_std,
                         torch.empty(n_mat * rows * K // 128, dtype=sdt, device=device), stream)

        t = {}
        t["router_w"] = fill_(L.FILL_BF16_NORMAL, tensor_seed(ls, "router_w"), cfg.weight_std,
                              torch.empty(E * H, dtype=torch.bfloat16, device=device), stream)
        t["shared_gate_w"] = (fill_(L.FILL_BF16_NORMAL, tensor_seed(ls, "shared_gate_w"),
                                    cfg.weight_std,
                                    torch.empty(H, dtype=torch.bfloat16, device=device), stream)
                              if cfg.shared_gate and Is > 0 else None)
        t["router_bias"] = (torch.from_numpy(zipf_bias(cfg, layer)).to(device)
                            if cfg.zipf > 0 else None)
        t["w_gate"], t["s_gate"] = packed("w_gate", I, H, E), scales("s_gate", I, H, E)
        t["w_up"], t["s_up"] = packed("w_up", I, H, E), scales("s_up", I, H, E)
        t["w_down"], t["s_down"] = packed("w_down", H, I, E), scales("s_down", H, I, E)
        if Is > 0:
            t["ws_gate"], t["ss_gate"] = packed("ws_gate", Is, H), scales("ss_gate", Is, H)
            t["ws_up"], t["ss_up"] = packed("ws_up", Is, H), scales("ss_up", Is, H)
            t["ws_down"], t["ss_down"] = packed("ws_down", H, Is), scales("ss_down", H, Is)
        self.t = t
        self.weights = L.Weights(*[_ptr(t.get(n)) for n, _ in L.Weights._fields_])

    def set_tensor(self, name: str, t):
        """Replace one device tensor (same layout) and refresh the C struct."""
        self.t[name] = t
        self.weights = L.Weights(*[_ptr(self.t.get(n)) for n, _ in L.Weights._fields_])

    def workspace(self, max_tokens: int) -> torch.Tensor:
        n = L.lib().ainfer_moe_workspace_bytes(C.byref(self.shape), max_tokens)
        if n == 0:
            raise L.MoeError("invalid shape or token count for workspace")
        ws = torch.empty(n + 256, dtype=torch.uint8, device=self.device)
        off = (-ws.data_ptr()) % 256
        ws = ws[off:off + n]
        L.check(L.lib().ainfer_moe_workspace_init(C.byref(self.shape), _ptr(ws), n, _stream(None)))
        return ws

    def workspace_check(self, ws, stream=None) -> int:
        """Status of the workspace's synchronisation words (OK when all zero)."""
        return L.lib().ainfer_moe_workspace_check(C.byref(self.shape), _ptr(ws), ws.numel(),
                                                  _stream(stream))

    def forward(self, x, y, ws, stream=None):
        T = x.shape[0]
        return L.check(L.lib().ainfer_moe_forward(
            C.byref(self.shape), C.byref(self.weights), _ptr(x), _ptr(y), T, _ptr(ws),
            ws.numel(), _stream(stream)))

    def block_forward(self, resid_in, resid_out, ws, norm_w=None, norm_mode=L.NORM_PLAIN,
                      eps=1e-6, stream=None):
        T = resid_in.shape[0]
        return L.check(L.lib().ainfer_moe_block_forward(
            C.byref(self.shape), C.byref(self.weights), _ptr(norm_w), norm_mode, eps,
            _ptr(resid_in), _ptr(resid_out), T, _ptr(ws), ws.numel(), _stream(stream)))

    def block_forward_noalloc(self, resid_in, resid_out, norm_w=None, norm_mode=L.NORM_PLAIN,
                              eps=1e-6, stream=None):
        """block_forward on the library's static per-GPU scratch (no workspace)."""
        T = resid_in.shape[0]
        return L.check(L.lib().ainfer_moe_block_forward_noalloc(
            C.byref(self.shape), C.byref(self.weights), _ptr(norm_w), norm_mode, eps,
            _ptr(resid_in), _ptr(resid_out), T, _stream(stream)))

    def route(self, x, ws, want_logits=False, stream=None):
        T, E, k = x.shape[0], self.cfg.n_experts, self.cfg.top_k
        dev = self.device
        idx = torch.empty(T, k, dtype=torch.int32, device=dev)
        w = torch.empty(T, k, dtype=torch.float32, device=dev)
        sg = torch.empty(T, dtype=torch.float32, device=dev)
        lg = torch.empty(T, E, dtype=torch.float32, device=dev) if want_logits else None
        L.check(L.lib().ainfer_moe_route(C.byref(self.shape), C.byref(self.weights), _ptr(x), T,
                                         _ptr(idx), _ptr(w), _ptr(sg), _ptr(lg), _ptr(ws),
                                         ws.numel(), _stream(stream)))
        return idx, w, sg, lg

    def experts(self, x, idx, ws, stream=None):
        """Expert rows in slot order: [T * k + T][H] bf16 (row t * k + j =
        expert idx[t][j] on token t, row T * k + t = the shared expert)."""
        T, k, H = x.shape[0], self.cfg.top_k, self.cfg.hidden
        o = torch.empty(T * k + T, H, dtype=torch.bfloat16, device=self.device)
        L.check(L.lib().ainfer_moe_experts(C.byref(self.shape), C.byref(self.weights), _ptr(x),
                                           _ptr(idx), T, _ptr(o), _ptr(ws), ws.numel(),
                                           _stream(stream)))
        return o

    def combine(self, o, w, sg, y, resid=None, stream=None):
        T = y.shape[0]
        L.check(L.lib().ainfer_moe_combine(C.byref(self.shape), _ptr(o), _ptr(w), _ptr(sg),
                                           _ptr(resid), _ptr(y), T, _stream(stream)))
        return y

    def dispatch(self, idx, ws, stream=None):
        T, E, k = idx.shape[0], self.cfg.n_experts, self.cfg.top_k
        dev = self.device
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        perm = torch.empty(max(T * k, 1), dtype=torch.int32, device=dev)
        inv = torch.empty(max(T * k, 1), dtype=torch.int32, device=dev)
        L.check(L.lib().ainfer_moe_dispatch(C.byref(self.shape), _ptr(idx), T, _ptr(counts),
                                            _ptr(offsets), _ptr(perm), _ptr(inv), _ptr(ws),
                                            ws.numel(), _stream(stream)))
        return counts, offsets, perm[:T * k], inv[:T * k]


def load_binfer_layer(bf, layer, device="cuda"):
    """Layer `layer` of an opened BinferFile, copied into a device arena: a
    MoeLayer whose weights are the file's (no synthetic fill); its norm
    weight (or None) is returned beside it."""
    shape, n_layers, eps = bf.moe_info()
    nbytes = bf.layer_bytes(layer)
    arena = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    off = (-arena.data_ptr()) % 256
    arena = arena[off:off + nbytes]
    w = L.Weights()
    nw = C.c_void_p()
    L.check(L.lib().ainfer_binfer_load_moe_layer(bf.h, layer, _ptr(arena), nbytes, C.byref(w),
                                                 C.byref(nw), _stream(None)))
    ly = MoeLayer.__new__(MoeLayer)
    ly.cfg = None
    ly.device = device
    ly.shape = shape
    ly.weights = w
    ly.t = {"arena": arena}
    norm = None
    if nw.value:
        # a view of the arena at the norm weight's offset
        norm = arena[nw.value - arena.data_ptr():][:shape.hidden * 2].view(torch.bfloat16)
    return ly, norm


def with_precision(layer, precision):
    """The same resident layer (shared weights) run in another precision."""
    twin = MoeLayer.__new__(MoeLayer)
    twin.__dict__.update(layer.__dict__)
    twin.shape = L.Shape.from_buffer_copy(layer.shape)
    twin.shape.precision = precision
    L.check(L.lib().ainfer_moe_validate(C.byref(twin.shape)))
    return twin


class MoeStack:
    """L decoder-block MLP halves as one call (ainfer_moe_stack_forward: the
    layers' kernels replayed, each layer's combine computing the next layer's
    RMSNorm; any T), or as one persistent launch
    (ainfer_moe_stack_forward_persistent, T <= 4).  The layers' weights and
    per-layer RMSNorm weights go into a device table once
    (ainfer_moe_stack_prepare)."""

    def __init__(self, layers, norm_ws=None, device="cuda"):
        assert layers, "a stack needs at least one layer"
        self.layers = list(layers)
        self.shape = self.layers[0].shape
        n = len(self.layers)
        lib = L.lib()
        self.table = torch.empty(lib.ainfer_moe_stack_table_bytes(n), dtype=torch.uint8,
                                 device=device)
        arr = (L.Weights * n)(*[ly.weights for ly in self.layers])
        self.norm_ws = list(norm_ws) if norm_ws is not None else None
        nw = None
        if self.norm_ws is not None:
            assert len(self.norm_ws) == n
            nw = (C.c_void_p * n)(*[_ptr(w) for w in self.norm_ws])
        L.check(lib.ainfer_moe_stack_prepare(C.byref(self.shape), arr, nw, n,
                                             _ptr(self.table), self.table.numel(), None))

    def workspace(self, max_tokens: int) -> torch.Tensor:
        lib = L.lib()
        n = lib.ainfer_moe_stack_workspace_bytes(C.byref(self.shape), max_tokens, len(self.layers))
        if n == 0:
            raise L.MoeError("invalid shape or token count for a stack workspace")
        ws = torch.empty(n + 256, dtype=torch.uint8, device=self.table.device)
        off = (-ws.data_ptr()) % 256
        ws = ws[off:off + n]
        L.check(lib.ainfer_moe_workspace_init(C.byref(self.shape), _ptr(ws), n, _stream(None)))
        return ws

    def forward(self, resid_in, resid_out, ws, norm_mode=L.NORM_PLAIN, eps=1e-6, stream=None,
                persistent=False):
        T = resid_in.shape[0]
        fn = (L.lib().ainfer_moe_stack_forward_persistent if persistent
              else L.lib().ainfer_moe_stack_forward)
        return L.check(fn(
            C.byref(self.shape), _ptr(self.table), len(self.layers), norm_mode, eps,
            _ptr(resid_in), _ptr(resid_out), T, _ptr(ws), ws.numel(), _stream(stream)))


def make_input(cfg: MoeConfig, T: int, tag: int = 0, device="cuda", stream=None):
    """x[T][H] bf16 ~ N(0, 1) (standardised Irwin-Hall), seeded by (cfg.seed, tag)."""
    x = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device=device)
    return fill_(L.FILL_BF16_NORMAL, input_seed(cfg.seed, tag), 1.0, x, stream)


def rmsnorm(x, y, w=None, mode=L.NORM_PLAIN, eps=1e-6, stream=None):
    T, H = x.shape
    return L.check(L.lib().ainfer_moe_rmsnorm(_ptr(x), _ptr(w), mode, eps, _ptr(y), T, H,
                                              _stream(stream)))
