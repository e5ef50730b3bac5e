"""The decode stack in both forms -- ainfer_moe_stack_forward (the layers'
kernels replayed, each layer's combine computing the next layer's RMSNorm)
and ainfer_moe_stack_forward_persistent (L blocks in one launch, T <= 4) --
against L chained ainfer_moe_block_forward calls, which the other GPU tests
pin to the oracle: the outputs must be bit-identical.  Config 4's shape
(H4096, E512, top-10, I1024 + shared) with four independent layers, T = 1..4
(the fused and the three-launch expert paths of block_forward) in both forms
and T = 5, 8, 16 and 64 replayed (the fused combine + next RMSNorm), both
RMSNorm weight forms with per-layer weights, in place and out of place,
repeated calls (the layer tags advance) and calls interleaved with
block_forward on the same workspace; config 1's shape (H2048) up to the
prefill path (T = 300) and a chunked call (T = 4100); the argument errors;
and the bounded waits made to run out from the host (NaN outputs, no hang)."""
import numpy as np
import pytest

from test_gpu_parity import check_close, host_copy, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _bits(t):
    import torch
    return t.view(torch.int16)


def _chain(layers, r, ws, norm_ws, mode):
    cur = r.clone()
    for ly, nw in zip(layers, norm_ws):
        ly.block_forward(cur, cur, ws, norm_w=nw, norm_mode=mode)
    return cur


@pytest.fixture(scope="module")
def c4_stack(torch):
    import test_gpu_parity as P
    from ainfer_amd.moe import MoeLayer
    from ainfer_amd.synthetic import CONFIGS
    P._layers.clear()
    torch.cuda.empty_cache()
    cfg = CONFIGS["c4"]
    layers = [MoeLayer(cfg, layer=i) for i in (0, 17, 30, 59)]
    g = torch.Generator().manual_seed(21)
    norm_ws = [None if i == 2 else (torch.randn(cfg.hidden, generator=g) * 0.3 + 0.5)
               .to(torch.bfloat16).cuda() for i in range(len(layers))]
    torch.cuda.synchronize()
    yield cfg, layers, norm_ws
    del layers
    torch.cuda.empty_cache()


CASES_C4 = [(T, "replay") for T in (1, 2, 3, 4, 5, 8, 16, 64)] + \
    [(T, "persistent") for T in (1, 2, 3, 4)]


@pytest.mark.parametrize("T,form", CASES_C4)
@pytest.mark.parametrize("mode", ["plain", "one_plus"])
def test_stack_equals_chained_blocks_c4(torch, c4_stack, T, form, mode):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, make_input
    cfg, layers, norm_ws = c4_stack
    nm = L.NORM_PLAIN if mode == "plain" else L.NORM_ONE_PLUS
    stack = MoeStack(layers, norm_ws)
    ws = stack.workspace(T)
    wsb = layers[0].workspace(T)
    pers = form == "persistent"
    for rep in range(2):
        print(f"[case] stack c4 T={T} {form} mode={mode} rep={rep}", flush=True)
        r0 = (make_input(cfg, T, tag=6100 + 10 * T + rep) * 4).contiguous()
        want = _chain(layers, r0, wsb, norm_ws, nm)
        out = torch.empty_like(r0)
        stack.forward(r0, out, ws, norm_mode=nm, persistent=pers)
        torch.cuda.synchronize()
        assert not torch.isnan(out.float()).any(), (T, mode, rep)
        assert torch.equal(_bits(out), _bits(want)), (T, mode, rep)
        # in place
        r = r0.clone()
        stack.forward(r, r, ws, norm_mode=nm, persistent=pers)
        torch.cuda.synchronize()
        assert torch.equal(_bits(r), _bits(want)), (T, mode, rep, "in place")
    assert layers[0].workspace_check(ws) == L.OK
    # the per-block entries run on the stack's workspace at T = 1
    if T == 1:
        r = r0.clone()
        layers[0].block_forward(r, r, ws, norm_w=norm_ws[0], norm_mode=nm)
        r1 = r0.clone()
        layers[0].block_forward(r1, r1, wsb, norm_w=norm_ws[0], norm_mode=nm)
        torch.cuda.synchronize()
        assert torch.equal(_bits(r), _bits(r1))


def test_stack_matches_oracle_per_block_c4(torch, oracle, c4_stack):
    """Independently of block_forward: a one-layer stack against the
    oracle's block, within the layer tolerance."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, make_input
    cfg, layers, norm_ws = c4_stack
    hl = host_copy(oracle, layers[1])
    stack = MoeStack([layers[1]], [norm_ws[1]])
    for T, pers in ((1, True), (3, True), (1, False), (8, False)):
        ws = stack.workspace(T)
        r0 = (make_input(cfg, T, tag=6300 + T) * 4).contiguous()
        out = torch.empty_like(r0)
        stack.forward(r0, out, ws, norm_mode=L.NORM_ONE_PLUS, persistent=pers)
        torch.cuda.synchronize()
        want = hl.block_forward(to_np(r0), T, norm_w=to_np(norm_ws[1]), mode=L.NORM_ONE_PLUS)
        check_close(to_np(out), oracle.bf16_to_f32(want), f"stack vs oracle T={T}")


@pytest.mark.parametrize("name", ["c1", "c0"])
def test_stack_equals_chained_blocks_small(torch, name):
    import test_gpu_parity as P
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeLayer, MoeStack, make_input
    from ainfer_amd.synthetic import CONFIGS
    P._layers.clear()
    torch.cuda.empty_cache()
    cfg = CONFIGS[name]
    layers = [MoeLayer(cfg, layer=i) for i in range(3)]
    norm_ws = [None] * 3
    stack = MoeStack(layers)
    cases = [(T, p) for T in (1, 2, 4) for p in (True, False)] + [(8, False), (300, False)]
    if name == "c1":
        cases.append((4100, False))  # two chunks, the second of 4 tokens
    for T, pers in cases:
        print(f"[case] stack {name} T={T} persistent={pers}", flush=True)
        ws = stack.workspace(T)
        r0 = (make_input(cfg, T, tag=6200 + T) * 2).contiguous()
        want = _chain(layers, r0, layers[0].workspace(T), norm_ws, L.NORM_PLAIN)
        out = torch.empty_like(r0)
        stack.forward(r0, out, ws, persistent=pers)
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(want)), (name, T, pers)
    del layers, stack
    torch.cuda.empty_cache()


def test_stack_argument_errors(torch, c4_stack):
    import ctypes as C
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, _ptr, _stream
    cfg, layers, _ = c4_stack
    stack = MoeStack(layers[:2])
    lib = L.lib()
    ws = stack.workspace(4)
    r = torch.zeros(5, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    sh = C.byref(stack.shape)
    for f in (lib.ainfer_moe_stack_forward_persistent, lib.ainfer_moe_stack_forward):
        fwd = lambda T, n=2, mode=L.NORM_PLAIN, tab=stack.table: f(
            sh, _ptr(tab), n, mode, 1e-6, _ptr(r), _ptr(r), T, _ptr(ws), ws.numel(), _stream(None))
        assert fwd(-1) == L.ERR_TOKENS
        assert fwd(0) == L.OK and fwd(2, n=0) == L.OK
        assert fwd(2, mode=7) == L.ERR_ARG
        assert fwd(2, tab=None) == L.ERR_NULL
        need = (ws.numel() if f == lib.ainfer_moe_stack_forward_persistent
                else lib.ainfer_moe_workspace_bytes(sh, 4))
        assert f(sh, _ptr(stack.table), 2, 0, 1e-6, _ptr(r), _ptr(r), 4,
                 _ptr(ws), need - 256, _stream(None)) == L.ERR_WORKSPACE
    assert lib.ainfer_moe_stack_forward_persistent(
        sh, _ptr(stack.table), 2, L.NORM_PLAIN, 1e-6, _ptr(r), _ptr(r), 5, _ptr(ws), ws.numel(),
        _stream(None)) == L.ERR_TOKENS
    # the replayed form needs the host copy ainfer_moe_stack_prepare keeps
    other = torch.zeros_like(stack.table)
    assert lib.ainfer_moe_stack_forward(sh, _ptr(other), 2, L.NORM_PLAIN, 1e-6, _ptr(r), _ptr(r),
                                        2, _ptr(ws), ws.numel(), _stream(None)) == L.ERR_ARG
    assert lib.ainfer_moe_stack_forward(sh, _ptr(stack.table), 3, L.NORM_PLAIN, 1e-6, _ptr(r),
                                        _ptr(r), 2, _ptr(ws), ws.numel(), _stream(None)) == L.ERR_ARG
    assert lib.ainfer_moe_stack_workspace_bytes(sh, 5, 2) >= lib.ainfer_moe_workspace_bytes(sh, 5)
    assert lib.ainfer_moe_stack_workspace_bytes(sh, L.MAX_TOKENS + 1, 2) == 0
    assert lib.ainfer_moe_stack_workspace_bytes(sh, 1, 0) == 0
    arr = (L.Weights * 1)(layers[0].weights)
    assert lib.ainfer_moe_stack_prepare(sh, arr, None, 1, _ptr(stack.table), 16, None) == L.ERR_ARG
    assert lib.ainfer_moe_stack_prepare(sh, arr, None, 0, _ptr(stack.table), 4096, None) == L.ERR_ARG
    bad = L.Weights.from_buffer_copy(layers[0].weights)
    bad.w_down = None
    arr2 = (L.Weights * 1)(bad)
    assert lib.ainfer_moe_stack_prepare(sh, arr2, None, 1, _ptr(stack.table), 4096,
                                        None) == L.ERR_NULL
    torch.cuda.synchronize()
    assert not _bits(r).any(), "rejected calls must not write"


def test_stack_wait_timeout_is_visible(torch, oracle, c4_stack):
    """With the spin limit at 0 every bounded wait of the stack kernel gives
    up at once: the kernel still ends, every output row is NaN and
    workspace_check reports AINFER_ERR_SYNC; after workspace_init the stack
    is exact again."""
    import ctypes as C
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, make_input, _ptr, _stream
    cfg, layers, norm_ws = c4_stack
    stack = MoeStack(layers[:2], norm_ws[:2])
    T = 2
    ws = stack.workspace(T)
    r0 = (make_input(cfg, T, tag=6400) * 4).contiguous()
    out = torch.zeros_like(r0)
    try:
        L.check(L.lib().ainfer_moe_debug_spin_limit(0))
        print("[case] stack forced timeout", flush=True)
        stack.forward(r0, out, ws, persistent=True)
        torch.cuda.synchronize()
    finally:
        L.check(L.lib().ainfer_moe_debug_spin_limit(1 << 20))
    assert torch.isnan(out.float()).all()
    assert layers[0].workspace_check(ws) == L.ERR_SYNC
    L.check(L.lib().ainfer_moe_workspace_init(C.byref(layers[0].shape), _ptr(ws), ws.numel(),
                                              _stream(None)))
    want = _chain(layers[:2], r0, layers[0].workspace(T), norm_ws[:2], L.NORM_PLAIN)
    stack.forward(r0, out, ws, persistent=True)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(want))
