"""The layer and stack entry points enqueue kernels only (no allocation, no host sync,
no memset), so a HIP graph can capture them: the analogue of the
reference's recorded command lists (tools/decode/decode_l0.cpp:553-677).
Each replay is checked bit for bit against the eager call, with eager work
on other inputs between replays."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("T", [1, 3, 16, 64, 300])
def test_forward_graph_replays_match_eager(torch, T):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeLayer, make_input
    from ainfer_amd.synthetic import CONFIGS
    print(f"[case] graph forward c1 T={T}", flush=True)
    cfg = CONFIGS["c1"]
    layer = MoeLayer(cfg)
    ws = layer.workspace(T)
    x = make_input(cfg, T, tag=31 + T)
    other = make_input(cfg, T, tag=77 + T)
    want = torch.empty(T, cfg.hidden, dtype=torch.bfloat16, device="cuda")
    layer.forward(x, want, ws)
    torch.cuda.synchronize()
    y = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.forward(x, y, ws, s)          # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        layer.forward(x, y, ws, s)
    scratch = torch.empty_like(want)
    for rep in range(4):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), rep
        layer.forward(other, scratch, ws)   # eager work between replays
        torch.cuda.synchronize()
    assert layer.workspace_check(ws) == L.OK
    del g


def test_block_forward_graph_replays_match_eager(torch):
    from ainfer_amd.moe import MoeLayer, make_input
    from ainfer_amd.synthetic import CONFIGS
    import dataclasses
    print("[case] graph block_forward c4-shaped, 64 experts, T=8", flush=True)
    cfg = dataclasses.replace(CONFIGS["c4"], n_experts=64, layers=1)
    layer = MoeLayer(cfg)
    T = 8
    ws = layer.workspace(T)
    r0 = make_input(cfg, T, tag=5) * 4
    want = torch.empty_like(r0)
    layer.block_forward(r0, want, ws)
    torch.cuda.synchronize()
    out = torch.empty_like(r0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.block_forward(r0, out, ws, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        layer.block_forward(r0, out, ws, stream=s)
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
        layer.block_forward(r0 * 2, torch.empty_like(r0), ws)
        torch.cuda.synchronize()
    del g


@pytest.mark.parametrize("T", [1, 8])
def test_stack_forward_graph_replays_match_eager(torch, T):
    """The replayed 3-layer stack (at T = 8 with the next RMSNorm computed in
    each combine) captured once and replayed: every replay equals the eager
    call bit for bit."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeLayer, MoeStack, make_input
    from ainfer_amd.synthetic import CONFIGS
    print(f"[case] graph stack c1 x3 T={T}", flush=True)
    cfg = CONFIGS["c1"]
    layers = [MoeLayer(cfg, layer=i) for i in range(3)]
    g0 = torch.Generator().manual_seed(5)
    norm_ws = [(torch.randn(cfg.hidden, generator=g0) * 0.3 + 0.5).to(torch.bfloat16).cuda()
               for _ in layers]
    stack = MoeStack(layers, norm_ws)
    ws = stack.workspace(T)
    r0 = (make_input(cfg, T, tag=90 + T) * 2).contiguous()
    other = (make_input(cfg, T, tag=95 + T) * 2).contiguous()
    want = torch.empty_like(r0)
    stack.forward(r0, want, ws, norm_mode=L.NORM_ONE_PLUS)
    torch.cuda.synchronize()
    out = torch.empty_like(r0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        stack.forward(r0, out, ws, norm_mode=L.NORM_ONE_PLUS, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        stack.forward(r0, out, ws, norm_mode=L.NORM_ONE_PLUS, stream=s)
    scratch = torch.empty_like(r0)
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), (T, rep)
        stack.forward(other, scratch, ws, norm_mode=L.NORM_ONE_PLUS)  # eager work between replays
        torch.cuda.synchronize()
    assert layers[0].workspace_check(ws) == L.OK
    del g, layers, stack
    torch.cuda.empty_cache()
