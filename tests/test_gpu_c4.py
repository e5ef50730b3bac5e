"""Config 4 at its own shape (H4096, E512, top-10, I1024 + shared): chained
blocks with independent layers through both RMSNorm placements (folded into
the decode routing kernel at T <= 4, the separate kernel above), in place
(resid_out == resid_in) and out of place, against the oracle's block; and
the decode path's bounded waits made to run out from the host, which must
show up as NaN outputs and AINFER_ERR_SYNC until the workspace is re-inited.
"""
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


@pytest.fixture(scope="module")
def c4_layers(torch, oracle):
    import test_gpu_parity as P
    from ainfer_amd.moe import MoeLayer
    from ainfer_amd.synthetic import CONFIGS
    P._layers.clear()
    torch.cuda.empty_cache()
    cfg = CONFIGS["c4"]
    layers = [MoeLayer(cfg, layer=i) for i in (0, 17, 59)]
    torch.cuda.synchronize()
    hls = [host_copy(oracle, L) for L in layers]
    yield cfg, layers, hls
    del layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 3, 4, 8])
def test_c4_chained_blocks_real_shape(torch, oracle, c4_layers, T):
    """Three independent c4 layers chained, per block: the in-place call
    (the integration guide's usage) equals the out-of-place call bit for bit,
    and both match the oracle's block on the same input.  Block 1 uses a
    (1+w) norm weight, the others unit weight.  At T = 3 and 4 (RMSNorm in
    the routing kernel, E = 512 variant) each token's output also equals the
    T = 17 call's (separate RMSNorm kernel, MFMA router + exact refine) bit
    for bit, which pins the folded norm and its routing exactly."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    cfg, layers, hls = c4_layers
    g = torch.Generator().manual_seed(11)
    nw = (torch.randn(cfg.hidden, generator=g) * 0.3).to(torch.bfloat16).cuda()
    ws = layers[0].workspace(17)
    base = make_input(cfg, 17, tag=4000 + T) * 4
    r = base[:T].contiguous()
    for i, (layer, hl) in enumerate(zip(layers, hls)):
        print(f"[case] c4 block {i} T={T}", flush=True)
        norm = (nw, L.NORM_ONE_PLUS) if i == 1 else (None, L.NORM_PLAIN)
        inp = r.clone()
        out = torch.empty_like(r)
        layer.block_forward(inp, out, ws, norm_w=norm[0], norm_mode=norm[1])
        layer.block_forward(r, r, ws, norm_w=norm[0], norm_mode=norm[1])     # aliased
        torch.cuda.synchronize()
        assert torch.equal(r.view(torch.int16), out.view(torch.int16)), "in-place differs"
        want = hl.block_forward(to_np(inp), T, norm_w=None if norm[0] is None else to_np(norm[0]),
                                mode=norm[1])
        check_close(to_np(out), oracle.bf16_to_f32(want), f"c4 block {i} T={T}")
        if T in (3, 4):
            big = torch.cat([inp, base[T:]]).contiguous()
            o17 = torch.empty_like(big)
            layer.block_forward(big, o17, ws, norm_w=norm[0], norm_mode=norm[1])
            torch.cuda.synchronize()
            assert torch.equal(o17[:T].view(torch.int16), out.view(torch.int16)), \
                f"block {i}: folded RMSNorm path differs from the T=17 path"
    assert layers[0].workspace_check(ws) == L.OK


@pytest.mark.parametrize("T", [1, 2, 16])
def test_c1_block_in_place(torch, oracle, T):
    """block_forward(r, r) is bit-identical to block_forward(r', out) with r'
    a copy, on the fused expert kernel (T <= 2) and the staged path."""
    from ainfer_amd.moe import make_input
    import test_gpu_parity as P
    layer = P.get_layer(torch, "c1")
    ws = layer.workspace(T)
    r = make_input(layer.cfg, T, tag=600 + T) * 2
    inp = r.clone()
    out = torch.empty_like(r)
    layer.block_forward(inp, out, ws)
    layer.block_forward(r, r, ws)
    torch.cuda.synchronize()
    assert torch.equal(r.view(torch.int16), out.view(torch.int16))


def test_decode_wait_timeout_is_visible(torch, oracle):
    """With the spin limit at 0 every bounded device wait of the decode path
    gives up at once (no kernel waits or faults): the outputs of that call
    and of every later call on the workspace are NaN, workspace_check reports
    AINFER_ERR_SYNC, and after workspace_init normal calls are exact again."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    import test_gpu_parity as P
    layer = P.get_layer(torch, "c1")
    H = layer.cfg.hidden
    ws = layer.workspace(300)
    x = make_input(layer.cfg, 16, tag=321)
    try:
        L.check(L.lib().ainfer_moe_debug_spin_limit(0))
        for T in (1, 2, 16):
            print(f"[case] forced timeout T={T}", flush=True)
            y = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
            layer.forward(x[:T].contiguous(), y, ws)
            torch.cuda.synchronize()
            assert torch.isnan(y.float()).all(), T
    finally:
        L.check(L.lib().ainfer_moe_debug_spin_limit(1 << 20))
    assert layer.workspace_check(ws) == L.ERR_SYNC
    # sticky: a later call, also on the prefill path, is still NaN
    x300 = make_input(layer.cfg, 300, tag=322)
    y = torch.zeros(300, H, dtype=torch.bfloat16, device="cuda")
    layer.forward(x300, y, ws)
    torch.cuda.synchronize()
    assert torch.isnan(y.float()).all()
    # re-init clears it
    from ainfer_amd.moe import _ptr, _stream
    import ctypes as C
    L.check(L.lib().ainfer_moe_workspace_init(C.byref(layer.shape), _ptr(ws), ws.numel(),
                                              _stream(None)))
    assert layer.workspace_check(ws) == L.OK
    hl = host_copy(oracle, layer)
    for T in (1, 2, 16):
        y = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
        layer.forward(x[:T].contiguous(), y, ws)
        torch.cuda.synchronize()
        check_close(to_np(y), hl.forward(to_np(x[:T].contiguous()), T), f"after re-init T={T}")
    assert layer.workspace_check(ws) == L.OK
