"""Config 4 at its full depth: the 60-layer decode step (200 GB of weights
resident) through ainfer_moe_stack_forward at T = 1 and T = 8.  The step
equals 60 chained ainfer_moe_block_forward calls bit for bit and stays
finite; and at layers 0, 20, 40 and 59 the residual the stack carries into
the layer is fed to the oracle's block (teacher forcing): the layer's top-k
is bit-identical to the oracle's and its output is within the layer
tolerance of the oracle's block on the same input, as is the MoE output
alone on the normalized input."""
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
def c4_all(torch):
    import test_gpu_parity as P
    from ainfer_amd.moe import MoeLayer
    from ainfer_amd.synthetic import CONFIGS
    P._layers.clear()
    torch.cuda.empty_cache()
    cfg = CONFIGS["c4"]
    print(f"[case] c4 depth: allocating {cfg.layers} layers", flush=True)
    layers = [MoeLayer(cfg, layer=i) for i in range(cfg.layers)]
    torch.cuda.synchronize()
    yield cfg, layers
    del layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 8])
def test_c4_sixty_layer_step(torch, oracle, c4_all, T):
    from ainfer_amd.moe import MoeStack, make_input, rmsnorm
    cfg, layers = c4_all
    stack = MoeStack(layers)
    ws = stack.workspace(T)
    x0 = (make_input(cfg, T, tag=8800 + T) * 4).contiguous()
    out = torch.empty_like(x0)
    stack.forward(x0, out, ws)
    chained = x0.clone()
    wsb = layers[0].workspace(T)
    for ly in layers:
        ly.block_forward(chained, chained, wsb)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out.view(torch.int16), chained.view(torch.int16))
    for l in (0, 20, 40, 59):
        print(f"[case] c4 depth T={T} layer {l}", flush=True)
        r_in = x0.clone()
        if l:
            MoeStack(layers[:l]).forward(x0, r_in, ws)
        r_out = torch.empty_like(r_in)
        MoeStack(layers[:l + 1]).forward(x0, r_out, ws)
        h = torch.empty_like(r_in)
        rmsnorm(r_in, h)
        idx, _, _, _ = layers[l].route(h, wsb)
        torch.cuda.synchronize()
        hl = host_copy(oracle, layers[l])
        r_idx, _, _, _ = hl.route(to_np(h), T)
        assert np.array_equal(to_np(idx), r_idx), (T, l)
        want = hl.block_forward(to_np(r_in), T)
        check_close(to_np(r_out), oracle.bf16_to_f32(want), f"c4 depth T={T} layer {l}")
        # the layer's own output on that normalized input (the residual, which
        # grows with depth, does not mask it here)
        y = torch.empty_like(h)
        layers[l].forward(h, y, wsb)
        torch.cuda.synchronize()
        check_close(to_np(y), hl.forward(to_np(h), T), f"c4 depth T={T} layer {l} MoE output")
        del hl
