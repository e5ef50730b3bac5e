"""The MoE layer in W4A8 (AINFER_PRECISION_W4A8: per-group int8 activations,
Int4Gemv products, SiluMul and the combine in fp32) against the oracle's W4A8
layer (mo_forward_w4a8, built from the ScalesMax/Quantize and Int4Gemv
restatements that tests/test_gpu_w4a8.py pins bit for bit): routing and
dispatch bit-exact (as W4A16), outputs within the layer tolerance, and most
output elements bit-identical (only an act element whose SiluMul exp differs
by an ulp between the device and libm can move a quantised value).  Also
block_forward in W4A8 against the oracle's RMSNorm + W4A8 layer + residual,
the W4A8 and W4A16 layers close to each other, and the stack entry refusing
W4A8."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_parity import check_close, get_layer, host_copy, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


CASES = [("c0", 1), ("c0", 5), ("c1", 1), ("c1", 4), ("c1", 8), ("c1", 16), ("c1", 300), ("c2", 4096),
         ("c3", 1), ("c3", 2)]


@pytest.mark.parametrize("name,T", CASES)
def test_w4a8_layer_parity(torch, oracle, name, T):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input, with_precision
    print(f"[case] w4a8 {name} T={T}", flush=True)
    base = get_layer(torch, name)
    layer = with_precision(base, L.PRECISION_W4A8)
    cfg = base.cfg
    x = make_input(cfg, T, tag=7700 + T)
    ws = layer.workspace(T)
    y = torch.full((T, cfg.hidden), float("nan"), dtype=torch.bfloat16, device="cuda")
    layer.forward(x, y, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    hl = host_copy(oracle, base)
    xh = to_np(x)
    rows = np.arange(T)
    if T > 64:  # tokens are independent given their routing: a sample
        rng = np.random.default_rng(T)
        rows = np.sort(rng.choice(T, size=48, replace=False))
        rows[0], rows[-1] = 0, T - 1
    ref = hl.forward_w4a8(np.ascontiguousarray(xh[rows]), len(rows))
    got = to_np(y)[rows]
    check_close(got, ref, f"w4a8 {name} T={T}")
    exact = np.mean(got == oracle.f32_to_bf16(ref))
    print(f"[parity] w4a8 {name} T={T}: {100 * exact:.2f}% of outputs bit-identical", flush=True)
    assert exact > 0.9
    # deterministic, and close to the W4A16 layer
    y2 = torch.empty_like(y)
    layer.forward(x, y2, ws)
    y16 = torch.empty_like(y)
    base.forward(x, y16, base.workspace(T))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    a, b = y.float(), y16.float()
    cos = float((a * b).sum() / (a.norm() * b.norm()))
    assert cos > 0.999, cos


@pytest.mark.parametrize("Is", [1024, 256, 0])
def test_w4a8_layer_one_token_shared_widths(torch, oracle, Is):
    """T = 1 runs the one-token expert GEMVs (k_w4a8_expert_t1): a shared
    expert wider, narrower than the routed ones, or none."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input, with_precision
    print(f"[case] w4a8 c1 T=1 Is={Is}", flush=True)
    base = get_layer(torch, "c1", shared_inter=Is)
    layer = with_precision(base, L.PRECISION_W4A8)
    x = make_input(base.cfg, 1, tag=7900 + Is)
    ws = layer.workspace(1)
    y = torch.full((1, base.cfg.hidden), float("nan"), dtype=torch.bfloat16, device="cuda")
    layer.forward(x, y, ws)
    torch.cuda.synchronize()
    ref = host_copy(oracle, base).forward_w4a8(to_np(x), 1)
    got = to_np(y)
    check_close(got, ref, f"w4a8 c1 T=1 Is={Is}")
    assert np.mean(got == oracle.f32_to_bf16(ref)) > 0.9


def test_w4a8_block_forward(torch, oracle):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input, with_precision
    base = get_layer(torch, "c1")
    layer = with_precision(base, L.PRECISION_W4A8)
    cfg = base.cfg
    g = torch.Generator().manual_seed(3)
    nw = (torch.randn(cfg.hidden, generator=g) * 0.2).to(torch.bfloat16).cuda()
    hl = host_copy(oracle, base)
    for T in (1, 3, 17):
        print(f"[case] w4a8 block T={T}", flush=True)
        r = make_input(cfg, T, tag=7800 + T) * 3
        ws = layer.workspace(T)
        out = torch.empty_like(r)
        layer.block_forward(r, out, ws, norm_w=nw, norm_mode=L.NORM_ONE_PLUS)
        torch.cuda.synchronize()
        rh = to_np(r)
        h = oracle.rmsnorm_bf16(rh, to_np(nw), L.NORM_ONE_PLUS)
        y = hl.forward_w4a8(np.ascontiguousarray(h), T)
        want = oracle.bf16_to_f32(rh) + y
        check_close(to_np(out), want, f"w4a8 block T={T}")


def test_w4a8_shape_rules(torch):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, with_precision, _ptr, _stream
    base = get_layer(torch, "c1")
    s = L.Shape.from_buffer_copy(base.shape)
    s.precision = 2
    assert L.lib().ainfer_moe_validate(C.byref(s)) == L.ERR_SHAPE
    layer = with_precision(base, L.PRECISION_W4A8)
    n16 = L.lib().ainfer_moe_workspace_bytes(C.byref(base.shape), 16)
    n8 = L.lib().ainfer_moe_workspace_bytes(C.byref(layer.shape), 16)
    assert n8 > n16
    # the stack replays W4A8 blocks as the block entry runs them; the
    # persistent one-launch form has W4A16 items only
    assert L.lib().ainfer_moe_stack_workspace_bytes(C.byref(layer.shape), 1, 1) == \
        L.lib().ainfer_moe_workspace_bytes(C.byref(layer.shape), 1)
    from ainfer_amd.moe import make_input
    w8 = [layer, with_precision(get_layer(torch, "c1"), L.PRECISION_W4A8)]
    stack = MoeStack(w8)
    for T in (1, 8):
        ws = stack.workspace(T)
        r0 = (make_input(base.cfg, T, tag=7700 + T) * 2).contiguous()
        want = r0.clone()
        for ly in w8:
            ly.block_forward(want, want, w8[0].workspace(T))
        out = torch.empty_like(r0)
        stack.forward(r0, out, ws)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), T
        assert L.lib().ainfer_moe_stack_forward_persistent(
            C.byref(layer.shape), _ptr(stack.table), 2, L.NORM_PLAIN, 1e-6, _ptr(r0), _ptr(out), T,
            _ptr(ws), ws.numel(), _stream(None)) == (L.ERR_SHAPE if T == 1 else L.ERR_TOKENS)


@pytest.mark.parametrize("name", ["c1", "c3"])
def test_w4a8_one_token_equals_batched_rows(torch, name):
    """At T = 1 the down GEMV blocks quantize act into their LDS themselves;
    at T = 2 a quantization launch does it.  Tokens are independent and both
    GEMV forms sum the same terms in group order, so each token's row of a
    T = 2 call is bit-identical to a T = 1 call on that token."""
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input, with_precision
    base = get_layer(torch, name)
    layer = with_precision(base, L.PRECISION_W4A8)
    x = make_input(base.cfg, 2, tag=7800)
    ws = layer.workspace(2)
    y2 = torch.empty_like(x)
    layer.forward(x, y2, ws)
    for t in range(2):
        print(f"[case] w4a8 {name} one token {t}", flush=True)
        y1 = torch.empty_like(x[t:t + 1])
        layer.forward(x[t:t + 1].contiguous(), y1, ws)
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), y2[t:t + 1].view(torch.int16)), (name, t)
