"""The no-allocation block entry (static per-GPU scratch) against the
workspace entry: bit-identical outputs on two calls in a row, the second with
fewer tokens, in place and out of place, in both RMSNorm placements (folded
into decode routing at T <= 4, separate kernel above), and the size limit.
Runs last: it also holds when earlier tests left the scratch dirty."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _pair(torch, layer, r, nw, mode):
    """(workspace entry, no-alloc entry) outputs on resid r, out of place."""
    ws = layer.workspace(r.shape[0])
    a = torch.empty_like(r)
    b = torch.empty_like(r)
    layer.block_forward(r, a, ws, norm_w=nw, norm_mode=mode)
    layer.block_forward_noalloc(r, b, norm_w=nw, norm_mode=mode)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("name,Ts", [("c1", (16, 4, 1)), ("c3", (64, 8, 2))])
def test_noalloc_matches_workspace_entry(torch, name, Ts):
    import test_gpu_parity as P
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    layer = P.get_layer(torch, name)
    H = layer.cfg.hidden
    g = torch.Generator().manual_seed(5)
    nw = (torch.randn(H, generator=g) * 0.3).to(torch.bfloat16).cuda()
    for i, T in enumerate(Ts):
        mode = L.NORM_ONE_PLUS if i % 2 else L.NORM_PLAIN
        w = nw if i % 2 else None
        print(f"[case] noalloc {name} T={T} mode={mode}", flush=True)
        r = (make_input(layer.cfg, T, tag=7100 + T) * 3).contiguous()
        a, b = _pair(torch, layer, r, w, mode)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (name, T)
        assert not torch.isnan(b.float()).any()
        # in place: resid_out == resid_in
        rr = r.clone()
        layer.block_forward_noalloc(rr, rr, norm_w=w, norm_mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(rr.view(torch.int16), a.view(torch.int16)), (name, T, "in place")


def test_noalloc_rejects_calls_beyond_the_scratch(torch):
    import ctypes as C
    import test_gpu_parity as P
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import make_input
    layer = P.get_layer(torch, "c1")
    lib = L.lib()
    ok_T = max(T for T in range(1, 1024)
               if lib.ainfer_moe_workspace_bytes(C.byref(layer.shape), T) <= L.NOALLOC_SCRATCH_BYTES)
    big = ok_T + 1
    r = make_input(layer.cfg, big, tag=7300)
    out = torch.zeros_like(r)
    with pytest.raises(L.MoeError, match="static scratch"):
        layer.block_forward_noalloc(r, out)
    torch.cuda.synchronize()
    assert not out.view(torch.int16).any(), "a rejected call must not write"
    # the largest accepted size still works and matches
    a, b = _pair(torch, layer, r[:ok_T].contiguous(), None, L.NORM_PLAIN)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
