"""Chunked prefill: calls above AINFER_MOE_CHUNK_TOKENS (4096) tokens run as
consecutive chunks on one chunk-sized workspace.  Config 2's layer (Zipf(1.1)
routing) at T = 8192 and 16384 (and a ragged 9000): the routing of every token
is bit-exact against the oracle (it is per token, so chunking cannot change
it), a sample of output rows is within the layer tolerance of the oracle,
each chunk's rows equal a separate call on that chunk bit for bit (the chunk
plan is exactly consecutive independent calls), and the workspace does not
grow past one chunk."""
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


def test_workspace_stops_growing_at_one_chunk(torch):
    from ainfer_amd import _lib as L
    layer = get_layer(torch, "c2")
    lib = L.lib()
    sh = C.byref(layer.shape)
    chunk = lib.ainfer_moe_workspace_bytes(sh, 4096)
    assert lib.ainfer_moe_workspace_bytes(sh, 4095) < chunk
    for T in (4097, 8192, 16384, L.MAX_TOKENS):
        assert lib.ainfer_moe_workspace_bytes(sh, T) == chunk, T


# 4097 and 4100 end on a 1- and 4-token chunk, which runs the decode path
# (shared sync words, folded RMSNorm) on a workspace a 4096-token chunk just used
@pytest.mark.parametrize("T", [4097, 4100, 8192, 9000, 16384])
def test_chunked_prefill_parity(torch, oracle, T):
    from ainfer_amd.moe import make_input
    print(f"[case] chunked prefill c2 T={T}", flush=True)
    layer = get_layer(torch, "c2")
    cfg = layer.cfg
    x = make_input(cfg, T, tag=9100 + T)
    ws = layer.workspace(T)
    y = torch.full((T, cfg.hidden), float("nan"), dtype=torch.bfloat16, device="cuda")
    layer.forward(x, y, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    hl = host_copy(oracle, layer)
    xh = to_np(x)
    # routing of every token, bit-exact (the route entry chunks the same way)
    idx, w, sg, lg = layer.route(x, ws, want_logits=True)
    torch.cuda.synchronize()
    r_idx, r_w, r_sg, r_lg = hl.route(xh, T)
    assert np.array_equal(to_np(lg).view(np.uint32), r_lg.view(np.uint32)), "logits"
    assert np.array_equal(to_np(idx), r_idx), "top-k indices"
    np.testing.assert_allclose(to_np(w), r_w, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(to_np(sg), r_sg, rtol=2e-6, atol=1e-7)
    # a sample of rows from every chunk, including each chunk's first and last
    rng = np.random.default_rng(T)
    rows = set(rng.choice(T, size=64, replace=False).tolist())
    for c0 in range(0, T, 4096):
        rows |= {c0, min(c0 + 4095, T - 1)}
    rows = np.array(sorted(rows))
    ref = hl.forward(np.ascontiguousarray(xh[rows]), len(rows))
    check_close(to_np(y)[rows], ref, f"c2 T={T} sample")
    # each chunk equals a call on that chunk alone
    for c0 in range(0, T, 4096):
        n = min(4096, T - c0)
        yc = torch.empty(n, cfg.hidden, dtype=torch.bfloat16, device="cuda")
        layer.forward(x[c0:c0 + n].contiguous(), yc, ws)
        torch.cuda.synchronize()
        assert torch.equal(yc.view(torch.int16), y[c0:c0 + n].view(torch.int16)), (T, c0)


@pytest.mark.parametrize("T", [4097, 4100, 8200])
def test_chunked_block_forward_in_place(torch, T):
    """block_forward (RMSNorm + layer + residual) chunks the same way, also
    with resid_out == resid_in."""
    from ainfer_amd.moe import make_input
    print(f"[case] chunked block_forward c2 T={T}", flush=True)
    layer = get_layer(torch, "c2")
    cfg = layer.cfg
    r0 = make_input(cfg, T, tag=9300) * 3
    ws = layer.workspace(T)
    out = torch.empty_like(r0)
    layer.block_forward(r0, out, ws)
    r = r0.clone()
    layer.block_forward(r, r, ws)
    parts = []
    for c0 in range(0, T, 4096):
        n = min(4096, T - c0)
        o = torch.empty(n, cfg.hidden, dtype=torch.bfloat16, device="cuda")
        layer.block_forward(r0[c0:c0 + n].contiguous(), o, ws)
        parts.append(o)
    torch.cuda.synchronize()
    whole = torch.cat(parts)
    assert torch.equal(out.view(torch.int16), whole.view(torch.int16))
    assert torch.equal(r.view(torch.int16), whole.view(torch.int16))
    assert torch.isfinite(out.float()).all()


def test_dispatch_rejects_more_than_a_chunk(torch):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import _ptr, _stream
    layer = get_layer(torch, "c2")
    lib = L.lib()
    T = 4097
    ws = layer.workspace(T)
    idx = torch.zeros(T, layer.cfg.top_k, dtype=torch.int32, device="cuda")
    E = layer.cfg.n_experts
    buf = [torch.zeros(n, dtype=torch.int32, device="cuda") for n in (E, E + 1, T * 10, T * 10)]
    assert lib.ainfer_moe_dispatch(C.byref(layer.shape), _ptr(idx), T, *[_ptr(b) for b in buf],
                                   _ptr(ws), ws.numel(), _stream(None)) == L.ERR_TOKENS
