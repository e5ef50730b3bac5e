"""Strict mode (ainfer_moe_set_strict): with the bounded device-side waits
made to run out from the host (spin limit 0, every kernel still exits
normally), the decode entry points return AINFER_ERR_SYNC instead of
AINFER_OK with NaN rows; the error word stays set (so later calls on the
workspace report it too) until ainfer_moe_workspace_init, after which the
same calls return AINFER_OK with the oracle-checked outputs of the other
tests.  Strict off, the same failing calls return AINFER_OK (the default
contract: the failure shows in the rows and in ainfer_moe_workspace_check)."""
import ctypes as C

import pytest

from test_gpu_parity import get_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def test_strict_reports_wait_timeouts(torch):
    from ainfer_amd import _lib as L
    from ainfer_amd.moe import MoeStack, _ptr, _stream, make_input
    lib = L.lib()
    layer = get_layer(torch, "c1")
    cfg = layer.cfg
    sh = C.byref(layer.shape)
    T = 1
    stack = MoeStack([layer, layer])
    ws = stack.workspace(T)
    x = make_input(cfg, T, tag=7700)
    y = torch.empty_like(x)

    def fwd():
        return lib.ainfer_moe_forward(sh, C.byref(layer.weights), _ptr(x), _ptr(y), T, _ptr(ws),
                                      ws.numel(), _stream(None))

    def blk():
        return lib.ainfer_moe_block_forward(sh, C.byref(layer.weights), None, L.NORM_PLAIN, 1e-6,
                                            _ptr(x), _ptr(y), T, _ptr(ws), ws.numel(), _stream(None))

    def stk(pers):
        f = lib.ainfer_moe_stack_forward_persistent if pers else lib.ainfer_moe_stack_forward
        return f(sh, _ptr(stack.table), 2, L.NORM_PLAIN, 1e-6, _ptr(x), _ptr(y), T, _ptr(ws),
                 ws.numel(), _stream(None))

    def reinit():
        L.check(lib.ainfer_moe_workspace_init(sh, _ptr(ws), ws.numel(), _stream(None)))
        torch.cuda.synchronize()

    try:
        print("[case] strict: forced timeouts", flush=True)
        L.check(lib.ainfer_moe_debug_spin_limit(0))
        # strict off: the default contract
        assert fwd() == L.OK
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all()
        assert layer.workspace_check(ws) == L.ERR_SYNC
        reinit()
        L.check(lib.ainfer_moe_set_strict(1))
        for call in (fwd, blk, lambda: stk(False), lambda: stk(True)):
            assert call() == L.ERR_SYNC
            reinit()
        # the error word is sticky: a later call whose waits all succeed
        # still reports the earlier one's timeout
        assert fwd() == L.ERR_SYNC
        L.check(lib.ainfer_moe_debug_spin_limit(1 << 20))
        assert fwd() == L.ERR_SYNC
        reinit()
        print("[case] strict: normal calls", flush=True)
        for call in (fwd, blk, lambda: stk(False), lambda: stk(True)):
            assert call() == L.OK
            assert bool(torch.isfinite(y.float()).all())
        want = torch.empty_like(y)
        L.check(lib.ainfer_moe_set_strict(0))
        layer.forward(x, want, ws)
        L.check(lib.ainfer_moe_set_strict(1))
        assert fwd() == L.OK
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    finally:
        lib.ainfer_moe_set_strict(0)
        lib.ainfer_moe_debug_spin_limit(1 << 20)
        torch.cuda.synchronize()
    assert layer.workspace_check(ws) == L.OK
