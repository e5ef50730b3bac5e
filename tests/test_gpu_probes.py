"""The measurement probes on the GPU: the MFMA-rate probe
(ainfer_moe_mfma_probe) gives a positive rate below the bf16 spec peak (plus
margin), and VALU work between the MFMAs does not make the loop faster; the
read-roof probe (ainfer_moe_read_probe) gives a positive rate below the HBM
spec and checks its arguments."""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def test_mfma_probe_rates(torch):
    from ainfer_amd import _lib as L
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rates = {}
    for nv in (0, 4):
        r = C.c_float()
        assert L.lib().ainfer_moe_mfma_probe(nv, 2, 500, s, C.byref(r)) == L.OK
        rates[nv] = r.value
    assert 0 < rates[4] <= rates[0] * 1.05, rates
    assert rates[0] < 2500 * 1.2, rates


def test_read_probe_rate_and_arguments(torch):
    """The read-roof probe (ainfer_moe_read_probe): a positive rate below
    the 8 TB/s spec over 1 GiB of random bytes, the buffer's bytes left as
    they were (the fold is never stored for this data), and the argument
    checks."""
    from ainfer_amd import _lib as L
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    n = 1 << 30
    g = torch.Generator(device="cuda").manual_seed(3)
    buf = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    before = buf[:4096].clone()
    r = C.c_float()
    lib = L.lib()
    assert lib.ainfer_moe_read_probe(C.c_void_p(buf.data_ptr()), n, 4, 2, 3, s, C.byref(r)) == L.OK
    torch.cuda.synchronize()
    assert 0 < r.value < 8000 * 1.05, r.value
    assert torch.equal(buf[:4096], before)
    p = C.c_void_p(buf.data_ptr())
    assert lib.ainfer_moe_read_probe(p, n, 3, 2, 3, s, C.byref(r)) == L.ERR_ARG     # unroll
    assert lib.ainfer_moe_read_probe(p, n, 4, 0, 3, s, C.byref(r)) == L.ERR_ARG     # blocks/CU
    assert lib.ainfer_moe_read_probe(p, n - 8, 4, 2, 3, s, C.byref(r)) == L.ERR_ARG  # size % 16
    assert lib.ainfer_moe_read_probe(C.c_void_p(buf.data_ptr() + 8), 1024, 4, 2, 3, s,
                                     C.byref(r)) == L.ERR_ARG                        # alignment
    assert lib.ainfer_moe_read_probe(p, n, 4, 2, 0, s, C.byref(r)) == L.ERR_ARG     # iters
    assert lib.ainfer_moe_read_probe(None, n, 4, 2, 3, s, C.byref(r)) == L.ERR_ARG
