"""The MFMA-rate probe (ainfer_moe_mfma_probe) on the GPU: a positive rate
below the bf16 spec peak (plus margin), and VALU work between the MFMAs does
not make the loop faster."""
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
