"""W4A8 entries (the reference's production GEMV numerics) vs the CPU
oracle, through the C ABI.  Bar: int8 codes, scales and GEMV outputs
bit-exact (the reference's own test allows 1e-6 relative,
tools/cmdlist/gemv_replay.cpp:250-261)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _p(t):
    return C.c_void_p(t.data_ptr())


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_act_quant(torch, x_np, dtype):
    from ainfer_amd import _lib as L
    T, K = x_np.shape
    x = _dev(torch, x_np.view(np.int16) if dtype == L.ACT_BF16 else x_np)
    q = torch.empty(T, K, dtype=torch.int8, device="cuda")
    sq = torch.empty(T, K // 128, dtype=torch.float32, device="cuda")
    L.check(L.lib().ainfer_moe_act_quant_i8(_p(x), dtype, T, K, _p(q), _p(sq), None))
    torch.cuda.synchronize()
    return q.cpu().numpy(), sq.cpu().numpy()


def gpu_gemv(torch, packed, scales, sdt, q, sq, M, K):
    from ainfer_amd import _lib as L
    T = q.shape[0]
    dp, ds = _dev(torch, packed), _dev(torch, scales.view(np.int16))
    dq, dsq = _dev(torch, q), _dev(torch, sq)
    y = torch.full((T, M), float("nan"), dtype=torch.float32, device="cuda")
    L.check(L.lib().ainfer_moe_int4_gemv_i8(_p(dp), _p(ds), sdt, _p(dq), _p(dsq), M, K, T,
                                            _p(y), None))
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("T,K", [(1, 128), (5, 1024), (16, 5120), (33, 2048)])
def test_act_quant_bit_exact(torch, oracle, T, K):
    from ainfer_amd import _lib as L
    print(f"[case] act_quant T={T} K={K}", flush=True)
    rng = np.random.default_rng(T * 7 + K)
    x = (rng.standard_normal((T, K)) * rng.choice([1e-4, 1, 50], (T, 1))).astype(np.float32)
    x[0, :128] = 0                                  # zero group -> scale 1
    x[-1, 5] = 127 * 4.0                            # exact halves after the division
    x[-1, 6:9] = [2.0, -2.0, 6.0]
    for dtype in (L.ACT_F32, L.ACT_BF16):
        xin = oracle.f32_to_bf16(x) if dtype == L.ACT_BF16 else x
        q, sq = gpu_act_quant(torch, xin, dtype)
        rq, rsq = oracle.act_quant_i8(xin)
        assert np.array_equal(sq.view(np.uint32), rsq.view(np.uint32)), dtype
        assert np.array_equal(q, rq), dtype


@pytest.mark.parametrize("M,K,T,sdt", [(16, 128, 1, 0), (100, 1024, 5, 1), (512, 2048, 16, 1),
                                       (2048, 512, 17, 0), (77, 384, 40, 0),
                                       # T = 1: 1 to 4 chunks per lane, partial last
                                       # chunk round, rows past a wave's end
                                       (101, 1024, 1, 1), (333, 5120, 1, 1), (70, 8192, 1, 0),
                                       (50, 2176, 1, 0), (19, 8320, 1, 1)])
def test_int4_gemv_i8_bit_exact(torch, oracle, M, K, T, sdt):
    print(f"[case] gemv_i8 M={M} K={K} T={T} sdt={sdt}", flush=True)
    rng = np.random.default_rng(M + K + T)
    packed = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    sf = np.abs(rng.standard_normal(M * K // 128) * 0.02).astype(np.float32)
    scales = oracle.f32_to_bf16(sf) if sdt == 0 else sf.astype(np.float16).view(np.uint16)
    x = (rng.standard_normal((T, K)) * 3).astype(np.float32)
    q, sq = oracle.act_quant_i8(x)
    y = gpu_gemv(torch, packed, scales, sdt, q, sq, M, K)
    ref = oracle.int4_gemv_i8(packed, scales, sdt, q, sq, M, K)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_int4_gemv_i8_on_the_reference_test_inputs(torch, oracle):
    """The reference's own GEMV test: M=17408, K=5120, its LCG weights and
    activations (gemv_replay.cpp:57,158-204), quantised on the GPU; the
    reference allows 1e-6 relative, this asserts bit equality."""
    from ainfer_amd import _lib as L
    M, K, nv = 17408, 5120, 3
    print(f"[case] gemv_i8 reference inputs M={M} K={K}", flush=True)
    packed, scales, x = oracle.ref_gemv_inputs(M, K, nv)
    q, sq = gpu_act_quant(torch, x, L.ACT_F32)
    rq, rsq = oracle.act_quant_i8(x)
    assert np.array_equal(q, rq) and np.array_equal(sq, rsq)
    y = gpu_gemv(torch, packed, scales, 0, q, sq, M, K)
    ref = oracle.int4_gemv_i8(packed, scales, 0, rq, rsq, M, K)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_w4a8_argument_errors(torch):
    from ainfer_amd import _lib as L
    lib = L.lib()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = _p(buf)
    assert lib.ainfer_moe_act_quant_i8(p, 0, 1, 100, p, p, None) == L.ERR_SHAPE
    assert lib.ainfer_moe_act_quant_i8(p, 7, 1, 128, p, p, None) == L.ERR_ARG
    assert lib.ainfer_moe_act_quant_i8(None, 0, 1, 128, p, p, None) == L.ERR_NULL
    assert lib.ainfer_moe_act_quant_i8(p, 0, 0, 128, p, p, None) == L.OK
    assert lib.ainfer_moe_int4_gemv_i8(p, p, 0, p, p, 0, 128, 1, p, None) == L.ERR_SHAPE
    assert lib.ainfer_moe_int4_gemv_i8(p, p, 2, p, p, 16, 128, 1, p, None) == L.ERR_ARG
    odd = C.c_void_p(buf.data_ptr() + 8)
    assert lib.ainfer_moe_int4_gemv_i8(odd, p, 0, p, p, 16, 128, 1, p, None) == L.ERR_ARG
