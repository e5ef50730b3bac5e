"""Layers loaded from a .binfer file (ainfer_binfer_load_moe_layer) run the
same bits as the layers the synthetic fill builds on the GPU: the file is
written from the oracle's host copy of the same seeded weights (config 0 and
config 1 shapes, fp16 scales, a norm weight per layer), loaded into device
arenas, and block_forward must give bit-identical outputs at T = 1, 4 and 300
(decode and staged paths), with the file's norm weight in the (1+w) form."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("name", ["c0", "c1"])
def test_binfer_layers_match_synthetic(torch, oracle, tmp_path, name):
    from ainfer_amd import _lib as L
    from ainfer_amd import binfer as B
    from ainfer_amd.moe import MoeLayer, load_binfer_layer, make_input
    from ainfer_amd.synthetic import CONFIGS
    cfg = CONFIGS[name]
    H = cfg.hidden
    arrays = []
    for l in range(2):
        a = dict(oracle.HostLayer.synthetic(cfg, layer=l).a)
        a["norm_w"] = oracle.f32_to_bf16(((np.arange(H) % 11) * 0.05 - 0.2).astype(np.float32))
        arrays.append(a)
    c = dict(hidden=H, n_experts=cfg.n_experts, top_k=cfg.top_k, inter=cfg.inter,
             shared_inter=cfg.shared_inter)
    path = tmp_path / f"{name}.binfer"
    B.write_moe(path, c, arrays)
    bf = L.BinferFile(path)
    for l in range(2):
        print(f"[case] binfer {name} layer {l}", flush=True)
        fl, nw = load_binfer_layer(bf, l)
        assert nw is not None
        ref = MoeLayer(cfg, layer=l)
        nw_ref = torch.from_numpy(arrays[l]["norm_w"].view(np.int16)).cuda().view(torch.bfloat16)
        assert torch.equal(nw.view(torch.int16), nw_ref.view(torch.int16))
        for T in (1, 4, 300):
            x = make_input(cfg, T, tag=8800 + T) * 3
            ws = ref.workspace(T)
            a = torch.empty_like(x)
            b = torch.empty_like(x)
            ref.block_forward(x, a, ws, norm_w=nw_ref, norm_mode=L.NORM_ONE_PLUS)
            fl.block_forward(x, b, ws, norm_w=nw, norm_mode=L.NORM_ONE_PLUS)
            torch.cuda.synchronize()
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (name, l, T)
        del fl, ref
    bf.close()
