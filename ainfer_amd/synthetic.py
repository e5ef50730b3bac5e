"""Synthetic MoE layer configurations and their seeds.

The five configurations are the benchmark's (BASELINE.json configs[0..4]).
Every tensor is a pure function of (config seed, layer, tensor id): element i
of a tensor is drawn by the counter-based generator of ainfer_moe_fill, so
the GPU fill and the CPU oracle's fill produce the same bits.
"""
import math
from dataclasses import dataclass, field

import numpy as np

M64 = (1 << 64) - 1


def splitmix(seed: int, i: int) -> int:
    """Element i of the splitmix64 stream `seed` (same as mo_rnd / rnd64)."""
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


TENSORS = ("router_w", "shared_gate_w", "w_gate", "s_gate", "w_up", "s_up", "w_down",
           "s_down", "ws_gate", "ss_gate", "ws_up", "ss_up", "ws_down", "ss_down", "zipf")


def layer_seed(seed: int, layer: int) -> int:
    return splitmix(seed ^ 0xA1F0E5D3C2B1A097, layer)


def tensor_seed(lseed: int, name: str) -> int:
    return splitmix(lseed, 16 + TENSORS.index(name))


def input_seed(seed: int, tag: int = 0) -> int:
    return splitmix(seed ^ 0x5EED5EED5EED5EED, tag)


@dataclass(frozen=True)
class MoeConfig:
    name: str
    hidden: int
    n_experts: int
    top_k: int
    inter: int
    shared_inter: int
    tokens: tuple
    zipf: float = 0.0          # router bias -s*ln(rank) when > 0
    layers: int = 1
    shared_gate: bool = True
    weight_std: float = 0.02   # router / gate weights ~ N(0, std)
    scale_std: float = 0.02    # |N(0, std)| fp16 scales
    seed: int = 0
    note: str = ""

    def shape_tuple(self):
        return (self.hidden, self.n_experts, self.top_k, self.inter, self.shared_inter)

    def expert_bytes(self, inter=None):
        """INT4 nibbles + fp16 g128 scales of one expert (gate, up, down)."""
        I = self.inter if inter is None else inter
        return 3 * self.hidden * I // 2 + (3 * self.hidden * I // 128) * 2

    def layer_weight_bytes(self):
        return (self.n_experts * self.expert_bytes() + self.expert_bytes(self.shared_inter)
                + self.n_experts * self.hidden * 2 + self.hidden * 2)


CONFIGS = {
    "c0": MoeConfig("c0", 1024, 64, 8, 256, 256, (1,),
                    note="small MoE layer, decode, 1 token (CPU reference path)"),
    "c1": MoeConfig("c1", 2048, 512, 10, 512, 512, (1, 4, 16),
                    note="Qwen3.5-MoE-style decode, batch 1/4/16"),
    "c2": MoeConfig("c2", 2048, 512, 10, 512, 512, (4096,), zipf=1.1,
                    note="prefill 4096 tokens, Zipf(1.1) expert popularity"),
    "c3": MoeConfig("c3", 4096, 512, 10, 1024, 1024, (64,),
                    note="speculative-decode verify, 64 tokens"),
    "c4": MoeConfig("c4", 4096, 512, 10, 1024, 1024, (1, 8), layers=60,
                    note="60-layer stack decode, RMSNorm before each router"),
}


def zipf_bias(cfg: MoeConfig, layer: int = 0) -> np.ndarray:
    """Router bias b_e = -s * ln(rank_e), rank = a seeded permutation of 1..E
    (Fisher-Yates driven by the splitmix stream), so softmax popularity is
    proportional to rank^-s."""
    E = cfg.n_experts
    zs = tensor_seed(layer_seed(cfg.seed, layer), "zipf")
    ranks = list(range(1, E + 1))
    for i in range(E - 1, 0, -1):
        j = splitmix(zs, i) % (i + 1)
        ranks[i], ranks[j] = ranks[j], ranks[i]
    return (-cfg.zipf * np.log(np.array(ranks, dtype=np.float64))).astype(np.float32)


def algorithmic_bytes(cfg: MoeConfig, T: int, unique_experts: int) -> int:
    """Bytes one layer step must move: (U+1) experts' INT4 weights + scales,
    the router matrix, the shared gate vector, x in and y out (bf16)."""
    H = cfg.hidden
    shared = cfg.expert_bytes(cfg.shared_inter) if cfg.shared_inter else 0
    return (unique_experts * cfg.expert_bytes() + shared + cfg.n_experts * H * 2 + H * 2
            + 2 * T * H * 2)


def algorithmic_flops(cfg: MoeConfig, T: int) -> int:
    H, I, Is = cfg.hidden, cfg.inter, cfg.shared_inter
    return 2 * T * (cfg.top_k * 3 * H * I + 3 * H * Is) + 2 * T * H * cfg.n_experts
