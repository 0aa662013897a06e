"""Seeded synthetic MatMulNBits workloads (weights are random, no checkpoint).

Shapes follow the decoder projections the library serves:
* Phi-3-mini: per layer qkv 3072->9216, o_proj 3072->3072, gate_up 3072->16384,
  down 8192->3072 (32 layers), lm_head 3072->32064.
* Qwen2.5-0.5B: qkv 896->1152, o_proj 896->896, gate_up 896->9728,
  down 4864->896 (24 layers), lm_head 896->151936.
* SmolLM2-135M-shaped tails: K=576 N=1536 and K=1536 N=576.

Weights: uint8 [N, kb, bs/2] with both nibbles uniform in 0..15; scales
fp16 [N, kb] uniform in [0.005, 0.02] (fp32 draw rounded to nearest fp16);
optional zero points uint8 [N, ceil(kb/2)] (ONNX row-padded) with nibbles
uniform 0..15; activations fp16 [M, K] from N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

PHI3_LAYER: List[Tuple[str, int, int]] = [("qkv", 3072, 9216), ("o_proj", 3072, 3072),
                                          ("gate_up", 3072, 16384), ("down", 8192, 3072)]
PHI3_LM_HEAD = ("lm_head", 3072, 32064)
PHI3_LAYERS = 32
QWEN_LAYER: List[Tuple[str, int, int]] = [("qkv", 896, 1152), ("o_proj", 896, 896),
                                          ("gate_up", 896, 9728), ("down", 4864, 896)]
QWEN_LM_HEAD = ("lm_head", 896, 151936)
QWEN_LAYERS = 24
SMOL_SHAPES = [(576, 1536), (1536, 576)]


@dataclass
class QuantTensor:
    N: int
    K: int
    bs: int
    q: np.ndarray            # uint8 [N * kb * bs/2]
    scales_f16: np.ndarray   # float16 [N * kb]
    zp_row_padded: Optional[np.ndarray]   # uint8 [N, ceil(kb/2)] or None

    @property
    def kb(self) -> int:
        return -(-self.K // self.bs)

    def algorithmic_bytes(self, M: int) -> int:
        """Packed nibbles + fp16 scales (+ packed zero points) + fp16 x and y."""
        kb = self.kb
        b = self.N * kb * self.bs // 2 + self.N * kb * 2 + 2 * M * self.K + 2 * M * self.N
        if self.zp_row_padded is not None:
            b += self.N * ((kb + 1) // 2)
        return b


def make_weight(seed: int, N: int, K: int, bs: int = 32, with_zp: bool = False) -> QuantTensor:
    rng = np.random.default_rng(seed)
    kb = -(-K // bs)
    nbytes = N * kb * bs // 2
    q = np.frombuffer(rng.bytes(nbytes), np.uint8)
    scales = rng.uniform(0.005, 0.02, N * kb).astype(np.float32).astype(np.float16)
    zp = None
    if with_zp:
        rowb = (kb + 1) // 2
        nib = rng.integers(0, 16, (N, 2 * rowb), dtype=np.uint8)
        if kb % 2:
            nib[:, -1] = 0     # the pad nibble of an odd row
        zp = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return QuantTensor(N, K, bs, q, scales, zp)


def make_x(seed: int, M: int, K: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)


def zp_row_padded_to_flat(zp_rp: np.ndarray, N: int, kb: int) -> np.ndarray:
    """ONNX [N, ceil(kb/2)] -> the flat nibble stream n*kb+blk (for the oracle)."""
    rowb = (kb + 1) // 2
    nib = np.empty((N, 2 * rowb), np.uint8)
    nib[:, 0::2] = zp_rp & 0xF
    nib[:, 1::2] = zp_rp >> 4
    flat = nib[:, :kb].reshape(-1)
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, np.uint8)])
    return (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)


def qwen_decode_step() -> List[Tuple[str, int, int, int]]:
    """(name, layer, K, N) of every quantized projection of one Qwen2.5-0.5B
    decode step with a quantized lm_head."""
    out = []
    for layer in range(QWEN_LAYERS):
        for name, K, N in QWEN_LAYER:
            out.append((name, layer, K, N))
    out.append((QWEN_LM_HEAD[0], QWEN_LAYERS, QWEN_LM_HEAD[1], QWEN_LM_HEAD[2]))
    return out


def phi3_decode_step() -> List[Tuple[str, int, int, int]]:
    """(name, layer, K, N) of every quantized projection of one Phi-3 decode step."""
    out = []
    for layer in range(PHI3_LAYERS):
        for name, K, N in PHI3_LAYER:
            out.append((name, layer, K, N))
    out.append((PHI3_LM_HEAD[0], PHI3_LAYERS, PHI3_LM_HEAD[1], PHI3_LM_HEAD[2]))
    return out
