"""Write the small golden fixtures used by the CPU and GPU parity tests.

The reference ships no tests or vectors for the AWQ path (its .gitignore lists
``tests``), so these fixtures are produced by the oracle (oracle/awq_oracle.py)
from seeded generators and committed; the oracle itself is pinned by the
closed-form and known-answer checks in tests/test_oracle.py.  Re-running this
script must reproduce the committed file bit for bit.

    python tests/golden/gen_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import awq_oracle as oracle  # noqa: E402

# (name, K, N, group_size, dtype, M values, seed)
CASES = [
    ("k256_n64_g128_fp16", 256, 64, 128, torch.float16, (1, 4), 11),
    ("k96_n24_g32_fp16", 96, 24, 32, torch.float16, (3,), 12),
    ("k256_n32_gm1_bf16", 256, 32, -1, torch.bfloat16, (2,), 13),
    ("k128_n48_g64_fp16_bias", 128, 48, 64, torch.float16, (5,), 14),
]

KAT_WORDS = np.array([0x76543210, 0x75316420, 0x0000000F, 0xF0000000, 0x12345678, 0xFFFFFFFF, 0x00000000],
                     dtype=np.uint32)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def build() -> dict:
    out = {"kat_words": KAT_WORDS, "kat_unpacked": oracle.unpack_awq(KAT_WORDS.view(np.int32)[None, :]).reshape(-1, 8)}
    for name, K, N, G, dt, Ms, seed in CASES:
        t = oracle.make_awq_linear(K, N, G, seed=seed, dtype=dt)
        out[f"{name}/qweight"] = t["qweight"].numpy()
        out[f"{name}/qzeros"] = t["qzeros"].numpy()
        out[f"{name}/scales"] = bits(t["scales"])
        out[f"{name}/shape"] = np.array([K, N, G], dtype=np.int64)
        out[f"{name}/W"] = bits(oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G))
        bias = None
        if name.endswith("_bias"):
            bias = (torch.randn(N, generator=torch.Generator().manual_seed(seed + 1000)) * 0.5).to(dt)
            out[f"{name}/bias"] = bits(bias)
        for M in Ms:
            x = oracle.make_activation(M, K, seed=seed + M, dtype=dt)
            out[f"{name}/x{M}"] = bits(x)
            out[f"{name}/y{M}"] = bits(oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G))
    return out


if __name__ == "__main__":
    path = os.path.join(HERE, "awq_golden.npz")
    np.savez_compressed(path, **build())
    print("wrote", path, os.path.getsize(path), "bytes")
