"""Synthetic GGUF shards generated on the GPU (benchmarks and full-size tests).

Every bit pattern of the quantized fields of the eleven formats is valid, so a shard is uniform
random bytes with its fp16 scale fields overwritten by finite positive values (the pattern of
gguf-plugin/gluon/kq_ref.py:94-112; IQ3_S / IQ4_XS super-scales |N(0, 1e-3)| as BASELINE config 3
asks).  Kernel time does not depend on the values, so these stand in for quantized N(0, 0.02)
weights in timing runs.
"""
from __future__ import annotations

import torch

from .ops import type_info

# per type: byte offsets of the fp16 scale fields inside one block, and their magnitude
_SCALE_FIELDS = {
    2: ((0,), 2.0 ** -6), 6: ((0,), 2.0 ** -6), 8: ((0,), 2.0 ** -6), 20: ((0,), 2.0 ** -6),
    10: ((80, 82), 2.0 ** -8), 11: ((108,), 2.0 ** -8), 12: ((0, 2), 2.0 ** -8), 13: ((0, 2), 2.0 ** -8),
    14: ((208,), 2.0 ** -8), 21: ((0,), None), 23: ((0,), None),
}


def random_shard(n: int, K: int, weight_type: int, device, seed: int = 0) -> torch.Tensor:
    """uint8 [n, row_bytes] of random valid GGUF blocks of the type."""
    bw, bb, _, _ = type_info(weight_type)
    nblk = K // bw
    g = torch.Generator(device=device).manual_seed(seed)
    raw = torch.randint(0, 256, (n, nblk, bb), dtype=torch.uint8, device=device, generator=g)
    offs, mag = _SCALE_FIELDS[weight_type]
    for o in offs:
        if mag is None:
            v = torch.randn((n, nblk), device=device, generator=g).abs() * 1e-3
        else:
            v = (torch.rand((n, nblk), device=device, generator=g) * 0.75 + 0.25) * mag
        raw[:, :, o:o + 2] = v.to(torch.float16).view(torch.uint8).reshape(n, nblk, 2)
    return raw.reshape(n, nblk * bb)
