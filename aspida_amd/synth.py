"""Synthetic K-quant weights and activations for tests and benchmarks.

Recipe (the benchmark configurations' generation rule): every byte of a
super-block is uniform random, except the f16 super-scales (d, and dmin where
the format has one), which are float16(|N(0, 2e-3)|).  Uniform scale bytes make
the 6-bit scales/mins of Q4_K/Q5_K uniform in 0..63.  Activations are f32
N(0, 1).  `blocks_np` draws on the host from a seeded PCG64 generator;
`blocks_torch` draws the same distribution directly in device memory for
multi-GB weight streams.
"""
import numpy as np

BLOCK_BYTES = {0: 144, 1: 210, 2: 176, 3: 110, 4: 84, 5: 272}

# Byte offsets of the f16 scale fields inside one 256-element super-block.
SCALE_OFFSETS = {0: (0, 2), 2: (0, 2), 1: (208,), 3: (108,), 4: (80, 82), 5: tuple(34 * k for k in range(8))}


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def blocks_np(kind, nblocks, gen):
    """uint8 [nblocks * block_bytes] of random super-blocks."""
    bb = BLOCK_BYTES[kind]
    b = gen.integers(0, 256, (nblocks, bb), dtype=np.uint8)
    for o in SCALE_OFFSETS[kind]:
        v = np.abs(gen.normal(0.0, 2e-3, nblocks)).astype(np.float16).view(np.uint16)
        b[:, o] = (v & 0xFF).astype(np.uint8)
        b[:, o + 1] = (v >> 8).astype(np.uint8)
    return b.reshape(-1)


def weight_np(kind, out_dim, in_dim, gen):
    return blocks_np(kind, out_dim * (in_dim // 256), gen)


def activations_np(n, gen):
    return gen.standard_normal(n).astype(np.float32)


def blocks_torch(kind, nblocks, device="cuda", generator=None):
    """The same distribution, generated on the device (torch is plumbing)."""
    import torch
    bb = BLOCK_BYTES[kind]
    b = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, device=device, generator=generator)
    for o in SCALE_OFFSETS[kind]:
        v = (torch.randn(nblocks, device=device, generator=generator) * 2e-3).abs().to(torch.float16)
        b[:, o:o + 2] = v.view(torch.uint8).view(nblocks, 2)
    return b.reshape(-1)
