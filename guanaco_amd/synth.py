"""Seed derivation of the synthetic-input generator (csrc/gq_synth.h), in
Python so the host side can name every tensor's stream without a GPU."""

M64 = (1 << 64) - 1


def mix64(z: int) -> int:
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def subseed(seed: int, tag: int) -> int:
    return mix64((seed & M64) ^ mix64((tag + 0x632BE59BD9B4E019) & M64))


def tensor_seed(model_seed: int, layer: int, slot: int) -> int:
    """gq_tensor_seed(): layer = -1 for global tensors."""
    return subseed(model_seed, (((layer + 1) & M64) << 8 | (slot & 0xFFFFFFFF)) & M64)
