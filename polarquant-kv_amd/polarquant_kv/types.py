"""Cache containers.

PQCache plays the role of the reference's CompressedKVCacheGPU
(src/polarquant_kv_cuda/types.py:7-21) for the codebook (PolarQuant /
TurboQuant) format: instead of SoA radius + group parameters it holds
block_pq4 / block_pq2 vectors (README.md:73-78) in one uint8 tensor.

Layout of `blocks`:
  uniform widths: [B, H, S_max, vector_bytes]
  mixed widths:   [B, sum_h S_max * vector_bytes(h)], head h's run of S_max
                  vectors starting at head_offset(h)
"""

from __future__ import annotations

from dataclasses import dataclass, field

BLOCK = 32


def block_bytes(n_bits: int) -> int:
    if n_bits == 4:
        return 18
    if n_bits == 2:
        return 10
    raise ValueError(f"n_bits must be 2 or 4, got {n_bits}")


def vector_bytes(d: int, n_bits: int) -> int:
    if d % BLOCK:
        raise ValueError(f"head_dim must be a multiple of {BLOCK}, got {d}")
    return d // BLOCK * block_bytes(n_bits)


@dataclass
class PQCache:
    blocks: "object"                  # torch.uint8 tensor, layout above
    head_dim: int
    n_bits: int | tuple               # one width, or one per kv head
    seq_len: int                      # valid positions
    max_seq_len: int
    codebooks: "object"               # torch.float32 [16] or [H, 16]
    qjl_signs: "object | None" = None  # torch.uint8 [B, H, S_max, m/8] (keys only)
    jl_dim: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def mixed(self) -> bool:
        return not isinstance(self.n_bits, int)

    @property
    def num_heads(self) -> int:
        if self.mixed:
            return len(self.n_bits)
        return self.blocks.shape[1]

    @property
    def batch(self) -> int:
        return self.blocks.shape[0]

    def head_bits(self) -> list:
        return list(self.n_bits) if self.mixed else [self.n_bits] * self.num_heads

    def head_offset(self, h: int) -> int:
        """Byte offset of head h's run inside one batch row."""
        return sum(self.max_seq_len * vector_bytes(self.head_dim, b) for b in self.head_bits()[:h])

    def memory_bytes(self) -> int:
        n = self.blocks.numel()
        if self.qjl_signs is not None:
            n += self.qjl_signs.numel()
        return n


@dataclass
class QJLSignatures:
    """Sign sketch of one residual (python/polarquant_kv/types.py:19-25):
    signs [jl_dim] bool, the sketch size, and the residual's norm, which the
    correction uses only to return 0 for a zero residual."""
    signs: "object"
    jl_dim: int
    residual_norm: float = 0.0


@dataclass
class CompressedKV:
    """One vector in the group (min / scale) format
    (python/polarquant_kv/types.py:7-16 of the reference): fp32 radius,
    uint8 codes of the padded direction, fp32 per-group minimum and scale."""
    radius: "object"                  # np.float32
    quantized_direction: "object"     # np.uint8 [ceil(d / group_size) * group_size]
    group_mins: "object"              # np.float32 [ceil(d / group_size)]
    group_scales: "object"            # np.float32 [ceil(d / group_size)]
    n_bits: int
    group_size: int
    original_dim: int
